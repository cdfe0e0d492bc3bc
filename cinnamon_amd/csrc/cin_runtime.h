// Host-side error reporting shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/cinnamon_fp8.h"

// Record a formatted message for cin_last_error() and return `code`.
int cin_set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Check for a launch error after hipLaunchKernelGGL; returns CIN_OK or CIN_ERR_HIP.
int cin_check_launch(const char* what);

#define CIN_CHECK_ARG(cond, ...)                    \
  do {                                              \
    if (!(cond)) return cin_set_error(CIN_ERR_ARG, __VA_ARGS__); \
  } while (0)
