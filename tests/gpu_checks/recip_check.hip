// Test infrastructure, not part of the library: compares the library's recip_ge1 (the SwiGLU
// backward's sigmoid reciprocal, cin_common.h) with the IEEE division 1.0f / d on every fp32
// bit pattern in a range, on the device, with the library's own compile flags.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../cinnamon_amd/csrc/cin_common.h"

using namespace cin;

namespace {

__global__ void k_recip_check(uint32_t first, uint32_t count, unsigned long long* bad, uint32_t* first_bad) {
  const uint32_t stride = gridDim.x * blockDim.x;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
    const uint32_t bits = first + i;
    const float d = __uint_as_float(bits);
    const float want = 1.0f / d, got = recip_ge1(d);
    const bool same = __float_as_uint(want) == __float_as_uint(got) || (want != want && got != got);
    if (!same) {
      atomicAdd(bad, 1ull);
      atomicMin(first_bad, bits);
    }
  }
}

}  // namespace

// Mismatches of recip_ge1 against 1.0f / d over the bit patterns [first, last] (both NaN
// counts as equal); *first_bad gets the smallest mismatching pattern (0xffffffff if none).
// Returns -1 on a HIP error.
extern "C" long long cin_test_recip_ge1_mismatches(uint32_t first, uint32_t last, uint32_t* first_bad) {
  if (last < first) return 0;
  unsigned long long* bad = nullptr;
  uint32_t* fb = nullptr;
  if (hipMalloc(&bad, sizeof(*bad)) != hipSuccess) return -1;
  if (hipMalloc(&fb, sizeof(*fb)) != hipSuccess) { (void)hipFree(bad); return -1; }
  const unsigned long long zero = 0;
  const uint32_t none = 0xffffffffu;
  long long result = -1;
  unsigned long long hb = 0;
  if (hipMemcpy(bad, &zero, sizeof(zero), hipMemcpyHostToDevice) == hipSuccess &&
      hipMemcpy(fb, &none, sizeof(none), hipMemcpyHostToDevice) == hipSuccess) {
    const uint64_t count = (uint64_t)last - first + 1;  // <= 2^32: split in two launches if it is
    uint64_t done = 0;
    bool ok = true;
    while (ok && done < count) {
      const uint64_t n = count - done < 0x80000000ull ? count - done : 0x80000000ull;
      hipLaunchKernelGGL(k_recip_check, 8192, 256, 0, 0, (uint32_t)(first + done), (uint32_t)n, bad, fb);
      ok = hipGetLastError() == hipSuccess;
      done += n;
    }
    if (ok && hipDeviceSynchronize() == hipSuccess &&
        hipMemcpy(&hb, bad, sizeof(hb), hipMemcpyDeviceToHost) == hipSuccess &&
        hipMemcpy(first_bad, fb, sizeof(*fb), hipMemcpyDeviceToHost) == hipSuccess)
      result = (long long)hb;
  }
  (void)hipFree(bad);
  (void)hipFree(fb);
  return result;
}
