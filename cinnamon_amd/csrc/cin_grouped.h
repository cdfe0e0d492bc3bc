// Expert-range helpers shared by the grouped (MoE) quantizers and GEMMs.
//
// Tokens are sorted by expert; expert e owns rows [starts[e], ends[e]) of a [T, ...]
// operand (reference src/layers.py:141-149: counts -> cumsum -> starts/ends).  The ranges
// are read on the device, so no host synchronisation is needed.  Ranges are clamped to
// [0, T); an empty or inverted range owns no rows.
//
// The backward of the grouped GEMM reduces over each expert's tokens, so its operands are
// quantized in 128-token chunks aligned at the expert's first row (the A7 recipe of the
// reference, src/kernels.py:771-788, applied per expert slice).  Chunk c of expert e holds
// rows [s_e + 128 c, min(s_e + 128 (c + 1), e_e)) and is stored in a padded token axis at
// [p_e + 128 c, p_e + 128 (c + 1)), with p_e = sum over e' < e of 128 * ceil(m_e' / 128).
// The padded length is at most T + 127 E.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cin {

__device__ inline void clamp_range(const int64_t* starts, const int64_t* ends, int64_t e, int64_t T,
                                   int64_t& s0, int64_t& s1) {
  s0 = starts[e];
  s1 = ends[e];
  if (s0 < 0) s0 = 0;
  if (s1 > T) s1 = T;
  if (s1 < s0) s1 = s0;
}

}  // namespace cin
