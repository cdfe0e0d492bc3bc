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

// 128-row chunk `id` in expert order.  Returns false past the last chunk.
struct Chunk {
  int64_t r0;  // first row of the chunk
  int nr;      // rows in the chunk (1..128)
  int64_t t0;  // position of the chunk on the padded token axis
};

__device__ inline bool find_chunk(const int64_t* starts, const int64_t* ends, int64_t E, int64_t T,
                                  int64_t id, Chunk& c) {
  int64_t seen = 0, pad = 0;
  for (int64_t e = 0; e < E; ++e) {
    int64_t s0, s1;
    clamp_range(starts, ends, e, T, s0, s1);
    const int64_t n = (s1 - s0 + 127) / 128;
    if (id < seen + n) {
      const int64_t k = id - seen;
      c.r0 = s0 + 128 * k;
      const int64_t left = s1 - c.r0;
      c.nr = (int)(left < 128 ? left : 128);
      c.t0 = pad + 128 * k;
      return true;
    }
    seen += n;
    pad += 128 * n;
  }
  return false;
}

// Padded offset p_e and row count m_e of expert e.
__device__ inline void padded_range(const int64_t* starts, const int64_t* ends, int64_t e, int64_t T,
                                    int64_t& p, int64_t& m) {
  p = 0;
  for (int64_t x = 0; x < e; ++x) {
    int64_t s0, s1;
    clamp_range(starts, ends, x, T, s0, s1);
    p += 128 * ((s1 - s0 + 127) / 128);
  }
  int64_t s0, s1;
  clamp_range(starts, ends, e, T, s0, s1);
  m = s1 - s0;
}

}  // namespace cin
