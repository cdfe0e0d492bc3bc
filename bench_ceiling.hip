// Calibration kernels for bench.py (not part of the library).  k_mfma_ceiling: the FP8
// GEMM's per-K-block instruction mix with no memory traffic, to measure the MFMA rate the
// GPU sustains on random e4m3 operands under its power limit.  k_stream_mix (below): the
// HBM rate of a given read : write byte mix in linear order.
//
// Each wave runs the inner step of k_gemm_fp8_bs_256 on fragments held in registers: 32
// v_mfma_scale_f32_16x16x128_f8f6f4 per "K block" (8 m-tiles x 4 n-tiles) and, with
// `promote`, the 4 scale-FMAs of the MFMA three steps earlier before each MFMA (the
// per-block promotion acc += P * sa * sb of the block-scaled GEMM).  Without `promote` the
// MFMAs accumulate in hardware (what a per-tensor-scaled FP8 GEMM does).  Operands come
// from `codes` (random e4m3 bytes supplied by the caller): the datapath's switching
// activity, and with it the power-limited clock, depends on the operand bits.  512
// threads (8 waves) per workgroup, one workgroup per CU, as the GEMM.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

template <bool PROMOTE>
__global__ __launch_bounds__(512) void k_mfma_ceiling(const int* __restrict__ codes, float* __restrict__ out,
                                                      int iters) {
  const int t = threadIdx.x;
  const int64_t g = (int64_t)blockIdx.x * 512 + t;
  v8i af[2], bf[4];
  for (int i = 0; i < 2; ++i)
    for (int e = 0; e < 8; ++e) af[i][e] = codes[(g * 6 + i) * 8 + e];
  for (int j = 0; j < 4; ++j)
    for (int e = 0; e < 8; ++e) bf[j][e] = codes[(g * 6 + 2 + j) * 8 + e];
  float cs[8];
  for (int i = 0; i < 8; ++i) cs[i] = 1.0f + 0.001f * (t & 15) + 0.01f * i;
  v4f acc[8][4];
  for (int i = 0; i < 8; ++i)
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
  const v4f zero = {0.f, 0.f, 0.f, 0.f};
  v4f p[4] = {zero, zero, zero, zero};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int s8 = 0; s8 < 32; ++s8) {
      const int i = s8 >> 2, j = s8 & 3;
      if (PROMOTE) {
        // the GEMM's order: FMAs of MFMA(s8 - 3), then MFMA(s8), pinned by operand fences
        const int ti = s8 >= 3 ? (s8 - 3) >> 2 : 7, tj = (s8 + 1) & 3;
        asm volatile("" : "+v"(acc[ti][tj]));
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[ti][tj][r] = fmaf(p[(s8 + 1) & 3][r], cs[ti], acc[ti][tj][r]);
        asm volatile("" : "+v"(acc[ti][tj]));
        asm volatile("" : "+v"(bf[j]));
        p[s8 & 3] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf[j], af[i & 1], zero, 0, 0, 0, 0, 0, 0);
        asm volatile("" : "+v"(bf[j]));
      } else {
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf[j], af[i & 1], acc[i][j], 0, 0, 0, 0, 0, 0);
      }
    }
  }
  float sum = 0.0f;
  for (int i = 0; i < 8; ++i)
    for (int j = 0; j < 4; ++j)
      for (int r = 0; r < 4; ++r) sum += acc[i][j][r];
  for (int j = 0; j < 4; ++j)
    for (int r = 0; r < 4; ++r) sum += p[j][r];
  out[g] = sum;
}

// The same wave tile (128 x 64 outputs) and per-K-block work with v_mfma_scale_f32_32x32x64
// _f8f6f4: 8 output tiles of 32 x 32, each taking two MFMAs per K block (K halves 0-63 and
// 64-127, the second accumulating onto the first in hardware; one block scale covers both),
// then, two tiles later, 16 scale-FMAs per lane.  Half as many MFMA instructions, each
// reading its 32-byte A and B operands once for twice the FLOP of a 16 x 16 x 128.
template <bool PROMOTE>
__global__ __launch_bounds__(512) void k_mfma_ceiling32(const int* __restrict__ codes, float* __restrict__ out,
                                                        int iters) {
  const int t = threadIdx.x;
  const int64_t g = (int64_t)blockIdx.x * 512 + t;
  v8i af[2], bf[4];
  for (int i = 0; i < 2; ++i)
    for (int e = 0; e < 8; ++e) af[i][e] = codes[(g * 6 + i) * 8 + e];
  for (int j = 0; j < 4; ++j)
    for (int e = 0; e < 8; ++e) bf[j][e] = codes[(g * 6 + 2 + j) * 8 + e];
  float cs[4];
  for (int i = 0; i < 4; ++i) cs[i] = 1.0f + 0.001f * (t & 15) + 0.01f * i;
  v16f acc[8], zero;
  for (int r = 0; r < 16; ++r) zero[r] = 0.f;
  for (int i = 0; i < 8; ++i) acc[i] = zero;
  v16f p[3] = {zero, zero, zero};  // partial ring; slot s % 3 holds tile s
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int i = s >> 1, j = s & 1;
      if (PROMOTE) {
        const int ts = (s + 6) & 7;  // tile s - 2, wrapping over K blocks
        asm volatile("" : "+v"(acc[ts]));
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[ts][r] = fmaf(p[(s + 1) % 3][r], cs[ts >> 1], acc[ts][r]);
        asm volatile("" : "+v"(acc[ts]));
        asm volatile("" : "+v"(bf[2 * j]), "+v"(bf[2 * j + 1]));
        const v16f q = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bf[2 * j], af[i & 1], zero, 0, 0, 0, 0, 0, 0);
        p[s % 3] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bf[2 * j + 1], af[(i + 1) & 1], q, 0, 0, 0, 0, 0, 0);
        asm volatile("" : "+v"(bf[2 * j]), "+v"(bf[2 * j + 1]));
      } else {
        acc[s] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bf[2 * j], af[i & 1], acc[s], 0, 0, 0, 0, 0, 0);
        acc[s] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bf[2 * j + 1], af[(i + 1) & 1], acc[s], 0, 0, 0, 0, 0, 0);
      }
    }
  }
  float sum = 0.0f;
  for (int i = 0; i < 8; ++i)
    for (int r = 0; r < 16; ++r) sum += acc[i][r];
  for (int j = 0; j < 3; ++j)
    for (int r = 0; r < 16; ++r) sum += p[j][r];
  out[g] = sum;
}

// Streaming calibration for the HBM-bound kernels: per unit, R 16-byte chunks in
// (non-temporal loads) and W 16-byte chunks out, every chunk stream linear and coalesced (R
// read streams, W write streams, lane i of a workgroup at chunk i), the friendliest access
// pattern for a given read : write mix.  Written data depends on what was read, so no load
// can be dropped.  Grid-stride over units with two units in flight per thread.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
template <int R, int W>
__global__ __launch_bounds__(256) void k_stream_mix(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                    int64_t units) {
  const int64_t T = (int64_t)gridDim.x * 256;
  for (int64_t u0 = (int64_t)blockIdx.x * 256 + threadIdx.x; u0 < units; u0 += 2 * T) {
    u32x4 v[2][R];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t u = u0 + h * T;
#pragma unroll
      for (int r = 0; r < R; ++r)
        v[h][r] = u < units ? __builtin_nontemporal_load(src + r * units + u) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t u = u0 + h * T;
      if (u >= units) break;
      u32x4 x = v[h][0];
#pragma unroll
      for (int r = 1; r < R; ++r) x ^= v[h][r];
#pragma unroll
      for (int w = 0; w < W; ++w) dst[w * units + u] = x + (unsigned)w;
    }
  }
}

}  // namespace

extern "C" {

// src: R * units 16-byte chunks, dst: W * units; (R, W) in {(1, 1), (2, 1), (4, 1), (1, 4)}.
int bench_stream_mix(const void* src, void* dst, int64_t units, int r, int w, int grid, void* stream) {
  if (!src || !dst || units <= 0 || grid <= 0) return -1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const u32x4* a = static_cast<const u32x4*>(src);
  u32x4* b = static_cast<u32x4*>(dst);
  if (r == 1 && w == 1)
    hipLaunchKernelGGL((k_stream_mix<1, 1>), grid, 256, 0, s, a, b, units);
  else if (r == 2 && w == 1)
    hipLaunchKernelGGL((k_stream_mix<2, 1>), grid, 256, 0, s, a, b, units);
  else if (r == 4 && w == 1)
    hipLaunchKernelGGL((k_stream_mix<4, 1>), grid, 256, 0, s, a, b, units);
  else if (r == 1 && w == 4)
    hipLaunchKernelGGL((k_stream_mix<1, 4>), grid, 256, 0, s, a, b, units);
  else
    return -1;
  return hipGetLastError() == hipSuccess ? 0 : -3;
}


// codes: blocks * 512 * 48 int32 of random e4m3 bytes; out: blocks * 512 fp32.  Each launch
// performs blocks * 8 * iters * 2^21 FLOP: 32 MFMAs of 16 x 16 x 128 (shape 16) or 16 of
// 32 x 32 x 64 (shape 32) per wave and iteration.
int bench_mfma_ceiling(const int* codes, float* out, int blocks, int iters, int promote, int shape,
                       void* stream) {
  if (!codes || !out || blocks <= 0 || iters <= 0 || (shape != 16 && shape != 32)) return -1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (shape == 32) {
    if (promote)
      hipLaunchKernelGGL(k_mfma_ceiling32<true>, blocks, 512, 0, s, codes, out, iters);
    else
      hipLaunchKernelGGL(k_mfma_ceiling32<false>, blocks, 512, 0, s, codes, out, iters);
  } else if (promote) {
    hipLaunchKernelGGL(k_mfma_ceiling<true>, blocks, 512, 0, s, codes, out, iters);
  } else {
    hipLaunchKernelGGL(k_mfma_ceiling<false>, blocks, 512, 0, s, codes, out, iters);
  }
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

}  // extern "C"
