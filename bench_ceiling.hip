// Calibration kernel for bench.py (not part of the library): the FP8 GEMM's per-K-block
// instruction mix with no memory traffic, to measure the MFMA rate the GPU sustains on
// random e4m3 operands under its power limit.
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

}  // namespace

extern "C" {

// codes: blocks * 512 * 48 int32 of random e4m3 bytes; out: blocks * 512 fp32.  Each launch
// performs blocks * 8 * iters * 32 MFMAs of 16 x 16 x 128 (2 * 16 * 16 * 128 FLOP each).
int bench_mfma_ceiling(const int* codes, float* out, int blocks, int iters, int promote, void* stream) {
  if (!codes || !out || blocks <= 0 || iters <= 0) return -1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (promote)
    hipLaunchKernelGGL(k_mfma_ceiling<true>, blocks, 512, 0, s, codes, out, iters);
  else
    hipLaunchKernelGGL(k_mfma_ceiling<false>, blocks, 512, 0, s, codes, out, iters);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

}  // extern "C"
