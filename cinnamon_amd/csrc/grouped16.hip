// Unquantized grouped GEMM for MoE experts on gfx950 fp16 MFMA: the reference's
// moe_grouped_gemm / grouped_gemm_kernel (src/kernels.py:440-581).
//
//   C[r, n] = fp16( sum_k fp16(A[r, k]) * fp16(B_e[n, k]) )   for rows r of expert e
//
// Operands are rounded to fp16 (round-to-nearest-even) as the reference's
// a.to(tl.float16) / b.to(tl.float16) do, the products are summed in fp32 by
// v_mfma_f32_16x16x32_f16, and the result is stored as fp16 (RNE).  One launch covers all
// experts: a workgroup finds its (expert, 128-row tile) by scanning the device-side
// ranges, so there is no host synchronisation and no grid sized by the largest expert.
// Rows outside every expert range are not written (the reference returns torch.empty).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cin_common.h"
#include "cin_grouped.h"
#include "cin_runtime.h"

using namespace cin;

namespace {

constexpr int BM = 128, BN = 128, BK = 64;  // workgroup tile, K step per LDS stage
constexpr int kThreads = 256;               // 4 waves in 2 x 2, wave tile 64 x 64
constexpr int kRowBytes = BK * 2;           // one fp16 tile row: 8 chunks of 16 bytes

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

// chunk c of tile row r sits at slot c ^ f(r) (the same swizzle as the FP8 GEMM's
// 128-byte rows: conflict-free fragment reads)
__device__ inline int swz_f(int r) { return (r & 7) ^ ((r >> 3) & 1); }

template <int DT>
__device__ inline float elem(const void* p, int64_t i) {
  if constexpr (DT == CIN_DT_BF16) return __uint_as_float(((uint32_t)((const uint16_t*)p)[i]) << 16);
  else if constexpr (DT == CIN_DT_F16) return (float)((const _Float16*)p)[i];
  else return ((const float*)p)[i];
}

// 32 consecutive elements of one row (zero past `nvalid`), rounded to fp16, as 4 chunks.
// VEC: the 32 elements are in range and 16-byte aligned (vector loads).
template <int DT, bool VEC>
__device__ inline void load32(const void* base, int64_t off, int64_t nvalid, h8 (&o)[4]) {
  if constexpr (VEC) {
    if constexpr (DT == CIN_DT_F32) {
      const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + off);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float4 a = p[2 * c], b = p[2 * c + 1];
        o[c] = h8{(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w,
                  (_Float16)b.x, (_Float16)b.y, (_Float16)b.z, (_Float16)b.w};
      }
    } else if constexpr (DT == CIN_DT_F16) {
      const h8* p = reinterpret_cast<const h8*>(static_cast<const _Float16*>(base) + off);
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] = p[c];
    } else {
      const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + off);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint4 w = p[c];
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          o[c][2 * e] = (_Float16)bf16_lo(ws[e]);
          o[c][2 * e + 1] = (_Float16)bf16_hi(ws[e]);
        }
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int k = c * 8 + e;
        o[c][e] = k < nvalid ? (_Float16)elem<DT>(base, off + k) : (_Float16)0.0f;
      }
  }
}

template <int ADT, int BDT, bool VEC>
__global__ __launch_bounds__(kThreads) void k_grouped_gemm_f16(
    const void* __restrict__ A, int64_t lda, const void* __restrict__ B, int64_t sbe, int64_t ldb,
    const int64_t* __restrict__ starts, const int64_t* __restrict__ ends, int64_t E, int64_t T,
    int64_t N, int64_t K, _Float16* __restrict__ C, int64_t ldc, uint32_t tiles_n) {
  __shared__ __attribute__((aligned(16))) uint8_t sa[2][BM * kRowBytes];
  __shared__ __attribute__((aligned(16))) uint8_t sb[2][BN * kRowBytes];
  const uint32_t tile = blockIdx.x / tiles_n, tn = blockIdx.x - tile * tiles_n;
  // (expert, 128-row tile) of this workgroup
  int64_t seen = 0, e = -1, r0 = 0, r1 = 0;
  for (int64_t x = 0; x < E; ++x) {
    int64_t s0, s1;
    clamp_range(starts, ends, x, T, s0, s1);
    const int64_t nt = (s1 - s0 + BM - 1) / BM;
    if ((int64_t)tile < seen + nt) {
      e = x;
      r0 = s0 + ((int64_t)tile - seen) * BM;
      r1 = s1;
      break;
    }
    seen += nt;
  }
  if (e < 0) return;  // surplus workgroup, before any barrier
  const int nr = (int)(r1 - r0 < BM ? r1 - r0 : BM);
  const int64_t n0 = (int64_t)tn * BN;
  const uint8_t* Be = static_cast<const uint8_t*>(B) + e * sbe * (BDT == CIN_DT_F32 ? 4 : 2);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l16 = lane & 15, kq = lane >> 4;
  // loads: thread = (tile row tid / 2, 32-element half tid % 2)
  const int lr = tid >> 1, lh = tid & 1;
  const bool arow = lr < nr, brow = n0 + lr < N;
  const int64_t aoff = (r0 + lr) * lda, boff = (n0 + lr) * ldb;

  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  h8 ga[4], gb[4];
  auto fetch = [&](int64_t k0) {
    const int64_t k = k0 + lh * 32;
    const int64_t nv = K - k;
    if (arow) load32<ADT, VEC>(A, aoff + k, nv, ga);
    else for (int c = 0; c < 4; ++c) ga[c] = h8{};
    if (brow) load32<BDT, VEC>(Be, boff + k, nv, gb);
    else for (int c = 0; c < 4; ++c) gb[c] = h8{};
  };
  auto store = [&](int st) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int slot = (lh * 4 + c) ^ swz_f(lr);
      *reinterpret_cast<h8*>(&sa[st][lr * kRowBytes + slot * 16]) = ga[c];
      *reinterpret_cast<h8*>(&sb[st][lr * kRowBytes + slot * 16]) = gb[c];
    }
  };
  // fragment: row `row`, K elements [8 q, 8 q + 8) of k-step ks (chunk 4 ks + q)
  auto frag = [&](const uint8_t* base, int row, int ks) -> h8 {
    const int slot = (4 * ks + kq) ^ swz_f(row);
    return *reinterpret_cast<const h8*>(base + row * kRowBytes + slot * 16);
  };

  const int nkt = (int)((K + BK - 1) / BK);
  fetch(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < nkt; ++kt) {
    const int st = kt & 1;
    if (kt + 1 < nkt) fetch((int64_t)(kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      h8 bfr[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) bfr[j] = frag(sb[st], wn * 64 + j * 16 + l16, ks);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const h8 afr = frag(sa[st], wm * 64 + i * 16 + l16, ks);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bfr[j], afr, acc[i][j], 0, 0, 0);
      }
    }
    if (kt + 1 < nkt) store(st ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds C[m][n .. n+3]
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = wm * 64 + i * 16 + l16;
    if (m >= nr) continue;
    _Float16* crow = C + (r0 + m) * ldc;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + wn * 64 + j * 16 + kq * 4;
      const _Float16 h0 = (_Float16)acc[i][j][0], h1 = (_Float16)acc[i][j][1];
      const _Float16 h2 = (_Float16)acc[i][j][2], h3 = (_Float16)acc[i][j][3];
      if (n + 4 <= N && (((uintptr_t)(crow + n)) & 7) == 0) {
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        *reinterpret_cast<h4*>(crow + n) = h4{h0, h1, h2, h3};
      } else {
        const _Float16 hv[4] = {h0, h1, h2, h3};
        for (int r = 0; r < 4; ++r)
          if (n + r < N) crow[n + r] = hv[r];
      }
    }
  }
}

inline bool valid_dtype(int dt) { return dt == CIN_DT_BF16 || dt == CIN_DT_F32 || dt == CIN_DT_F16; }
inline int elem_size(int dt) { return dt == CIN_DT_F32 ? 4 : 2; }

template <int ADT, int BDT>
void launch(bool vec, unsigned grid, hipStream_t s, const void* A, int64_t lda, const void* B,
            int64_t sbe, int64_t ldb, const int64_t* starts, const int64_t* ends, int64_t E,
            int64_t T, int64_t N, int64_t K, _Float16* C, int64_t ldc, uint32_t tiles_n) {
  if (vec)
    hipLaunchKernelGGL((k_grouped_gemm_f16<ADT, BDT, true>), grid, kThreads, 0, s, A, lda, B, sbe,
                       ldb, starts, ends, E, T, N, K, C, ldc, tiles_n);
  else
    hipLaunchKernelGGL((k_grouped_gemm_f16<ADT, BDT, false>), grid, kThreads, 0, s, A, lda, B, sbe,
                       ldb, starts, ends, E, T, N, K, C, ldc, tiles_n);
}

template <int ADT>
void launch_b(int b_dtype, bool vec, unsigned grid, hipStream_t s, const void* A, int64_t lda,
              const void* B, int64_t sbe, int64_t ldb, const int64_t* starts, const int64_t* ends,
              int64_t E, int64_t T, int64_t N, int64_t K, _Float16* C, int64_t ldc, uint32_t tn) {
  if (b_dtype == CIN_DT_BF16)
    launch<ADT, CIN_DT_BF16>(vec, grid, s, A, lda, B, sbe, ldb, starts, ends, E, T, N, K, C, ldc, tn);
  else if (b_dtype == CIN_DT_F16)
    launch<ADT, CIN_DT_F16>(vec, grid, s, A, lda, B, sbe, ldb, starts, ends, E, T, N, K, C, ldc, tn);
  else
    launch<ADT, CIN_DT_F32>(vec, grid, s, A, lda, B, sbe, ldb, starts, ends, E, T, N, K, C, ldc, tn);
}

}  // namespace

extern "C" {

int cin_grouped_gemm_f16(const void* A, int a_dtype, int64_t lda, const void* B, int b_dtype,
                         int64_t sbe, int64_t ldb, const int64_t* starts, const int64_t* ends,
                         int64_t E, int64_t T, int64_t N, int64_t K, void* C, int64_t ldc,
                         void* stream) {
  CIN_CHECK_ARG(valid_dtype(a_dtype) && valid_dtype(b_dtype), "grouped_gemm_f16: unsupported dtype");
  CIN_CHECK_ARG(E >= 0 && T >= 0 && N >= 0 && K >= 0, "grouped_gemm_f16: negative shape");
  if (E == 0 || T == 0 || N == 0) return CIN_OK;
  CIN_CHECK_ARG(A && B && starts && ends && C, "grouped_gemm_f16: null pointer");
  CIN_CHECK_ARG(lda >= K && ldb >= K && ldc >= N && sbe >= 0, "grouped_gemm_f16: bad strides");
  // full 32-element vector loads need every row and tile start aligned to the vector
  const int ea = elem_size(a_dtype), eb = elem_size(b_dtype);
  const bool vec = K % BK == 0 && ((uintptr_t)A % 16) == 0 && ((uintptr_t)B % 16) == 0 &&
                   (lda * ea) % 16 == 0 && (ldb * eb) % 16 == 0 && (sbe * eb) % 16 == 0;
  const int64_t tiles = cdiv(T, BM) + E;
  const int64_t tn = cdiv(N, BN);
  CIN_CHECK_ARG(tiles * tn < ((int64_t)1 << 31), "grouped_gemm_f16: grid too large");
  const unsigned grid = (unsigned)(tiles * tn);
  hipStream_t s = static_cast<hipStream_t>(stream);
  _Float16* Ch = static_cast<_Float16*>(C);
  if (a_dtype == CIN_DT_BF16)
    launch_b<CIN_DT_BF16>(b_dtype, vec, grid, s, A, lda, B, sbe, ldb, starts, ends, E, T, N, K, Ch, ldc, (uint32_t)tn);
  else if (a_dtype == CIN_DT_F16)
    launch_b<CIN_DT_F16>(b_dtype, vec, grid, s, A, lda, B, sbe, ldb, starts, ends, E, T, N, K, Ch, ldc, (uint32_t)tn);
  else
    launch_b<CIN_DT_F32>(b_dtype, vec, grid, s, A, lda, B, sbe, ldb, starts, ends, E, T, N, K, Ch, ldc, (uint32_t)tn);
  return cin_check_launch("grouped_gemm_f16");
}

}  // extern "C"
