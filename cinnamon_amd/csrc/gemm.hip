// Block-scaled FP8 GEMM (dense and grouped) for gfx950.
//
//   C[m, n] = sum_kb sa[m, kb] * sb[n / 128, kb] * P_kb[m, n],
//   P_kb[m, n] = sum_{k in block kb} A[m, k] * B[n, k]      (e4m3 x e4m3 -> fp32)
//
// This is the reference fp8_gemm_kernel (src/kernels.py:588-664) restated for
// CDNA4: instead of dequantizing both tiles to fp32 and calling an fp32 dot, the
// 128-deep K block is one v_mfma_f32_16x16x128_f8f6f4 per 16x16 output tile
// (e4m3 operands, exact products, fp32 sums) and the two block scales are
// applied once per K block in the fp32 epilogue (acc += P_kb * sa * sb).
//
// Both operands are K-contiguous ("TN"): A[M, K] and B[N, K].  The forward GEMM
// takes the weight codes W[N, K] as B directly, so the reference's
// w_fp8.t().contiguous() copy disappears; dgrad/wgrad pass the transposed codes
// produced by the quantizers.
//
// Workgroup tile 128 x 128 x 128, 4 waves in 2 x 2, wave tile 64 x 64.  K blocks
// are staged global -> registers -> LDS (XOR-swizzled 16-byte chunks, double
// buffered, one barrier per K block).  The MFMA is issued as B x A^T so each
// lane ends up holding 4 consecutive columns of one row (one 8-byte bf16 or
// 16-byte fp32 store per fragment) and a single combined scale sa[m] * sb.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "cin_common.h"
#include "cin_grouped.h"
#include "cin_runtime.h"

using namespace cin;

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 128;
constexpr int kThreads = 256;

struct TileArgs {
  const uint8_t* A;  // first row of this tile's A rows
  const float* sa;   // sa for the first row (advance by ssam per row, ssak per kb)
  const uint8_t* B;  // first row of this tile's B rows
  const float* sb;   // sb for this tile's 128-column block (advance by ssbk per kb)
  int rows_a;        // valid A rows in the tile (<= BM)
  int rows_b;        // valid B rows in the tile (<= BN)
};

__device__ inline int swz(int row, int chunk) { return row * BK + ((chunk ^ (row & 7)) << 4); }

__device__ inline void load_tile_regs(const uint8_t* base, int64_t ld, int rows_valid, int64_t k0,
                                      int64_t K, uint4 (&r)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = threadIdx.x + i * kThreads;
    const int row = c >> 3, ch = c & 7;
    const int64_t k = k0 + ch * 16;
    if (row < rows_valid && k < K)
      r[i] = *reinterpret_cast<const uint4*>(base + (int64_t)row * ld + k);
    else
      r[i] = make_uint4(0, 0, 0, 0);
  }
}

__device__ inline void store_tile_lds(uint8_t* lds, const uint4 (&r)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = threadIdx.x + i * kThreads;
    const int row = c >> 3, ch = c & 7;
    *reinterpret_cast<uint4*>(lds + swz(row, ch)) = r[i];
  }
}

__device__ inline v8i read_frag(const uint8_t* lds, int row, int kq) {
  // kq in 0..3: the lane's 32-byte quarter of the 128-deep K block
  const uint4 lo = *reinterpret_cast<const uint4*>(lds + swz(row, 2 * kq));
  const uint4 hi = *reinterpret_cast<const uint4*>(lds + swz(row, 2 * kq + 1));
  v8i v;
  v[0] = (int)lo.x; v[1] = (int)lo.y; v[2] = (int)lo.z; v[3] = (int)lo.w;
  v[4] = (int)hi.x; v[5] = (int)hi.y; v[6] = (int)hi.z; v[7] = (int)hi.w;
  return v;
}

// One workgroup tile: rows [0, rows_a) of A x rows [0, rows_b) of B.
__device__ inline void gemm_tile(const TileArgs& t, int64_t lda, int64_t ldb, int64_t ssam,
                                 int64_t ssak, int64_t ssbk, int64_t K, void* Cp, int c_dtype,
                                 int64_t ldc, int64_t c_row0, int64_t c_col0, int64_t ncols_valid) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_a[2][BM * BK];
  __shared__ __attribute__((aligned(16))) uint8_t lds_b[2][BN * BK];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;  // wave's 64x64 sub-tile
  const int l16 = lane & 15, kq = lane >> 4;

  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  const int nk = (int)cdiv(K, BK);
  uint4 ra[4], rb[4];
  load_tile_regs(t.A, lda, t.rows_a, 0, K, ra);
  load_tile_regs(t.B, ldb, t.rows_b, 0, K, rb);
  store_tile_lds(lds_a[0], ra);
  store_tile_lds(lds_b[0], rb);
  __syncthreads();

  // per-lane A-scale rows: m = wm*64 + i*16 + l16
  const float* sa_row[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int m = wm * 64 + i * 16 + l16;
    if (m >= t.rows_a) m = t.rows_a - 1;  // rows beyond the tile are never stored
    sa_row[i] = t.sa + (int64_t)m * ssam;
  }

  for (int kb = 0; kb < nk; ++kb) {
    const int cur = kb & 1;
    if (kb + 1 < nk) {
      load_tile_regs(t.A, lda, t.rows_a, (int64_t)(kb + 1) * BK, K, ra);
      load_tile_regs(t.B, ldb, t.rows_b, (int64_t)(kb + 1) * BK, K, rb);
    }
    const float sbv = t.sb[(int64_t)kb * ssbk];
    float cs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) cs[i] = sa_row[i][(int64_t)kb * ssak] * sbv;

    v8i af[4], bf[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) af[i] = read_frag(lds_a[cur], wm * 64 + i * 16 + l16, kq);
#pragma unroll
    for (int j = 0; j < 4; ++j) bf[j] = read_frag(lds_b[cur], wn * 64 + j * 16 + l16, kq);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const v4f zero = {0.f, 0.f, 0.f, 0.f};
        // D[n][m] = sum_k B[n,k] A[m,k]; lane holds m = l16, n = 4*kq + r
        v4f p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf[j], af[i], zero, 0, 0, 0, 0,
                                                                 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][j][r] = fmaf(p[r], cs[i], acc[i][j][r]);
      }
    }
    if (kb + 1 < nk) {
      store_tile_lds(lds_a[cur ^ 1], ra);
      store_tile_lds(lds_b[cur ^ 1], rb);
    }
    __syncthreads();
  }

  // epilogue: lane stores C[m][n .. n+3]
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = wm * 64 + i * 16 + l16;
    if (m >= t.rows_a) continue;
    const int64_t crow = c_row0 + m;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = wn * 64 + j * 16 + kq * 4;
      const int64_t ccol = c_col0 + n;
      if (c_dtype == CIN_DT_F32) {
        float* cp = static_cast<float*>(Cp) + crow * ldc + ccol;
        if (n + 4 <= ncols_valid && (((uintptr_t)cp) & 15) == 0) {
          *reinterpret_cast<float4*>(cp) = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
        } else {
          for (int r = 0; r < 4; ++r)
            if (n + r < ncols_valid) cp[r] = acc[i][j][r];
        }
      } else {
        uint16_t* cp = static_cast<uint16_t*>(Cp) + crow * ldc + ccol;
        const uint32_t b0 = f32_to_half_bits(c_dtype, acc[i][j][0]), b1 = f32_to_half_bits(c_dtype, acc[i][j][1]);
        const uint32_t b2 = f32_to_half_bits(c_dtype, acc[i][j][2]), b3 = f32_to_half_bits(c_dtype, acc[i][j][3]);
        if (n + 4 <= ncols_valid && (((uintptr_t)cp) & 7) == 0) {
          *reinterpret_cast<uint2*>(cp) = make_uint2(b0 | (b1 << 16), b2 | (b3 << 16));
        } else {
          const uint32_t bb[4] = {b0, b1, b2, b3};
          for (int r = 0; r < 4; ++r)
            if (n + r < ncols_valid) cp[r] = (uint16_t)bb[r];
        }
      }
    }
  }
}

__global__ __launch_bounds__(kThreads, 2) void k_gemm_fp8_bs(
    const uint8_t* __restrict__ A, int64_t lda, const float* __restrict__ sa, int64_t ssam,
    int64_t ssak, const uint8_t* __restrict__ B, int64_t ldb, const float* __restrict__ sb,
    int64_t ssbn, int64_t ssbk, int64_t M, int64_t N, int64_t K, void* C, int c_dtype,
    int64_t ldc, uint32_t ntn) {
  // 1-D grid, n-tiles fastest so neighbouring workgroups share an A row panel
  const uint32_t mt = blockIdx.x / ntn, nt = blockIdx.x - mt * ntn;
  const int64_t n0 = (int64_t)nt * BN, m0 = (int64_t)mt * BM;
  TileArgs t;
  t.A = A + m0 * lda;
  t.sa = sa + m0 * ssam;
  t.B = B + n0 * ldb;
  t.sb = sb + (n0 / 128) * ssbn;
  t.rows_a = (int)((M - m0) < BM ? (M - m0) : BM);
  t.rows_b = (int)((N - n0) < BN ? (N - n0) : BN);
  gemm_tile(t, lda, ldb, ssam, ssak, ssbk, K, C, c_dtype, ldc, m0, n0, t.rows_b);
}

// Grouped: blockIdx.y enumerates (expert, 128-row tile) pairs through the
// device-side table built from starts/ends; workgroups past the last tile exit.
__global__ __launch_bounds__(kThreads, 2) void k_grouped_gemm_fp8(
    const uint8_t* __restrict__ A, int64_t lda, const float* __restrict__ sa, int64_t ssam,
    int64_t ssak, const uint8_t* __restrict__ B, int64_t sbe, int64_t ldb,
    const float* __restrict__ sb, int64_t ssbe, int64_t ssbn, int64_t ssbk,
    const int64_t* __restrict__ starts, const int64_t* __restrict__ ends, int64_t E, int64_t T,
    int64_t N, int64_t K, void* C, int c_dtype, int64_t ldc, uint32_t ntn) {
  const uint32_t tile32 = blockIdx.x / ntn, nt = blockIdx.x - tile32 * ntn;
  const int64_t tile = tile32;
  int64_t acc_tiles = 0, e = -1, row0 = 0, rows = 0;
  for (int64_t x = 0; x < E; ++x) {
    int64_t s = starts[x], en = ends[x];
    if (s < 0) s = 0;
    if (en > T) en = T;
    const int64_t m = en > s ? en - s : 0;
    const int64_t nt = cdiv(m, BM);
    if (tile < acc_tiles + nt) {
      e = x;
      row0 = s + (tile - acc_tiles) * BM;
      rows = en - row0 < BM ? en - row0 : BM;
      break;
    }
    acc_tiles += nt;
  }
  if (e < 0) return;  // uniform per workgroup, before any barrier
  const int64_t n0 = (int64_t)nt * BN;
  TileArgs t;
  t.A = A + row0 * lda;
  t.sa = sa + row0 * ssam;
  t.B = B + e * sbe + n0 * ldb;
  t.sb = sb + e * ssbe + (n0 / 128) * ssbn;
  t.rows_a = (int)rows;
  t.rows_b = (int)((N - n0) < BN ? (N - n0) : BN);
  gemm_tile(t, lda, ldb, ssam, ssak, ssbk, K, C, c_dtype, ldc, row0, n0, t.rows_b);
}


// ---------------------------------------------------------------------------
// Large-tile kernel for K % 128 == 0: workgroup tile 256 x 256, 8 waves (2 x 4),
// wave tile 128 (m) x 64 (n).  Operand tiles go global -> LDS directly
// (global_load_lds_dwordx4, no register staging); the XOR swizzle is applied by
// choosing which global chunk each lane fetches.  The 256 A-scales of a K block
// are staged into LDS the same way.  Two LDS stages, one barrier per K block.
// ---------------------------------------------------------------------------
namespace big {

// Workgroup tile 256 x 256 x 128, 8 waves (2 per SIMD), wave tile 128 (m) x 64 (n), two
// LDS stages.  Per K block a wave issues 32 MFMAs (8 m-tiles x 4 n-tiles) and the 4
// scale-FMAs of each, from a 4-slot partial ring (an FMA reads the MFMA three steps back,
// long finished, so no wave waits on its own MFMA).  The one-round kernels here run the
// ping-pong schedule of tile_body; the persistent kernels (namespace pers) interleave each
// wave's fragment reads with its own MFMAs instead.
//
// Operands move global -> LDS by DMA (buffer_load ... lds), one K block ahead, with no
// VGPR staging and no ds_write.  The DMA is issued from inline assembly: the compiler
// treats its own LDS-DMA builtin as aliasing every LDS read and would wait for it before
// each one.
constexpr int TM = 256, TN = 256, TK = 128;
constexpr int kThreads = 512;
constexpr int kTileBytes = TM * TK;  // 32 KB per operand per stage

struct __attribute__((aligned(16))) Smem {
  uint8_t a[2][kTileBytes];
  uint8_t b[2][kTileBytes];
  float sa[2][TM];  // A-row scales, slot q holds row sa_row(q)
};
// After the K loop the same LDS stages a bf16 C tile: 256 rows of 512 bytes, each padded
// by 16 bytes (a row stride of 132 dwords, 4 banks apart modulo 64): the 8-byte stores of
// the 16 rows x 2 column groups that one pass of a fragment store serves land on 64
// distinct banks.  (A 32-byte pad put rows l and l + 8 on the same banks.)
constexpr int kCStride = TN * 2 + 16;
union SmemAll {
  Smem s;
  uint8_t c[TM * kCStride];
};

// Slot q = 128 wm + 64 h + 4 l + e holds row 128 wm + 16 (4 h + e) + l: the lane (wm, l)
// finds the scales of m-tiles 0-3 in the 16 bytes at slot 128 wm + 4 l and those of m-tiles
// 4-7 at slot 128 wm + 64 + 4 l, so the 16 lanes of one 16-byte LDS read cover 64
// consecutive dwords, one per bank.  (32 contiguous bytes per lane put lanes l and l + 8 on
// the same banks: 0.7 M of the kernel's 1.7 M bank-conflict cycles on the config-2 shape.)
__device__ inline int sa_row(int q) {
  return (q & ~127) + (((q >> 6) & 1) * 4 + (q & 3)) * 16 + ((q >> 2) & 15);
}

// 16-byte chunk c of tile row r lives at slot c ^ f(r), f(r) = (r % 8) ^ ((r / 8) % 2):
// the 8 rows a 32-bank LDS serves together, and the 8 same-parity rows a 64-bank LDS
// serves together, all hit distinct banks.
__device__ inline int swz_f(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// DMA of 16 (4) bytes per lane from the buffer to LDS: lane t's bytes land at LDS byte
// address lds + 16 t (4 t).  lds is wave-uniform.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(lds), "v"(voff), "s"(r), "s"(soff) : "memory");
}
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds"
               :: "s"(lds), "v"(voff), "s"(r), "s"(soff) : "memory");
}
// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima)
__device__ __forceinline__ void wait_dma() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// Vector memory operations a wave issues for one K block's DMA: 4 row groups x (A, B), plus
// the A scales on waves 0-3.  s_waitcnt vmcnt(8): everything but the last 8 has completed.
constexpr int kDmaOpsPerBlock = 8;
__device__ __forceinline__ void wait_dma_but_block() {
  static_assert(kDmaOpsPerBlock == 8, "encoding below is vmcnt(8)");
  __builtin_amdgcn_s_waitcnt(0x0F78);
}

// One full 256 x 256 tile.  A / sa point at the tile's first row, B / sb at its first
// column block; the tile stores local rows [row_lo, row_hi) and local columns >= col_lo.
struct Tile {
  const uint8_t* A;
  const float* sa;
  const uint8_t* B;
  const float* sb;
  void* C;  // element (0, 0) of the tile
  int row_lo, row_hi, col_lo;
  int nk = 0;  // K blocks of this tile, where they vary per tile (grouped wgrad)
};

// Four consecutive fp32 columns of one accumulator entry -> four packed values of the
// 16-bit dtype OUT (two 32-bit words, lowest column in the lowest bits).
template <int OUT>
__device__ __forceinline__ uint2 pack4(const v4f& a) {
  return make_uint2(f32x2_to_half2_bits<OUT>(a[0], a[1]), f32x2_to_half2_bits<OUT>(a[2], a[3]));
}

// The 16-bit tile into LDS as a row-major 256 x 256 array (row stride kCStride bytes).
template <int OUT>
__device__ __forceinline__ void stage_tile16(const v4f (&acc)[8][4], SmemAll& smu, int wm, int wn,
                                             int l16, int kq) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int m = wm * 128 + i * 16 + l16;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = wn * 64 + j * 16 + kq * 4;
      *reinterpret_cast<uint2*>(&smu.c[m * kCStride + n * 2]) = pack4<OUT>(acc[i][j]);
    }
  }
}

// The finished 256 x 256 tile out of the accumulators: lane (wave, lane) holds rows
// 128 wm + 16 i + l16 and columns 64 wn + 16 j + 4 kq .. + 3 of m-tile i, n-tile j.
__device__ __forceinline__ void store_tile(const Tile& T, const v4f (&acc)[8][4], SmemAll& smu, int wave,
                                           int lane, int c_dtype, int64_t ldc) {
  const int wm = wave >> 2, wn = wave & 3;
  const int l16 = lane & 15, kq = lane >> 4;
  // bf16 epilogue through LDS: the fragments go to a row-major tile, then every wave
  // stores 32 whole rows, 512 contiguous bytes per row (the direct stores below write
  // each row in 32-byte pieces).  All tiles finish together, so the 32 MB or so of C
  // leave in one burst bounded by HBM write bandwidth; full rows keep it near that bound,
  // and non-temporal stores (C is not read again by this kernel) shave ~1% more.
  if (c_dtype != CIN_DT_F32 && ((((uintptr_t)T.C) & 15) == 0) && (ldc & 7) == 0) {
    __syncthreads();  // every wave is past its last fragment read
    if (c_dtype == CIN_DT_F16)
      stage_tile16<CIN_DT_F16>(acc, smu, wm, wn, l16, kq);
    else
      stage_tile16<CIN_DT_BF16>(acc, smu, wm, wn, l16, kq);
    __syncthreads();
    const int half = lane >> 5, c16 = lane & 31;  // lane: row half, 16-byte column chunk
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = wave * 32 + r * 2 + half;
      const uint4 v = *reinterpret_cast<const uint4*>(&smu.c[m * kCStride + c16 * 16]);
      if (m >= T.row_lo && m < T.row_hi && c16 * 8 >= T.col_lo)
        __builtin_nontemporal_store(u32x4v{v.x, v.y, v.z, v.w},
                                    reinterpret_cast<u32x4v*>(static_cast<uint16_t*>(T.C) + (int64_t)m * ldc + c16 * 8));
    }
    return;
  }
  // epilogue: lane holds C[m][n .. n+3] (n a multiple of 4, so a shifted tile's
  // column skip, a multiple of 128, never splits a lane's 4 columns)
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int m = wm * 128 + i * 16 + l16;
    if (m < T.row_lo || m >= T.row_hi) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = wn * 64 + j * 16 + kq * 4;
      if (n < T.col_lo) continue;
      if (c_dtype == CIN_DT_F32) {
        float* cp = static_cast<float*>(T.C) + (int64_t)m * ldc + n;
        if ((((uintptr_t)cp) & 15) == 0) {
          *reinterpret_cast<float4*>(cp) = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
        } else {
          for (int r = 0; r < 4; ++r) cp[r] = acc[i][j][r];
        }
      } else {
        uint16_t* cp = static_cast<uint16_t*>(T.C) + (int64_t)m * ldc + n;
        const uint32_t b0 = f32_to_half_bits(c_dtype, acc[i][j][0]), b1 = f32_to_half_bits(c_dtype, acc[i][j][1]);
        const uint32_t b2 = f32_to_half_bits(c_dtype, acc[i][j][2]), b3 = f32_to_half_bits(c_dtype, acc[i][j][3]);
        if ((((uintptr_t)cp) & 7) == 0) {
          *reinterpret_cast<uint2*>(cp) = make_uint2(b0 | (b1 << 16), b2 | (b3 << 16));
        } else {
          cp[0] = (uint16_t)b0; cp[1] = (uint16_t)b1; cp[2] = (uint16_t)b2; cp[3] = (uint16_t)b3;
        }
      }
    }
  }
}

// s_waitcnt lgkmcnt(0) (vmcnt and expcnt left at their maxima), then a workgroup barrier
// that the compiler may not move LDS accesses across.  No vmcnt wait: operand DMA stays in
// flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Read half H of block kb: its four A fragments, and for H = 0 the B fragments and the
// combined scales sa * sb of the wave's eight m-tiles
#define CIN_PP_LOAD(kb, H)                                                                    \
  do {                                                                                        \
    const int stg_ = (kb) & 1;                                                                \
    if ((H) == 0) {                                                                           \
      _Pragma("unroll") for (int j_ = 0; j_ < 4; ++j_) bf[j_] = CIN_BFRAG(stg_, j_);          \
      const float4 lo_ = *reinterpret_cast<const float4*>(lds + fs + (uint32_t)(stg_ * TM * 4)); \
      const float4 hi_ = *reinterpret_cast<const float4*>(lds + fs + (uint32_t)(stg_ * TM * 4 + 256)); \
      const float sb_ = kSbEarly ? sbn : (float)sbp[(int64_t)kphys(kb) * ssbk];               \
      cs[0] = lo_.x * sb_; cs[1] = lo_.y * sb_; cs[2] = lo_.z * sb_; cs[3] = lo_.w * sb_;     \
      cs[4] = hi_.x * sb_; cs[5] = hi_.y * sb_; cs[6] = hi_.z * sb_; cs[7] = hi_.w * sb_;     \
    }                                                                                         \
    _Pragma("unroll") for (int q_ = 0; q_ < 4; ++q_) af[q_] = CIN_AFRAG(stg_, 4 * (H) + q_);  \
  } while (0)
// The 16 MFMAs of half H; before MFMA s, the scale-FMAs of MFMA s - 3 (for s < 3, of the
// previous half's last m-tile, whose combined scale is cprev)
#define CIN_PP_COMPUTE(H, SBL)                                                                \
  do {                                                                                        \
    __builtin_amdgcn_s_setprio(1);                                                            \
    _Pragma("unroll") for (int s_ = 0; s_ < 16; ++s_) {                                       \
      {                                                                                       \
        const int ti = s_ >= 3 ? 4 * (H) + ((s_ - 3) >> 2) : ((H) ? 3 : 7);                   \
        const int tj = (s_ + 1) & 3;                                                          \
        const float c = s_ >= 3 ? cs[4 * (H) + ((s_ - 3) >> 2)] : cprev;                      \
        asm volatile("" : "+v"(acc[ti][tj]));                                                 \
        _Pragma("unroll") for (int r = 0; r < 4; ++r)                                         \
          acc[ti][tj][r] = fmaf(p[(s_ + 1) & 3][r], c, acc[ti][tj][r]);                       \
        asm volatile("" : "+v"(acc[ti][tj]));                                                 \
      }                                                                                       \
      asm volatile("" : "+v"(bf[s_ & 3]));                                                    \
      p[s_ & 3] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf[s_ & 3], af[s_ >> 2], zero, 0, 0, 0, 0, 0, 0); \
      asm volatile("" : "+v"(bf[s_ & 3]));                                                    \
      if (kSbEarly && (SBL) && s_ == 12) CIN_PP_SB_NEXT();                                    \
    }                                                                                         \
    cprev = cs[4 * (H) + 3];                                                                  \
    __builtin_amdgcn_s_setprio(0);                                                            \
  } while (0)

// CIN_PP_COMPUTE(0) with the reads of half 1's A fragments of the same block interleaved:
// A fragment q of half 1 right after MFMA 4q + 3, the last MFMA to read af[q].  (Reading the
// next block's half 0 the same way under half 1 measured no faster.)
#define CIN_PP_COMPUTE0_READ1(kbl, SBL)                                                       \
  do {                                                                                        \
    const int stgl_ = (kbl) & 1;                                                              \
    __builtin_amdgcn_s_setprio(1);                                                            \
    _Pragma("unroll") for (int s_ = 0; s_ < 16; ++s_) {                                       \
      {                                                                                       \
        const int ti = s_ >= 3 ? (s_ - 3) >> 2 : 7;                                           \
        const int tj = (s_ + 1) & 3;                                                          \
        const float c = s_ >= 3 ? cs[(s_ - 3) >> 2] : cprev;                                  \
        asm volatile("" : "+v"(acc[ti][tj]));                                                 \
        _Pragma("unroll") for (int r = 0; r < 4; ++r)                                         \
          acc[ti][tj][r] = fmaf(p[(s_ + 1) & 3][r], c, acc[ti][tj][r]);                       \
        asm volatile("" : "+v"(acc[ti][tj]));                                                 \
      }                                                                                       \
      asm volatile("" : "+v"(bf[s_ & 3]));                                                    \
      p[s_ & 3] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf[s_ & 3], af[s_ >> 2], zero, 0, 0, 0, 0, 0, 0); \
      asm volatile("" : "+v"(bf[s_ & 3]));                                                    \
      if ((s_ & 3) == 3) {                                                                    \
        asm volatile("" : "+v"(af[s_ >> 2]));                                                 \
        af[s_ >> 2] = CIN_AFRAG(stgl_, 4 + (s_ >> 2));                                        \
      }                                                                                       \
      if (kSbEarly && (SBL) && s_ == 12) CIN_PP_SB_NEXT();                                    \
    }                                                                                         \
    cprev = cs[3];                                                                            \
    __builtin_amdgcn_s_setprio(0);                                                            \
  } while (0)

// kSbEarly (a constant of the enclosing function): the next block's B-block scale (a scalar
// load; the loop defines kb and more) is issued after MFMA 12 of the compute half that
// precedes the block's barrier, where every fragment that half reads has been waited for and
// the barrier's lgkmcnt(0) covers the load.  Otherwise it is loaded with the block's
// fragments; scalar loads return out of order with LDS reads, so the wait before the scale
// products is then lgkmcnt(0), behind every fragment read issued so far.  Early, on two
// boxes: C2 100.5 -> 99.3 and 101.0 -> 100.4 us, C4 wgrad 108.1 -> 105.5 and 105.4 -> 105.7
// us; in the persistent walks 0.7-1.1% slower (C3 gate/up, down), which keep the loads
// together.
#define CIN_PP_SB_NEXT() (sbn = sbp[(int64_t)kphys(more ? kb + 1 : kb) * ssbk])

// The K loop of the ping-pong schedule and its drain, for a workgroup whose operands of
// block 0 have landed (blocks 0 and 1 DMA'd by all eight waves, block 0 waited for and a
// barrier passed).  kLoadsFirst (a constant of the enclosing function) orders a group's
// fragment reads before its DMA burst in the same slot, so the reads do not queue behind
// DMA issue stalls: faster in the persistent walks (C4 dgrad 150.8 -> 144.8 us, C3 down
// 2304 -> 2281 us), 0.8 us slower on the one-round C2 GEMM, which keeps the DMA first.
// The enclosing function defines the per-group DMA of the loop:
// CIN_DMA_A4(kb, stg) (waves 0-3: block kb's A rows and A scales) and CIN_DMA_B4(kb, stg)
// (waves 4-7: block kb's B rows), and the fragment reads CIN_AFRAG / CIN_BFRAG.
#define CIN_PP_KLOOP()                                                                              \
  do {                                                                                              \
/* each group runs its own copy of the K loop (the same barriers in the same order), so */          \
/* the compiler sees one straight sequence of slots per wave */                                     \
  float sbn = kSbEarly ? (float)sbp[(int64_t)kphys(0) * ssbk] : 0.0f;                              \
  if (grp == 0) {                                                                                   \
    CIN_PP_LOAD(0, 0);                                                                              \
    for (int kb = 0; kb < nk; ++kb) {                                                               \
      const int st = kb & 1;                                                                        \
      const bool more = kb < kl;                                                                    \
      CIN_PP_COMPUTE0_READ1(kb, 0);  /* slots A and B: half 1's A fragments read under half 0 */    \
      CIN_PP_COMPUTE(1, 1);  /* slot C: block kb's stage is read for the last time; kb+1 lands */   \
      wait_dma();                                                                                   \
      lds_barrier();                                                                                \
      if (more) {  /* slot D */                                                                     \
        if (!kLoadsFirst && kb + 2 < nk) CIN_DMA_A4(kb + 2, st);                                    \
        CIN_PP_LOAD(kb + 1, 0);                                                                     \
        if (kLoadsFirst && kb + 2 < nk) CIN_DMA_A4(kb + 2, st);                                     \
      }                                                                                             \
      /* a use outside slot D, so the scale load is not sunk past the barrier into it */            \
      if (kSbEarly) asm volatile("" ::"s"(sbn));                                                    \
    }                                                                                               \
  } else {                                                                                          \
    for (int kb = 0; kb < nk; ++kb) {                                                               \
      const int st = kb & 1;                                                                        \
      const bool more = kb < kl;                                                                    \
      if (!kLoadsFirst && kb >= 1 && more) CIN_DMA_B4(kb + 1, st ^ 1);  /* slot A */                \
      CIN_PP_LOAD(kb, 0);                                                                           \
      if (kLoadsFirst && kb >= 1 && more) CIN_DMA_B4(kb + 1, st ^ 1);                               \
      CIN_PP_COMPUTE0_READ1(kb, 1);  /* slots B and C */                                            \
      wait_dma();                                                                                   \
      lds_barrier();                                                                                \
      CIN_PP_COMPUTE(1, 0);                                                                         \
    }                                                                                               \
  }                                                                                                 \
/* drain: FMAs of the last half's MFMAs 13-15 (m-tile 7) */                                         \
_Pragma("unroll")                                                                                   \
  for (int s = 13; s < 16; ++s) {                                                                   \
_Pragma("unroll")                                                                                   \
    for (int r = 0; r < 4; ++r) acc[7][s & 3][r] = fmaf(p[s & 3][r], cprev, acc[7][s & 3][r]);      \
  }                                                                                                 \
  } while (0)

// One full tile, scheduled as a ping-pong between the two waves of each SIMD.  Waves 0-3
// (rows 0-127, one per SIMD) and waves 4-7 (rows 128-255) run half a K block apart: while
// one wave of a SIMD issues the 16 MFMAs of half a K block (m-tiles 4h .. 4h+3 against its
// 4 n-tiles) from fragments already in its registers, at raised issue priority, the other
// reads its next half's fragments from LDS and issues operand DMA.  A K block is four slots:
//   A: waves 0-3 compute (kb, 0); waves 4-7 read (kb, 0) and DMA B of block kb+1
//   B: waves 4-7 compute (kb, 0); waves 0-3 read (kb, 1)
//   C: waves 0-3 compute (kb, 1); waves 4-7 read (kb, 1); then block kb+1 has landed
//   D: waves 4-7 compute (kb, 1); waves 0-3 read (kb+1, 0) and DMA A of block kb+2
// (Both groups read half 1's A fragments between half 0's MFMAs, as each MFMA frees its
// fragment registers, so a wave does not wait for them at its next half.)
// One barrier per K block, after C: block kb's stage is no longer read and block kb+1's DMA
// is complete.  (A barrier after every slot, to hold the alternation exactly, measured
// slower.)  Before MFMA s of a half, the wave issues the 4 scale-FMAs of MFMA s - 3 from a
// 4-slot partial ring that runs across halves and K blocks, so an FMA reads a result whose
// MFMA finished long ago.
__device__ __forceinline__ void tile_body(const Tile& T, int64_t lda, int64_t ssam, int64_t ssak,
                                          int64_t ldb, int64_t ssbn, int64_t ssbk, int64_t K,
                                          int c_dtype, int64_t ldc) {
  __shared__ SmemAll smu;
  Smem& sm = smu.s;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2, w4 = wave & 3;
  const int wm = grp, wn = w4;
  const int l16 = lane & 15, kq = lane >> 4;
  const int nk = (int)(K / TK);

  // prologue DMA (blocks 0 and 1, all eight waves): as in tile_body
  const int r0 = tid >> 3;
  const uint32_t q16 = (uint32_t)(((tid & 7) ^ swz_f(r0)) * 16);
  const uint32_t offA = (uint32_t)(r0 * lda) + q16;
  const uint32_t offB = (uint32_t)(r0 * ldb) + q16;
  const uint32_t stepa = (uint32_t)(64 * lda), stepb = (uint32_t)(64 * ldb);
  // loop DMA, one group of four waves per operand: operation i of wave w4 covers tile rows
  // 32 i + 8 w4 .. + 7 (lane t: row 32 i + 8 w4 + t / 8, chunk (t % 8) ^ f(row)), landing
  // at LDS slot 256 i + 64 w4 + t -- the layout the eight-wave DMA writes
  const int r4 = 8 * w4 + (lane >> 3);
  const uint32_t q4 = (uint32_t)(((lane & 7) ^ swz_f(r4)) * 16);
  const uint32_t offA4 = (uint32_t)(r4 * lda) + q4, offB4 = (uint32_t)(r4 * ldb) + q4;
  const uint32_t stepa4 = (uint32_t)(32 * lda), stepb4 = (uint32_t)(32 * ldb);
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(T.A, 255 * lda + K);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(T.B, 255 * ldb + K);
  const int kl = nk - 1;
  const __amdgpu_buffer_rsrc_t rsa = make_rsrc(T.sa, (255 * ssam + (int64_t)kl * ssak + 1) * 4);
  const uint32_t offS = (uint32_t)(sa_row(w4 * 64 + lane) * ssam * 4);
  const uint32_t stepsa = (uint32_t)(ssak * 4);
  const float* sbp = T.sb + (int64_t)(wn >> 1) * ssbn;
  const int kb0 = nk >= 16 ? (int)(((blockIdx.x & 7u) * (uint32_t)nk) >> 3) : 0;
  auto kphys = [&](int kb) { const int p = kb + kb0; return p < nk ? p : p - nk; };
  const uint32_t lds_a = (uint32_t)(uintptr_t)&sm.a[0][0] + (uint32_t)(wave * 64 * 16);
  const uint32_t lds_b = (uint32_t)(uintptr_t)&sm.b[0][0] + (uint32_t)(wave * 64 * 16);
  const uint32_t lds_a4 = (uint32_t)(uintptr_t)&sm.a[0][0] + (uint32_t)(w4 * 64 * 16);
  const uint32_t lds_b4 = (uint32_t)(uintptr_t)&sm.b[0][0] + (uint32_t)(w4 * 64 * 16);
  const uint32_t lds_s = (uint32_t)(uintptr_t)&sm.sa[0][0] + (uint32_t)(w4 * 64 * 4);
#define CIN_DMA_GROUP(kb, stg, g)                                                             \
  do {                                                                                        \
    const uint32_t ko = (uint32_t)kphys(kb) * TK;                                             \
    const uint32_t so = (uint32_t)(stg) * kTileBytes;                                         \
    dma16(ra, offA, ko + (g) * stepa, lds_a + so + (g) * kThreads * 16);                      \
    dma16(rb, offB, ko + (g) * stepb, lds_b + so + (g) * kThreads * 16);                      \
    if ((g) == 0 && wave < 4)                                                                 \
      dma4(rsa, offS, (uint32_t)kphys(kb) * stepsa, lds_s + (uint32_t)(stg) * TM * 4);        \
  } while (0)
#define CIN_DMA(kb, stg)                                                                      \
  do {                                                                                        \
    _Pragma("unroll") for (int g_ = 0; g_ < 4; ++g_) CIN_DMA_GROUP(kb, stg, g_);              \
  } while (0)
// all of block kb's A rows and A scales into stage stg (waves 0-3), or all its B rows (4-7)
#define CIN_DMA_A4(kb, stg)                                                                   \
  do {                                                                                        \
    const uint32_t ko = (uint32_t)kphys(kb) * TK;                                             \
    const uint32_t so = (uint32_t)(stg) * kTileBytes;                                         \
    _Pragma("unroll") for (int i_ = 0; i_ < 8; ++i_)                                          \
      dma16(ra, offA4, ko + i_ * stepa4, lds_a4 + so + i_ * 4096);                            \
    dma4(rsa, offS, (uint32_t)kphys(kb) * stepsa, lds_s + (uint32_t)(stg) * TM * 4);          \
  } while (0)
#define CIN_DMA_B4(kb, stg)                                                                   \
  do {                                                                                        \
    const uint32_t ko = (uint32_t)kphys(kb) * TK;                                             \
    const uint32_t so = (uint32_t)(stg) * kTileBytes;                                         \
    _Pragma("unroll") for (int i_ = 0; i_ < 8; ++i_)                                          \
      dma16(rb, offB4, ko + i_ * stepb4, lds_b4 + so + i_ * 4096);                            \
  } while (0)

  const uint8_t* lds = reinterpret_cast<const uint8_t*>(&sm);
  const int fsw = swz_f(l16);
  uint32_t fa = (uint32_t)((wm * 128 + l16) * TK + (((2 * kq) ^ fsw) << 4));
  uint32_t fb = (uint32_t)(offsetof(Smem, b) + (wn * 64 + l16) * TK + (((2 * kq) ^ fsw) << 4));
  uint32_t fs = (uint32_t)(offsetof(Smem, sa) + (wm * 128 + l16 * 4) * 4);
  uint32_t fa_hi = fa ^ 16u, fb_hi = fb ^ 16u;
  asm volatile("" : "+v"(fa), "+v"(fb), "+v"(fs), "+v"(fa_hi), "+v"(fb_hi));
#define CIN_FRAG(base, base_hi, cofs)                                                       \
  ({                                                                                        \
    const uint4 lo_ = *reinterpret_cast<const uint4*>(lds + (base) + (cofs));               \
    const uint4 hi_ = *reinterpret_cast<const uint4*>(lds + (base_hi) + (cofs));            \
    v8i v_;                                                                                 \
    v_[0] = (int)lo_.x; v_[1] = (int)lo_.y; v_[2] = (int)lo_.z; v_[3] = (int)lo_.w;         \
    v_[4] = (int)hi_.x; v_[5] = (int)hi_.y; v_[6] = (int)hi_.z; v_[7] = (int)hi_.w;         \
    v_;                                                                                     \
  })
#define CIN_AFRAG(stg, mt) CIN_FRAG(fa, fa_hi, (uint32_t)((stg) * kTileBytes + (mt) * 16 * TK))
#define CIN_BFRAG(stg, nt) CIN_FRAG(fb, fb_hi, (uint32_t)((stg) * kTileBytes + (nt) * 16 * TK))

  v4f acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
  const v4f zero = {0.f, 0.f, 0.f, 0.f};
  constexpr bool kLoadsFirst = false;
  constexpr bool kSbEarly = true;
  v8i af[4], bf[4];
  float cs[8];
  float cprev = 0.0f;  // the "previous half" FMAs of the first half add 0 * 0
  v4f p[4] = {zero, zero, zero, zero};  // partial ring; slot s % 4 holds MFMA(s) of a half

  // prologue: blocks 0 and 1 into stages 0 and 1; block 0 visible to all, then waves 0-3
  // read their first half
  CIN_DMA(0, 0);
  if (nk > 1) {
    CIN_DMA(1, 1);
    wait_dma_but_block();
  } else {
    wait_dma();
  }
  lds_barrier();
  CIN_PP_KLOOP();
#undef CIN_DMA
#undef CIN_DMA_GROUP
#undef CIN_DMA_A4
#undef CIN_DMA_B4
#undef CIN_FRAG
#undef CIN_AFRAG
#undef CIN_BFRAG

  store_tile(T, acc, smu, wave, lane, c_dtype, ldc);
}

// XCD-aware order: workgroup b runs on XCD b % 8; give each XCD a contiguous run of
// tile ids (n fastest) so its CUs share A row panels and B in their L2.
// Tile index v -> (tm, tn): groups of GM m-tiles swept n by n, m fastest, so the 32 tiles
// an XCD runs at once share GM A row panels and 32 / GM B column panels.  Measured
// alternating in one process: GM = 8 took the config-3 grouped gate/up GEMM 4055 -> 3991
// us and its dgrad 4486 -> 4370 us against GM = 4 (down the same; GM = 16 was 1.5-2%
// slower than 8 on all three); the grouped wgrad and
// the config-4 dgrad keep GM = 4 (8 was 0.6% slower, and the same).  In the one-round
// kernel, GM = 4 took the config-4 wgrad (8 x 28 tiles) 125.5 -> 113.1 us against whole
// m rows per XCD, where every XCD read all of B; config 2 maps the same either way.
template <uint32_t GM>
__device__ inline void raster(uint32_t v, uint32_t tiles_m, uint32_t tiles_n, uint32_t& tm, uint32_t& tn) {
  const uint32_t gsz = GM * tiles_n;
  const uint32_t grp = v / gsz, first = grp * GM;
  const uint32_t gm = tiles_m - first < GM ? tiles_m - first : GM;
  const uint32_t w = v - grp * gsz;
  tm = first + w % gm;
  tn = w / gm;
}

__device__ inline uint32_t xcd_remap(uint32_t b, uint32_t G) {
  const uint32_t Gfull = G & ~7u;
  return b < Gfull ? (b & 7u) * (Gfull >> 3) + (b >> 3) : b;
}

// Every tile is a full block inside the operands (M, N >= 256, N % 128 == 0): the
// last tile of a row/column shifts back onto its neighbour and stores only the
// rows/columns its neighbour does not.
__global__ __launch_bounds__(kThreads, 2) void k_gemm_fp8_bs_256(
    const uint8_t* __restrict__ A, int64_t lda, const float* __restrict__ sa, int64_t ssam,
    int64_t ssak, const uint8_t* __restrict__ B, int64_t ldb, const float* __restrict__ sb,
    int64_t ssbn, int64_t ssbk, int64_t M, int64_t N, int64_t K, void* C, int c_dtype,
    int64_t ldc, uint32_t tiles_m, uint32_t tiles_n) {
  const uint32_t b = xcd_remap(blockIdx.x, tiles_m * tiles_n);
  uint32_t tm, tn;
  raster<4>(b, tiles_m, tiles_n, tm, tn);
  const int64_t m_nom = (int64_t)tm * TM, n_nom = (int64_t)tn * TN;
  const int64_t m0 = m_nom + TM <= M ? m_nom : M - TM;
  const int64_t n0 = n_nom + TN <= N ? n_nom : N - TN;
  const size_t es = c_dtype == CIN_DT_F32 ? 4 : 2;
  Tile t;
  t.A = A + m0 * lda;
  t.sa = sa + m0 * ssam;
  t.B = B + n0 * ldb;
  t.sb = sb + (n0 >> 7) * ssbn;
  t.C = static_cast<uint8_t*>(C) + (m0 * ldc + n0) * es;
  t.row_lo = (int)(m_nom - m0);
  t.row_hi = TM;
  t.col_lo = (int)(n_nom - n0);
  tile_body(t, lda, ssam, ssak, ldb, ssbn, ssbk, K, c_dtype, ldc);
}

// Grouped: tile id -> (expert, 256-row tile of the expert, n tile) through a scan of
// the device-side expert ranges; ids past the last tile exit before any barrier.  A
// tile that would run past the token range (T >= 256) shifts back; rows outside its
// expert's range are computed but not stored.
__global__ __launch_bounds__(kThreads, 2) void k_grouped_gemm_fp8_256(
    const uint8_t* __restrict__ A, int64_t lda, const float* __restrict__ sa, int64_t ssam,
    int64_t ssak, const uint8_t* __restrict__ B, int64_t sbe, int64_t ldb,
    const float* __restrict__ sb, int64_t ssbe, int64_t ssbn, int64_t ssbk,
    const int64_t* __restrict__ starts, const int64_t* __restrict__ ends, int64_t E, int64_t Tn,
    int64_t N, int64_t K, void* C, int c_dtype, int64_t ldc, uint32_t tiles_n, uint32_t max_tiles) {
  const uint32_t b = xcd_remap(blockIdx.x, max_tiles * tiles_n);
  const uint32_t tile = b / tiles_n, tn = b - tile * tiles_n;
  int64_t acc_tiles = 0, e = -1, r_nom = 0, r_end = 0;
  for (int64_t x = 0; x < E; ++x) {
    int64_t s0 = starts[x], s1 = ends[x];
    if (s0 < 0) s0 = 0;
    if (s1 > Tn) s1 = Tn;
    const int64_t nt = s1 > s0 ? cdiv(s1 - s0, TM) : 0;
    if ((int64_t)tile < acc_tiles + nt) {
      e = x;
      r_nom = s0 + ((int64_t)tile - acc_tiles) * TM;
      r_end = s1;
      break;
    }
    acc_tiles += nt;
  }
  if (e < 0) return;
  const int64_t m0 = r_nom + TM <= Tn ? r_nom : Tn - TM;
  const int64_t n_nom = (int64_t)tn * TN;
  const int64_t n0 = n_nom + TN <= N ? n_nom : N - TN;
  const size_t es = c_dtype == CIN_DT_F32 ? 4 : 2;
  Tile t;
  t.A = A + m0 * lda;
  t.sa = sa + m0 * ssam;
  t.B = B + e * sbe + n0 * ldb;
  t.sb = sb + e * ssbe + (n0 >> 7) * ssbn;
  t.C = static_cast<uint8_t*>(C) + (m0 * ldc + n0) * es;
  t.row_lo = (int)(r_nom - m0);
  t.row_hi = (int)((r_end - m0) < TM ? (r_end - m0) : TM);
  t.col_lo = (int)(n_nom - n0);
  tile_body(t, lda, ssam, ssak, ldb, ssbn, ssbk, K, c_dtype, ldc);
}

// Grouped weight gradient: dW_e[n, k] = sum over expert e's tokens t of
// dC[t, n] * X[t, k], with both operands quantized per expert in 128-token chunks and
// stored transposed on the padded token axis (cin_grouped.h): A = dC^T codes [N, Tpad],
// B = X^T codes [K, Tpad].  Workgroup = (expert, 256 x 256 output tile); its reduction
// runs over the expert's padded range [p_e, p_e + 128 ceil(m_e / 128)), whose padding
// columns hold code 0.  An expert without tokens gets dW_e = 0.
__global__ __launch_bounds__(kThreads, 2) void k_grouped_wgrad_fp8_256(
    const uint8_t* __restrict__ A, int64_t lda, const float* __restrict__ sa, int64_t ssam,
    int64_t ssak, const uint8_t* __restrict__ B, int64_t ldb, const float* __restrict__ sb, int64_t ssbm,
    const int64_t* __restrict__ starts, const int64_t* __restrict__ ends, int64_t Tn, int64_t tcap,
    int64_t M, int64_t N, void* C, int c_dtype, int64_t ldc, int64_t sce, uint32_t tiles_m,
    uint32_t tiles_n, uint32_t ntot) {
  // No XCD remap here: a tile's work is its expert's token count, so contiguous runs of
  // tile ids per XCD would give the XCD holding the popular experts most of the work.
  // Plain ids spread every expert's tiles round-robin over the 8 XCDs.
  const uint32_t b = blockIdx.x;
  (void)ntot;
  const uint32_t per = tiles_m * tiles_n;
  const uint32_t e = b / per, r = b - e * per;
  const uint32_t tm = r / tiles_n, tn = r - tm * tiles_n;
  // p = padded offset of expert e = sum over experts x < e of 128 ceil(m_x / 128): every
  // thread adds a strided share of the experts, then a wave sum and a sum over the 8 waves
  // (one round of loads for any E, instead of a walk over the e experts before this one)
  __shared__ double psum[kThreads / 64];
  double part = 0.0;
  for (int64_t x = threadIdx.x; x < (int64_t)e; x += kThreads) {
    int64_t a0, a1;
    clamp_range(starts, ends, x, Tn, a0, a1);
    part += (double)(128 * ((a1 - a0 + 127) / 128));   // exact: sums stay far below 2^53
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) part += __shfl_xor(part, d, 64);
  if ((threadIdx.x & 63) == 0) psum[threadIdx.x >> 6] = part;
  __syncthreads();
  double ptot = 0.0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) ptot += psum[w];
  const int64_t p = (int64_t)ptot;
  int64_t s0e, s1e;
  clamp_range(starts, ends, e, Tn, s0e, s1e);
  const int64_t m = s1e - s0e;
  int nk = (int)((m + TK - 1) / TK);
  if (p + (int64_t)nk * TK > tcap) nk = 0;  // ranges inconsistent with the operands' columns
  const int64_t m_nom = (int64_t)tm * TM, n_nom = (int64_t)tn * TN;
  const int64_t m0 = m_nom + TM <= M ? m_nom : M - TM;
  const int64_t n0 = n_nom + TN <= N ? n_nom : N - TN;
  const size_t es = c_dtype == CIN_DT_F32 ? 4 : 2;
  uint8_t* Ce = static_cast<uint8_t*>(C) + ((int64_t)e * sce + m0 * ldc + n0) * es;
  const int row_lo = (int)(m_nom - m0), col_lo = (int)(n_nom - n0);
  if (nk == 0) {
    for (int idx = threadIdx.x; idx < TM * TN; idx += kThreads) {
      const int rr = idx / TN, cc = idx - rr * TN;
      if (rr < row_lo || cc < col_lo) continue;
      if (c_dtype == CIN_DT_F32)
        reinterpret_cast<float*>(Ce)[(int64_t)rr * ldc + cc] = 0.0f;
      else
        reinterpret_cast<uint16_t*>(Ce)[(int64_t)rr * ldc + cc] = 0;
    }
    return;  // uniform: before any barrier
  }
  Tile t;
  t.A = A + m0 * lda + p;
  t.sa = sa + m0 * ssam + (p / TK) * ssak;
  t.B = B + n0 * ldb + p;
  t.sb = sb + (p / TK) * ssbm + (n0 >> 7);
  t.C = Ce;
  t.row_lo = row_lo;
  t.row_hi = TM;
  t.col_lo = col_lo;
  tile_body(t, lda, ssam, ssak, ldb, 1, ssbm, (int64_t)nk * TK, c_dtype, ldc);
}

}  // namespace big

// ---------------------------------------------------------------------------
// Persistent GEMM (grouped, and dense above one round of tiles): one workgroup per CU
// walks the tiles v, v + G, v + 2G, ... (G = workgroups), so a CU never waits for a
// workgroup to exit and the next one to start, and the next tile's first two K blocks go
// out by DMA while the current tile's C stores drain.  The K loop is big::tile_body's.  A
// grouped tile's expert comes from a prefix table of the experts' tile counts, built once
// per workgroup in LDS and searched by bisection (no per-tile scan over the experts).
// Measured on config 3 against the one-tile-per-workgroup kernel (same box, interleaved):
// gate/up 4372 -> 4124 us, down 2593 -> 2494 us.  Dense GEMMs of one round or less (config
// 2: one tile per CU) keep big::k_gemm_fp8_bs_256; above that (the config-4 dgrad, 3.5
// tiles per CU) the walk with the counted epilogue measured 2% faster.
// ---------------------------------------------------------------------------
namespace pers {

using big::dma16;
using big::dma4;
using big::kCStride;
using big::kTileBytes;
using big::sa_row;
using big::Smem;
using big::SmemAll;
using big::swz_f;
using big::Tile;
using big::TK;
using big::TM;
using big::TN;
using big::wait_dma;
using big::wait_dma_but_block;
using big::lds_barrier;
constexpr int kThreads = big::kThreads;

// Scales and expert ranges do not change during a kernel: read through the constant address
// space they are scalar loads, which wait on nothing but themselves (a vector load would
// wait behind the operand DMA in flight).
typedef __attribute__((address_space(4))) const float cfloat;
typedef __attribute__((address_space(4))) const int64_t cint64;

using big::raster;

// First tile of workgroup b: workgroup b runs on XCD b % 8, so XCD x's workgroups take the
// contiguous tile range [x G/8, (x+1) G/8) of each round of G tiles.
__device__ inline uint32_t first_tile(uint32_t b, uint32_t G) {
  return (G & 7u) ? b : (b & 7u) * (G >> 3) + (b >> 3);
}

// Dense: walk index v -> tile id (XCD-major, below) -> (tm, tn) by the grouped raster; the
// last tile of a row / column shifts back onto its neighbour and stores only its own rows /
// columns.
struct DenseSrc {
  const uint8_t* A; const float* sa; const uint8_t* B; const float* sb; uint8_t* C;
  int64_t lda, ssam, ldb, ssbn, ldc, M, N;
  int es;
  uint32_t tiles_m, tiles_n, G;  // G: the grid
  // XCD-major walk: XCD x owns the tile ids [x T / 8, (x + 1) T / 8) (with the raster of 4,
  // whole groups of 4 m-tiles when T / 8 is a multiple of 4 tiles_n, so the XCD's A panels
  // stay the same in every round while it sweeps n), and its G / 8 workgroups take them in
  // turn.  The walk index v = k G + x G / 8 + j (first_tile, then + G per tile) names
  // round k of workgroup j of XCD x.  Against ids dealt round-robin over the XCDs, C4 dgrad
  // (896 tiles) measured 120.5 -> 116.9 us; the grouped walks keep round-robin, since
  // there a tile's cost follows its expert's size (contiguous ranges unbalance the XCDs).
  __device__ static uint32_t xcd_start(uint32_t x, uint32_t T) {
    return (uint32_t)(((uint64_t)x * T) >> 3);
  }
  __device__ bool remap(uint32_t v, uint32_t& u) const {
    const uint32_t T = tiles_m * tiles_n;
    if (G & 7u) { u = v; return v < T; }
    const uint32_t Gx = G >> 3, k = v / G, i = v - k * G, x = i / Gx, j = i - x * Gx;
    const uint32_t s0 = xcd_start(x, T), s1 = xcd_start(x + 1, T);
    const uint64_t w = (uint64_t)k * Gx + j;
    u = s0 + (uint32_t)w;
    return w < s1 - s0;
  }
  // the workgroup whose first walk index is v (< G) owns fewer tiles than the busiest
  __device__ bool fewer(uint32_t v) const {
    const uint32_t T = tiles_m * tiles_n;
    if (G & 7u) { const uint32_t rem = T % G; return T > G && rem != 0 && v >= rem; }
    const uint32_t Gx = G >> 3, x = v / Gx, j = v - x * Gx;
    const uint32_t len = xcd_start(x + 1, T) - xcd_start(x, T);
    const uint32_t mine = len > j ? (len - j + Gx - 1) / Gx : 0;
    const uint32_t most = (T / 8 + (T % 8 != 0) + Gx - 1) / Gx;
    return T > G && mine < most;
  }
  __device__ uint32_t count() const { return tiles_m * tiles_n; }
  __device__ bool get(uint32_t v, Tile& t) const {
    uint32_t u;
    if (!remap(v, u)) return false;
    uint32_t tm, tn;
    raster<4>(u, tiles_m, tiles_n, tm, tn);
    const int64_t m_nom = (int64_t)tm * TM, n_nom = (int64_t)tn * TN;
    const int64_t m0 = m_nom + TM <= M ? m_nom : M - TM;
    const int64_t n0 = n_nom + TN <= N ? n_nom : N - TN;
    t.A = A + m0 * lda;
    t.sa = sa + m0 * ssam;
    t.B = B + n0 * ldb;
    t.sb = sb + (n0 >> 7) * ssbn;
    t.C = C + (m0 * ldc + n0) * es;
    t.row_lo = (int)(m_nom - m0);
    t.row_hi = TM;
    t.col_lo = (int)(n_nom - n0);
    return true;
  }
};

// Grouped forward: global m-tile gm of the concatenated experts -> expert by binary search
// in tpre (tpre[e] = 256-row tiles of the experts before e, tpre[E] = all of them).
struct GroupedSrc {
  const uint8_t* A; const float* sa; const uint8_t* B; const float* sb; uint8_t* C;
  int64_t lda, ssam, ldb, sbe, ssbe, ssbn, ldc, Tn, N;
  int es;
  uint32_t tiles_n;
  const int64_t* starts; const int64_t* ends;
  int E;
  const int* tpre;
  __device__ uint32_t count() const { return (uint32_t)tpre[E] * tiles_n; }
  // the workgroups whose first tile id is rem = T % G or more own one tile fewer
  __device__ bool fewer(uint32_t v) const {
    const uint32_t T = count(), G = gridDim.x, rem = T % G;
    return T > G && rem != 0 && v >= rem;
  }
  __device__ bool get(uint32_t v, Tile& t) const {
    const uint32_t total_m = (uint32_t)tpre[E];
    if (v >= total_m * tiles_n) return false;
    uint32_t gm, tn;
    raster<8>(v, total_m, tiles_n, gm, tn);
    int lo = 0, hi = E;  // largest e with tpre[e] <= gm (then gm < tpre[e + 1])
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if ((uint32_t)tpre[mid] <= gm) lo = mid; else hi = mid;
    }
    const int e = lo;
    int64_t s0 = ((const cint64*)starts)[e], s1 = ((const cint64*)ends)[e];
    if (s0 < 0) s0 = 0;
    if (s1 > Tn) s1 = Tn;
    if (s1 < s0) s1 = s0;
    const int64_t r_nom = s0 + (int64_t)(gm - (uint32_t)tpre[e]) * TM;
    const int64_t m0 = r_nom + TM <= Tn ? r_nom : Tn - TM;
    const int64_t n_nom = (int64_t)tn * TN;
    const int64_t n0 = n_nom + TN <= N ? n_nom : N - TN;
    t.A = A + m0 * lda;
    t.sa = sa + m0 * ssam;
    t.B = B + (int64_t)e * sbe + n0 * ldb;
    t.sb = sb + (int64_t)e * ssbe + (n0 >> 7) * ssbn;
    t.C = C + (m0 * ldc + n0) * es;
    t.row_lo = (int)(r_nom - m0);
    t.row_hi = (int)((s1 - m0) < TM ? (s1 - m0) : TM);
    t.col_lo = (int)(n_nom - n0);
    return true;
  }
};

// C of one tile from the accumulators, straight from registers: lane holds C[m][n .. n+3].
__device__ __forceinline__ void store_direct(const Tile& T, const v4f (&acc)[8][4], int wm, int wn, int l16,
                                             int kq, int c_dtype, int64_t ldc) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int m = wm * 128 + i * 16 + l16;
    if (m < T.row_lo || m >= T.row_hi) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = wn * 64 + j * 16 + kq * 4;
      if (n < T.col_lo) continue;
      if (c_dtype == CIN_DT_F32) {
        float* cp = static_cast<float*>(T.C) + (int64_t)m * ldc + n;
        if ((((uintptr_t)cp) & 15) == 0) {
          *reinterpret_cast<float4*>(cp) = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
        } else {
          for (int r = 0; r < 4; ++r) cp[r] = acc[i][j][r];
        }
      } else {
        uint16_t* cp = static_cast<uint16_t*>(T.C) + (int64_t)m * ldc + n;
        const uint32_t b0 = f32_to_half_bits(c_dtype, acc[i][j][0]), b1 = f32_to_half_bits(c_dtype, acc[i][j][1]);
        const uint32_t b2 = f32_to_half_bits(c_dtype, acc[i][j][2]), b3 = f32_to_half_bits(c_dtype, acc[i][j][3]);
        if ((((uintptr_t)cp) & 7) == 0) {
          *reinterpret_cast<uint2*>(cp) = make_uint2(b0 | (b1 << 16), b2 | (b3 << 16));
        } else {
          cp[0] = (uint16_t)b0; cp[1] = (uint16_t)b1; cp[2] = (uint16_t)b2; cp[3] = (uint16_t)b3;
        }
      }
    }
  }
}

// Where the lanes of store_counted whose element lies outside the tile's rows or columns
// write instead: one 8-byte slot per lane, never read.
__device__ uint2 g_store_sink[64];

// 16-bit C of one tile with exactly kEpiStores 8-byte stores per wave, whatever the tile's
// row and column limits: a lane outside them writes its slot of g_store_sink.  The fixed
// count lets the next tile wait for its first K block with vmcnt(kEpiStores + 8): that
// block was issued before these stores and block 1 (at most 9 operations) after it, and
// vector memory operations retire from the count in issue order, so the stores drain while
// the next tile starts.  C must be 8-byte aligned with ldc a multiple of 4.
constexpr int kEpiStores = 32;
template <int OUT>
__device__ __forceinline__ void store_counted_t(const Tile& T, const v4f (&acc)[8][4], int wm, int wn, int l16,
                                                int kq, int64_t ldc) {
  const int rl = wm * 128 + l16, cl = wn * 64 + kq * 4;
  uint16_t* c0 = static_cast<uint16_t*>(T.C) + (int64_t)rl * ldc + cl;
  uint2* sink = &g_store_sink[threadIdx.x & 63];
  const uint32_t rows = (uint32_t)(T.row_hi - T.row_lo);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bool rok = (uint32_t)(rl + 16 * i - T.row_lo) < rows;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool ok = rok && cl + 16 * j >= T.col_lo;
      uint2* p = ok ? reinterpret_cast<uint2*>(c0 + (int64_t)(16 * i) * ldc + 16 * j) : sink;
      *p = big::pack4<OUT>(acc[i][j]);
    }
  }
}
__device__ __forceinline__ void store_counted(const Tile& T, const v4f (&acc)[8][4], int wm, int wn, int l16,
                                              int kq, int c_dtype, int64_t ldc) {
  if (c_dtype == CIN_DT_F16)
    store_counted_t<CIN_DT_F16>(T, acc, wm, wn, l16, kq, ldc);
  else
    store_counted_t<CIN_DT_BF16>(T, acc, wm, wn, l16, kq, ldc);
}
// s_waitcnt vmcnt(kEpiStores + 8): all but the last 40 vector memory operations done
__device__ __forceinline__ void wait_dma_past_stores() {
  static_assert(kEpiStores + 8 == 40, "encoding below is vmcnt(40)");
  __builtin_amdgcn_s_waitcnt(0x8F78);
}

// 16-bit C of one tile with kEpiStoresX4 16-byte stores per wave.  Entries (i, j) and
// (i, j + 1) hold columns 16 j + 4 kq .. + 3 and 16 j + 16 + 4 kq .. + 3 of row l16 in
// each lane; v_permlane16_swap trades the odd 16-lane rows of the first with the even rows
// of the second, after which a lane with even kq holds 8 consecutive columns of entry j
// and a lane with odd kq 8 of entry j + 1, so the four lanes of a row write one 64-byte
// run (32 bytes per run with store_counted).  Same sink rule and drain-by-count as
// store_counted.  C must be 16-byte aligned with ldc a multiple of 8; col_lo must be a
// multiple of 8 (it is 0 or 128 here, as N is a multiple of 128).
constexpr int kEpiStoresX4 = 16;
__device__ uint4 g_store_sink16[64];
template <int OUT>
__device__ __forceinline__ void store_counted_x4_t(const Tile& T, const v4f (&acc)[8][4], int wm, int wn, int l16,
                                                   int kq, int64_t ldc) {
  const int rl = wm * 128 + l16, cl = wn * 64 + 4 * kq + ((kq & 1) ? 12 : 0);
  uint16_t* c0 = static_cast<uint16_t*>(T.C) + (int64_t)rl * ldc + cl;
  uint4* sink = &g_store_sink16[threadIdx.x & 63];
  const uint32_t rows = (uint32_t)(T.row_hi - T.row_lo);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bool rok = (uint32_t)(rl + 16 * i - T.row_lo) < rows;
#pragma unroll
    for (int jp = 0; jp < 2; ++jp) {
      const v4f& X = acc[i][2 * jp];
      const v4f& Y = acc[i][2 * jp + 1];
      const uint32_t x0 = f32x2_to_half2_bits<OUT>(X[0], X[1]), x1 = f32x2_to_half2_bits<OUT>(X[2], X[3]);
      const uint32_t y0 = f32x2_to_half2_bits<OUT>(Y[0], Y[1]), y1 = f32x2_to_half2_bits<OUT>(Y[2], Y[3]);
      const auto s0 = __builtin_amdgcn_permlane16_swap(x0, y0, false, false);
      const auto s1 = __builtin_amdgcn_permlane16_swap(x1, y1, false, false);
      const bool ok = rok && cl + 32 * jp >= T.col_lo;
      uint4* p = ok ? reinterpret_cast<uint4*>(c0 + (int64_t)(16 * i) * ldc + 32 * jp) : sink;
      *p = make_uint4(s0[0], s1[0], s0[1], s1[1]);
    }
  }
}
__device__ __forceinline__ void store_counted_x4(const Tile& T, const v4f (&acc)[8][4], int wm, int wn, int l16,
                                                 int kq, int c_dtype, int64_t ldc) {
  if (c_dtype == CIN_DT_F16)
    store_counted_x4_t<CIN_DT_F16>(T, acc, wm, wn, l16, kq, ldc);
  else
    store_counted_x4_t<CIN_DT_BF16>(T, acc, wm, wn, l16, kq, ldc);
}
// s_waitcnt vmcnt(kEpiStoresX4 + 8)
__device__ __forceinline__ void wait_dma_past_stores_x4() {
  static_assert(kEpiStoresX4 + 8 == 24, "encoding below is vmcnt(24)");
  __builtin_amdgcn_s_waitcnt(0x4F78);
}

// fp32 C of one tile with exactly kEpiStores 16-byte stores per wave (a lane holds 4
// consecutive columns of one row), the same count as store_counted, so the next tile
// waits with the same vmcnt.  C must be 16-byte aligned with ldc a multiple of 4.
__device__ float4 g_store_sink32[64];
__device__ __forceinline__ void store_counted32(const Tile& T, const v4f (&acc)[8][4], int wm, int wn, int l16,
                                                int kq, int64_t ldc) {
  const int rl = wm * 128 + l16, cl = wn * 64 + kq * 4;
  float* c0 = static_cast<float*>(T.C) + (int64_t)rl * ldc + cl;
  float4* sink = &g_store_sink32[threadIdx.x & 63];
  const uint32_t rows = (uint32_t)(T.row_hi - T.row_lo);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bool rok = (uint32_t)(rl + 16 * i - T.row_lo) < rows;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool ok = rok && cl + 16 * j >= T.col_lo;
      float4* p = ok ? reinterpret_cast<float4*>(c0 + (int64_t)(16 * i) * ldc + 16 * j) : sink;
      *p = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
    }
  }
}

// How a persistent kernel stores C: every tile with store_direct (the next tile then waits
// for everything), or with a fixed count of stores per wave that the next tile's first wait
// looks past (16-bit C: store_counted_x4, or store_counted where C is only 8-byte aligned;
// fp32 C: store_counted32).
constexpr int kEpiDirect = 0, kEpiCounted16 = 1, kEpiCounted32 = 2, kEpiCounted16x4 = 3;

// Idles the wave for about `ticks` periods of the 100 MHz real-time clock (bounded: at
// most 2^16 sleeps of about 1000 cycles each).
__device__ __forceinline__ void idle_for(uint64_t ticks) {
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < (1 << 16); ++it) {
    if (__builtin_amdgcn_s_memrealtime() - t0 >= ticks) break;
    __builtin_amdgcn_s_sleep(16);
  }
}
// Start offset of a persistent workgroup that owns one tile fewer than the busiest ones,
// in real-time ticks (10 ns) per K block of its first tile.  Tiles of equal K take about
// equal time, so workgroups that start together reach every tile boundary together, and
// all of them then store C and fetch their next tile's first blocks at once; starting the
// short workgroups late puts their boundaries inside the others' K loops.  Owning one
// tile fewer, they lose nothing while the offset stays under a tile's duration (about
// 130 ticks per K block at full clock).
constexpr uint32_t kLateStartPerBlock = 30;

// A pointer as a wave-uniform value (the DMA's buffer descriptor lives in SGPRs).
template <class P>
__device__ __forceinline__ P* uniform_ptr(P* p) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
  return (P*)(uintptr_t)((hi << 32) | lo);
}

// EPI: kEpiCounted16x4 needs 16-bit C 16-byte aligned with ldc a multiple of 8,
// kEpiCounted16 16-bit C 8-byte aligned with ldc a multiple of 4,
// kEpiCounted32 fp32 C 16-byte aligned with ldc a multiple of 4; kEpiDirect takes any C.
// VARK: the K blocks vary per tile (Tile::nk, at least 1); K is then unused.
template <int EPI, class Src, bool VARK = false>
__device__ __forceinline__ void run_tiles(const Src& src, int64_t lda, int64_t ssam, int64_t ssak,
                                          int64_t ldb, int64_t ssbn, int64_t ssbk, int64_t K,
                                          int c_dtype, int64_t ldc) {
  __shared__ SmemAll smu;
  Smem& sm = smu.s;
  const uint32_t G = gridDim.x;
  uint32_t v = first_tile(blockIdx.x, G);
  {
    Tile T0;
    if (!src.get(v, T0)) return;  // uniform per workgroup
  }
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int l16 = lane & 15, kq = lane >> 4;
  int nk = (int)(K / TK);
  int kl = nk - 1;
  const int r0 = tid >> 3;
  const uint32_t q16 = (uint32_t)(((tid & 7) ^ swz_f(r0)) * 16);
  const uint32_t offA = (uint32_t)(r0 * lda) + q16;
  const uint32_t offB = (uint32_t)(r0 * ldb) + q16;
  const uint32_t stepa = (uint32_t)(64 * lda), stepb = (uint32_t)(64 * ldb);
  // the K loop's DMA, one group of four waves per operand (as in big::tile_body)
  const int grp = wm;
  const int r4 = 8 * wn + (lane >> 3);
  const uint32_t q4 = (uint32_t)(((lane & 7) ^ swz_f(r4)) * 16);
  const uint32_t offA4 = (uint32_t)(r4 * lda) + q4, offB4 = (uint32_t)(r4 * ldb) + q4;
  const uint32_t stepa4 = (uint32_t)(32 * lda), stepb4 = (uint32_t)(32 * ldb);
  const uint32_t offS = (uint32_t)(sa_row((wave & 3) * 64 + lane) * ssam * 4);
  const uint32_t stepsa = (uint32_t)(ssak * 4);
  int64_t bytesA = 255 * lda + K, bytesB = 255 * ldb + K;
  int64_t bytesS = (255 * ssam + (int64_t)kl * ssak + 1) * 4;
  int kb0 = nk >= 16 ? (int)(((blockIdx.x & 7u) * (uint32_t)nk) >> 3) : 0;
  auto kphys = [&](int kb) { const int p = kb + kb0; return p < nk ? p : p - nk; };
  // the K geometry of a tile with n blocks (VARK: set before the tile's first DMA)
  auto set_k = [&](int n) {
    nk = n;
    kl = n - 1;
    bytesA = 255 * lda + (int64_t)n * TK;
    bytesB = 255 * ldb + (int64_t)n * TK;
    bytesS = (255 * ssam + (int64_t)kl * ssak + 1) * 4;
    kb0 = n >= 16 ? (int)(((blockIdx.x & 7u) * (uint32_t)n) >> 3) : 0;
  };
  const uint32_t lds_a = (uint32_t)(uintptr_t)&sm.a[0][0] + (uint32_t)(wave * 64 * 16);
  const uint32_t lds_b = (uint32_t)(uintptr_t)&sm.b[0][0] + (uint32_t)(wave * 64 * 16);
  const uint32_t lds_s = (uint32_t)(uintptr_t)&sm.sa[0][0] + (uint32_t)((wave & 3) * 64 * 4);
  const uint32_t lds_a4 = (uint32_t)(uintptr_t)&sm.a[0][0] + (uint32_t)(wn * 64 * 16);
  const uint32_t lds_b4 = (uint32_t)(uintptr_t)&sm.b[0][0] + (uint32_t)(wn * 64 * 16);
  // Row group g of the operands of the tile at (pA, pB, pS), block kb, into stage stg
#define CIN_DMA_GROUP_P(pA, pB, pS, kb, stg, g)                                               \
  do {                                                                                        \
    const uint32_t ko = (uint32_t)kphys(kb) * TK;                                             \
    const uint32_t so = (uint32_t)(stg) * kTileBytes;                                         \
    dma16(make_rsrc(pA, bytesA), offA, ko + (g) * stepa, lds_a + so + (g) * kThreads * 16);   \
    dma16(make_rsrc(pB, bytesB), offB, ko + (g) * stepb, lds_b + so + (g) * kThreads * 16);   \
    if ((g) == 0 && wave < 4)                                                                 \
      dma4(make_rsrc(pS, bytesS), offS, (uint32_t)kphys(kb) * stepsa,                         \
           lds_s + (uint32_t)(stg) * TM * 4);                                                 \
  } while (0)
#define CIN_DMA_P(pA, pB, pS, kb, stg)                                                        \
  do {                                                                                        \
    _Pragma("unroll") for (int g_ = 0; g_ < 4; ++g_) CIN_DMA_GROUP_P(pA, pB, pS, kb, stg, g_); \
  } while (0)
// The K loop's DMA of this tile (pA, pB, pS): all of block kb's A rows and A scales into
// stage stg (waves 0-3), or all its B rows (waves 4-7)
#define CIN_DMA_A4(kb, stg)                                                                   \
  do {                                                                                        \
    const uint32_t ko = (uint32_t)kphys(kb) * TK;                                             \
    const uint32_t so = (uint32_t)(stg) * kTileBytes;                                         \
    const __amdgpu_buffer_rsrc_t ra_ = make_rsrc(pA, bytesA);                                 \
    _Pragma("unroll") for (int i_ = 0; i_ < 8; ++i_)                                          \
      dma16(ra_, offA4, ko + i_ * stepa4, lds_a4 + so + i_ * 4096);                           \
    dma4(make_rsrc(pS, bytesS), offS, (uint32_t)kphys(kb) * stepsa, lds_s + (uint32_t)(stg) * TM * 4); \
  } while (0)
#define CIN_DMA_B4(kb, stg)                                                                   \
  do {                                                                                        \
    const uint32_t ko = (uint32_t)kphys(kb) * TK;                                             \
    const uint32_t so = (uint32_t)(stg) * kTileBytes;                                         \
    const __amdgpu_buffer_rsrc_t rb_ = make_rsrc(pB, bytesB);                                 \
    _Pragma("unroll") for (int i_ = 0; i_ < 8; ++i_)                                          \
      dma16(rb_, offB4, ko + i_ * stepb4, lds_b4 + so + i_ * 4096);                           \
  } while (0)
  const uint8_t* lds = reinterpret_cast<const uint8_t*>(&sm);
  const int fsw = swz_f(l16);
  // Per-lane LDS addresses of the fragment reads, hidden from the compiler: it would
  // otherwise split each into a lane part and a constant and, where the constant passes
  // the 64 KB immediate-offset range (B's second stage, the scales), keep one register per
  // (stage, tile) address.  Each read below is one of these bases plus an offset < 64 KB.
  uint32_t fa = (uint32_t)((wm * 128 + l16) * TK + (((2 * kq) ^ fsw) << 4));
  uint32_t fb = (uint32_t)(offsetof(Smem, b) + (wn * 64 + l16) * TK + (((2 * kq) ^ fsw) << 4));
  uint32_t fs = (uint32_t)(offsetof(Smem, sa) + (wm * 128 + l16 * 4) * 4);
  uint32_t fa_hi = fa ^ 16u, fb_hi = fb ^ 16u;  // the fragments' high halves: chunk 2 kq + 1
  asm volatile("" : "+v"(fa), "+v"(fb), "+v"(fs), "+v"(fa_hi), "+v"(fb_hi));
#define CIN_FRAG(base, base_hi, cofs)                                                       \
  ({                                                                                        \
    const uint4 lo_ = *reinterpret_cast<const uint4*>(lds + (base) + (cofs));               \
    const uint4 hi_ = *reinterpret_cast<const uint4*>(lds + (base_hi) + (cofs));            \
    v8i v_;                                                                                 \
    v_[0] = (int)lo_.x; v_[1] = (int)lo_.y; v_[2] = (int)lo_.z; v_[3] = (int)lo_.w;         \
    v_[4] = (int)hi_.x; v_[5] = (int)hi_.y; v_[6] = (int)hi_.z; v_[7] = (int)hi_.w;         \
    v_;                                                                                     \
  })
#define CIN_AFRAG(stg, mt) CIN_FRAG(fa, fa_hi, (uint32_t)((stg) * kTileBytes + (mt) * 16 * TK))
#define CIN_BFRAG(stg, nt) CIN_FRAG(fb, fb_hi, (uint32_t)((stg) * kTileBytes + (nt) * 16 * TK))

  {
    // v < G here: the first walk index of this workgroup
    if (src.fewer(v)) idle_for((uint64_t)nk * kLateStartPerBlock);
  }
  // prologue of the first tile: blocks 0 and 1 into stages 0 and 1
  {
    Tile T0;
    src.get(v, T0);
    if constexpr (VARK) set_k(T0.nk);
    const uint8_t* pA = uniform_ptr(T0.A);
    const uint8_t* pB = uniform_ptr(T0.B);
    const float* pS = uniform_ptr(T0.sa);
    CIN_DMA_P(pA, pB, pS, 0, 0);
    if (nk > 1) CIN_DMA_P(pA, pB, pS, 1, 1);
  }
  const v4f zero = {0.f, 0.f, 0.f, 0.f};
  bool first = true;  // the first tile: both blocks' DMA and nothing after them
  for (;;) {
    // this tile's operands (its blocks 0 and 1 are already on their way)
    const uint8_t* pA;
    const uint8_t* pB;
    const float* pS;
    const cfloat* sbp;  // B-block scales, read as scalar loads (see cfloat)
    // VARK: this tile and the next are looked up here, before the accumulators are live,
    // and kept (in scalar registers) through the K loop rather than looked up again after
    // it, where the accumulators are live
    Tile Tcur, Tnxt;
    bool has_next = false;
    {
      Tile T;
      src.get(v, T);
      pA = uniform_ptr(T.A);
      pB = uniform_ptr(T.B);
      pS = uniform_ptr(T.sa);
      sbp = (const cfloat*)uniform_ptr(T.sb + (int64_t)(wn >> 1) * ssbn);
      if constexpr (VARK) {
        Tcur = T;
        has_next = src.get(v + G, Tnxt);
      }
    }
    // block 0 has landed: block 1 (and, counted, the previous tile's stores) may still
    // be in flight; they are waited for at the first K block's barrier
    if (nk > 1 && first)
      wait_dma_but_block();
    else if (EPI == kEpiCounted16x4 && nk > 1)
      wait_dma_past_stores_x4();
    else if (EPI != kEpiDirect && nk > 1)
      wait_dma_past_stores();
    else
      wait_dma();
    __syncthreads();
    v4f acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = zero;
    constexpr bool kLoadsFirst = true;
    constexpr bool kSbEarly = false;
    v8i af[4], bf[4];
    float cs[8];
    float cprev = 0.0f;
    v4f p[4] = {zero, zero, zero, zero};
    CIN_PP_KLOOP();
    __syncthreads();  // every wave is past its last fragment read: both stages are free
    Tile Tn;
    bool next;  // uniform per workgroup
    if constexpr (VARK) {
      next = has_next;
      Tn = Tnxt;
    } else {
      next = src.get(v + G, Tn);
    }
    if (next) {
      // the next tile's blocks 0 and 1 go out first, then this tile's stores
      if constexpr (VARK) set_k(Tn.nk);  // this tile's K loop is done
      const uint8_t* nA = uniform_ptr(Tn.A);
      const uint8_t* nB = uniform_ptr(Tn.B);
      const float* nS = uniform_ptr(Tn.sa);
      CIN_DMA_P(nA, nB, nS, 0, 0);
      if (nk > 1) CIN_DMA_P(nA, nB, nS, 1, 1);
    }
    Tile T;
    if constexpr (VARK)
      T = Tcur;
    else
      src.get(v, T);
    if (!next && c_dtype != CIN_DT_F32 && ((((uintptr_t)T.C) & 15) == 0) && (ldc & 7) == 0) {
      // last tile of this workgroup: the LDS-staged epilogue of big::tile_body
      if (c_dtype == CIN_DT_F16)
        big::stage_tile16<CIN_DT_F16>(acc, smu, wm, wn, l16, kq);
      else
        big::stage_tile16<CIN_DT_BF16>(acc, smu, wm, wn, l16, kq);
      __syncthreads();
      const int half = lane >> 5, c16 = lane & 31;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = wave * 32 + r * 2 + half;
        const uint4 w4 = *reinterpret_cast<const uint4*>(&smu.c[m * kCStride + c16 * 16]);
        if (m >= T.row_lo && m < T.row_hi && c16 * 8 >= T.col_lo)
          __builtin_nontemporal_store(u32x4v{w4.x, w4.y, w4.z, w4.w},
                                      reinterpret_cast<u32x4v*>(static_cast<uint16_t*>(T.C) + (int64_t)m * ldc + c16 * 8));
      }
      return;
    }
    if constexpr (EPI == kEpiCounted16x4)
      store_counted_x4(T, acc, wm, wn, l16, kq, c_dtype, ldc);
    else if constexpr (EPI == kEpiCounted16)
      store_counted(T, acc, wm, wn, l16, kq, c_dtype, ldc);
    else if constexpr (EPI == kEpiCounted32)
      store_counted32(T, acc, wm, wn, l16, kq, ldc);
    else
      store_direct(T, acc, wm, wn, l16, kq, c_dtype, ldc);
    if (!next) return;
    first = false;
    v += G;
  }
#undef CIN_DMA_P
#undef CIN_DMA_GROUP_P
#undef CIN_DMA_A4
#undef CIN_DMA_B4
#undef CIN_FRAG
#undef CIN_AFRAG
#undef CIN_BFRAG
}
#undef CIN_PP_LOAD
#undef CIN_PP_COMPUTE
#undef CIN_PP_COMPUTE0_READ1
#undef CIN_PP_KLOOP

template <int EPI>
__global__ __launch_bounds__(kThreads, 1) void k_gemm_fp8_bs_pers(
    const uint8_t* __restrict__ A, int64_t lda, const float* __restrict__ sa, int64_t ssam,
    int64_t ssak, const uint8_t* __restrict__ B, int64_t ldb, const float* __restrict__ sb,
    int64_t ssbn, int64_t ssbk, int64_t M, int64_t N, int64_t K, void* C, int c_dtype,
    int64_t ldc, uint32_t tiles_m, uint32_t tiles_n) {
  DenseSrc src;
  src.A = A; src.sa = sa; src.B = B; src.sb = sb; src.C = static_cast<uint8_t*>(C);
  src.lda = lda; src.ssam = ssam; src.ldb = ldb; src.ssbn = ssbn; src.ldc = ldc; src.M = M; src.N = N;
  src.es = c_dtype == CIN_DT_F32 ? 4 : 2;
  src.tiles_m = tiles_m; src.tiles_n = tiles_n; src.G = gridDim.x;
  run_tiles<EPI>(src, lda, ssam, ssak, ldb, ssbn, ssbk, K, c_dtype, ldc);
}

constexpr int kMaxExpertsLds = 4096;

template <int EPI>
__global__ __launch_bounds__(kThreads, 1) void k_grouped_gemm_fp8_pers(
    const uint8_t* __restrict__ A, int64_t lda, const float* __restrict__ sa, int64_t ssam,
    int64_t ssak, const uint8_t* __restrict__ B, int64_t sbe, int64_t ldb,
    const float* __restrict__ sb, int64_t ssbe, int64_t ssbn, int64_t ssbk,
    const int64_t* __restrict__ starts, const int64_t* __restrict__ ends, int E, int64_t Tn,
    int64_t N, int64_t K, void* C, int c_dtype, int64_t ldc, uint32_t tiles_n) {
  __shared__ int tpre[kMaxExpertsLds + 1];
  __shared__ int wtot[kThreads / 64];
  // tpre: exclusive prefix over experts of their 256-row tile counts.  Thread t owns
  // experts [t * per, (t + 1) * per).
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (E + kThreads - 1) / kThreads;
  int mine = 0;
  for (int e = tid * per; e < tid * per + per && e < E; ++e) {
    int64_t s0, s1;
    clamp_range(starts, ends, e, Tn, s0, s1);
    mine += (int)((s1 - s0 + TM - 1) / TM);
  }
  int incl = mine;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(incl, d, 64);
    if (lane >= d) incl += o;
  }
  if (lane == 63) wtot[wave] = incl;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += wtot[w];
  int run = base + incl - mine;
  for (int e = tid * per; e < tid * per + per && e < E; ++e) {
    tpre[e] = run;
    int64_t s0, s1;
    clamp_range(starts, ends, e, Tn, s0, s1);
    run += (int)((s1 - s0 + TM - 1) / TM);
  }
  if (tid == kThreads - 1) {
    int tot = 0;
    for (int w = 0; w < kThreads / 64; ++w) tot += wtot[w];
    tpre[E] = tot;
  }
  __syncthreads();
  GroupedSrc src;
  src.A = A; src.sa = sa; src.B = B; src.sb = sb; src.C = static_cast<uint8_t*>(C);
  src.lda = lda; src.ssam = ssam; src.ldb = ldb; src.sbe = sbe; src.ssbe = ssbe; src.ssbn = ssbn;
  src.ldc = ldc; src.Tn = Tn; src.N = N; src.es = c_dtype == CIN_DT_F32 ? 4 : 2;
  src.tiles_n = tiles_n; src.starts = starts; src.ends = ends; src.E = E; src.tpre = tpre;
  run_tiles<EPI>(src, lda, ssam, ssak, ldb, ssbn, ssbk, K, c_dtype, ldc);
}

// Grouped weight gradient on the persistent walk (same operands and result as
// big::k_grouped_wgrad_fp8_256): dW_e[n, k] = sum over expert e's tokens of dC[t, n] X[t, k],
// a 256 x 256 tile's reduction running over e's padded token range, so the K blocks vary
// per tile.  Each workgroup builds, in LDS, every expert's padded offset and K blocks and
// the experts with tokens in descending order of K blocks (ties by id).  Walk index v ->
// tile: every other full round of G tiles is taken in reverse, so with the experts sorted
// the long tiles are dealt out evenly and the static walk stays balanced.
constexpr int kMaxWgradExperts = 512;
static_assert(kMaxWgradExperts <= kThreads, "the wgrad's LDS tables give each thread one expert");

struct WgradSrc {
  const uint8_t* A; const float* sa; const uint8_t* B; const float* sb; uint8_t* C;
  int64_t lda, ssam, ssak, ldb, ssbm, ldc, sce, M, N;
  int es;
  uint32_t tiles_m, tiles_n, G, total;  // total = tiles of the experts with tokens
  const int* order;    // experts with tokens, most K blocks first
  const int* enk;      // K blocks per expert (0: no tokens, or a range past the operands)
  const int64_t* poff; // padded token offset per expert
  // no start offsets (run_tiles): the tiles' K lengths differ, so owning one tile fewer
  // says little about finishing earlier
  __device__ uint32_t count() const { return 0; }
  __device__ bool fewer(uint32_t) const { return false; }  // no start offsets (above)
  __device__ bool get(uint32_t v, Tile& t) const {
    if (v >= total) return false;
    const uint32_t i = v / G, b = v - i * G;
    const uint32_t u = ((i & 1u) && (i + 1) * G <= total) ? i * G + (G - 1 - b) : v;
    const uint32_t per = tiles_m * tiles_n;
    const uint32_t rank = u / per, r = u - rank * per;
    // LDS reads are per lane to the compiler: made wave-uniform, what follows stays scalar
    const int e = __builtin_amdgcn_readfirstlane(order[rank]);
    uint32_t tm, tn;
    raster<4>(r, tiles_m, tiles_n, tm, tn);  // an XCD's 32 tiles share 4 A and 8 B panels
    const uint64_t pu = (uint64_t)poff[e];
    const int64_t p = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(pu >> 32)) << 32) |
                                (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)pu));
    const int64_t m_nom = (int64_t)tm * TM, n_nom = (int64_t)tn * TN;
    const int64_t m0 = m_nom + TM <= M ? m_nom : M - TM;
    const int64_t n0 = n_nom + TN <= N ? n_nom : N - TN;
    t.A = A + m0 * lda + p;
    t.sa = sa + m0 * ssam + (p / TK) * ssak;
    t.B = B + n0 * ldb + p;
    t.sb = sb + (p / TK) * ssbm + (n0 >> 7);
    t.C = C + ((int64_t)e * sce + m0 * ldc + n0) * es;
    t.row_lo = (int)(m_nom - m0);
    t.row_hi = TM;
    t.col_lo = (int)(n_nom - n0);
    t.nk = __builtin_amdgcn_readfirstlane(enk[e]);
    return true;
  }
};

template <int EPI>
__global__ __launch_bounds__(kThreads, 1) void k_grouped_wgrad_fp8_pers(
    const uint8_t* __restrict__ A, int64_t lda, const float* __restrict__ sa, int64_t ssam,
    int64_t ssak, const uint8_t* __restrict__ B, int64_t ldb, const float* __restrict__ sb, int64_t ssbm,
    const int64_t* __restrict__ starts, const int64_t* __restrict__ ends, int E, int64_t Tn,
    int64_t tcap, int64_t M, int64_t N, void* C, int c_dtype, int64_t ldc, int64_t sce,
    uint32_t tiles_m, uint32_t tiles_n) {
  __shared__ int order[kMaxWgradExperts];
  __shared__ int enk[kMaxWgradExperts];
  __shared__ int64_t poff[kMaxWgradExperts];
  __shared__ int wtot[kThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // thread t owns expert t (E <= kThreads): K blocks, then the exclusive prefix of the
  // padded sizes 128 * nk (the padded token axis of the operands)
  int nkt = 0;
  if (tid < E) {
    int64_t s0, s1;
    clamp_range(starts, ends, tid, Tn, s0, s1);
    nkt = (int)((s1 - s0 + TK - 1) / TK);
  }
  int incl = nkt;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(incl, d, 64);
    if (lane >= d) incl += o;
  }
  if (lane == 63) wtot[wave] = incl;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += wtot[w];
  if (tid < E) {
    const int64_t p = (int64_t)(base + incl - nkt) * TK;
    poff[tid] = p;
    // ranges inconsistent with the operands' columns: the expert's dW is zero, as for an
    // expert without tokens
    enk[tid] = p + (int64_t)nkt * TK <= tcap ? nkt : 0;
  }
  __syncthreads();
  int nz = 0;
  if (tid < E && enk[tid] > 0) {
    const int mine = enk[tid];
    int rank = 0;
    for (int x = 0; x < E; ++x) {
      const int o = enk[x];
      rank += (o > mine || (o == mine && x < tid)) ? 1 : 0;
    }
    order[rank] = tid;
  }
  for (int x = 0; x < E; ++x) nz += enk[x] > 0 ? 1 : 0;
  __syncthreads();
  // experts without tokens: every workgroup zeroes its share of their dW.  These stores
  // come before any operand DMA, so the in-order waits of the walk cover them.
  if (nz < E) {
    const int64_t gid = (int64_t)blockIdx.x * kThreads + tid, gstride = (int64_t)gridDim.x * kThreads;
    for (int e = 0; e < E; ++e) {
      if (enk[e] != 0) continue;  // uniform
      for (int64_t idx = gid; idx < M * N; idx += gstride) {
        const int64_t rr = idx / N, cc = idx - rr * N;
        const int64_t off = (int64_t)e * sce + rr * ldc + cc;
        if (c_dtype == CIN_DT_F32)
          static_cast<float*>(C)[off] = 0.0f;
        else
          static_cast<uint16_t*>(C)[off] = 0;
      }
    }
  }
  WgradSrc src;
  src.A = A; src.sa = sa; src.B = B; src.sb = sb; src.C = static_cast<uint8_t*>(C);
  src.lda = lda; src.ssam = ssam; src.ssak = ssak; src.ldb = ldb; src.ssbm = ssbm; src.ldc = ldc; src.sce = sce;
  src.M = M; src.N = N; src.es = c_dtype == CIN_DT_F32 ? 4 : 2;
  src.tiles_m = tiles_m; src.tiles_n = tiles_n; src.G = gridDim.x;
  src.total = (uint32_t)nz * tiles_m * tiles_n;
  src.order = order; src.enk = enk; src.poff = poff;
  run_tiles<EPI, WgradSrc, true>(src, lda, ssam, ssak, ldb, 1, ssbm, 0, c_dtype, ldc);
}

}  // namespace pers

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Compute units of the current device (the persistent grid runs one workgroup per CU),
// looked up once per device.
// The persistent kernels' epilogue for this C (pers::kEpi*); sce is the wgrad's expert
// stride in elements (0 elsewhere).
int pers_epi(int c_dtype, const void* C, int64_t ldc, int64_t sce) {
  const uintptr_t a = (uintptr_t)C;
  if (c_dtype == CIN_DT_F32)
    return (a & 15) == 0 && ldc % 4 == 0 && sce % 4 == 0 ? pers::kEpiCounted32 : pers::kEpiDirect;
  if ((a & 15) == 0 && ldc % 8 == 0 && sce % 8 == 0) return pers::kEpiCounted16x4;
  return (a & 7) == 0 && ldc % 4 == 0 && sce % 4 == 0 ? pers::kEpiCounted16 : pers::kEpiDirect;
}

int device_cus() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// The 256 x 256 kernels address a tile's operands by 32-bit offsets from its first row
// (DMA descriptors): 255 rows of A and B plus a K span of `klen` bytes, and 255 rows of
// A-scales plus klen / 128 K blocks of them.  Shapes past that take the 128 x 128 kernels,
// which use 64-bit addresses.
bool big_offsets_fit(int64_t lda, int64_t ldb, int64_t klen, int64_t ssam, int64_t ssak) {
  const int64_t lim = (int64_t)1 << 32;
  const int64_t nkb = klen / 128 > 0 ? klen / 128 : 1;
  return 255 * lda + klen < lim && 255 * ldb + klen < lim && (255 * ssam + (nkb - 1) * ssak + 1) * 4 < lim;
}

}  // namespace

namespace {
// C[m, 0 .. w) = 0 for m < rows, in 16-bit words, rows `ld` words apart (grid-stride).
__global__ void k_zero_rows16(uint16_t* __restrict__ c, int64_t rows, int64_t w, int64_t ld) {
  const int64_t n = rows * w;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    c[(i / w) * ld + i % w] = 0;
}
}  // namespace

extern "C" {

int cin_gemm_fp8_bs(const uint8_t* A, int64_t lda, const float* sa, int64_t ssam, int64_t ssak,
                    const uint8_t* B, int64_t ldb, const float* sb, int64_t ssbn, int64_t ssbk,
                    int64_t M, int64_t N, int64_t K, void* C, int c_dtype, int64_t ldc,
                    void* stream) {
  CIN_CHECK_ARG(c_dtype == CIN_DT_BF16 || c_dtype == CIN_DT_F16 || c_dtype == CIN_DT_F32,
                "gemm_fp8_bs: C dtype must be bf16, fp16 or fp32");
  CIN_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "gemm_fp8_bs: negative shape");
  if (M == 0 || N == 0) return CIN_OK;
  CIN_CHECK_ARG(C && ldc >= N, "gemm_fp8_bs: bad C");
  CIN_CHECK_ARG(A && B && sa && sb, "gemm_fp8_bs: null pointer");
  CIN_CHECK_ARG(K % 16 == 0, "gemm_fp8_bs: K=%lld must be a multiple of 16", (long long)K);
  CIN_CHECK_ARG(lda >= K && ldb >= K && lda % 16 == 0 && ldb % 16 == 0 && aligned16(A) && aligned16(B),
                "gemm_fp8_bs: A/B rows must be 16-byte aligned and K-contiguous");
  CIN_CHECK_ARG(cdiv(M, BM) * cdiv(N, BN) < ((int64_t)1 << 31), "gemm_fp8_bs: grid too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (K == 0) {
    // empty reduction: C = 0 (same as the reference's zero-initialised accumulator), by a
    // kernel rather than a memset node, so the call can be captured in a graph
    const int64_t es = c_dtype == CIN_DT_F32 ? 4 : 2;
    const int64_t words = M * N * es / 2;
    const unsigned grid = (unsigned)(cdiv(words, 256) < 65536 ? cdiv(words, 256) : 65536);
    hipLaunchKernelGGL(k_zero_rows16, grid, 256, 0, s, static_cast<uint16_t*>(C), M, N * es / 2, ldc * es / 2);
    return cin_check_launch("gemm_fp8_bs");
  }
  if (K % big::TK == 0 && M >= big::TM && N >= big::TN && N % 128 == 0 && big_offsets_fit(lda, ldb, K, ssam, ssak)) {
    const uint32_t tm = (uint32_t)cdiv(M, big::TM), tn = (uint32_t)cdiv(N, big::TN);
    const uint32_t ncu = (uint32_t)device_cus();
    if (tm * tn > ncu) {
      // more tiles than CUs: the persistent walk, whose next tile's DMA overlaps this tile's
      // stores (16-bit C: the fixed-count epilogue).  Every output dtype takes it, so the K
      // order of a tile, and with it the fp32 sum, does not depend on the dtype.
#define CIN_LAUNCH_DENSE_PERS(EPI_)                                                                  \
  hipLaunchKernelGGL(pers::k_gemm_fp8_bs_pers<EPI_>, ncu, big::kThreads, 0, s, A, lda, sa, ssam, ssak, B, \
                     ldb, sb, ssbn, ssbk, M, N, K, C, c_dtype, ldc, tm, tn)
      const int epi = pers_epi(c_dtype, C, ldc, 0);
      if (epi == pers::kEpiCounted16x4)
        CIN_LAUNCH_DENSE_PERS(pers::kEpiCounted16x4);
      else if (epi == pers::kEpiCounted16)
        CIN_LAUNCH_DENSE_PERS(pers::kEpiCounted16);
      else if (epi == pers::kEpiCounted32)
        CIN_LAUNCH_DENSE_PERS(pers::kEpiCounted32);
      else
        CIN_LAUNCH_DENSE_PERS(pers::kEpiDirect);
#undef CIN_LAUNCH_DENSE_PERS
      return cin_check_launch("gemm_fp8_bs");
    }
    hipLaunchKernelGGL(big::k_gemm_fp8_bs_256, tm * tn, big::kThreads, 0, s, A, lda, sa, ssam,
                       ssak, B, ldb, sb, ssbn, ssbk, M, N, K, C, c_dtype, ldc, tm, tn);
    return cin_check_launch("gemm_fp8_bs");
  }
  const uint32_t ntn = (uint32_t)cdiv(N, BN);
  const unsigned grid = (unsigned)(cdiv(M, BM) * ntn);
  hipLaunchKernelGGL(k_gemm_fp8_bs, grid, kThreads, 0, s, A, lda, sa, ssam, ssak, B, ldb, sb, ssbn,
                     ssbk, M, N, K, C, c_dtype, ldc, ntn);
  return cin_check_launch("gemm_fp8_bs");
}

int cin_grouped_gemm_fp8(const uint8_t* A, int64_t lda, const float* sa, int64_t ssam,
                         int64_t ssak, const uint8_t* B, int64_t sbe, int64_t ldb, const float* sb,
                         int64_t ssbe, int64_t ssbn, int64_t ssbk, const int64_t* starts,
                         const int64_t* ends, int64_t E, int64_t T, int64_t N, int64_t K, void* C,
                         int c_dtype, int64_t ldc, void* stream) {
  CIN_CHECK_ARG(c_dtype == CIN_DT_BF16 || c_dtype == CIN_DT_F16 || c_dtype == CIN_DT_F32,
                "grouped_gemm_fp8: C dtype must be bf16, fp16 or fp32");
  CIN_CHECK_ARG(E >= 0 && T >= 0 && N >= 0 && K >= 0, "grouped_gemm_fp8: negative shape");
  if (E == 0 || T == 0 || N == 0) return CIN_OK;
  CIN_CHECK_ARG(A && B && sa && sb && starts && ends && C, "grouped_gemm_fp8: null pointer");
  CIN_CHECK_ARG(K > 0 && K % 16 == 0, "grouped_gemm_fp8: K=%lld must be a positive multiple of 16",
                (long long)K);
  CIN_CHECK_ARG(lda >= K && ldb >= K && lda % 16 == 0 && ldb % 16 == 0 && sbe % 16 == 0 &&
                    aligned16(A) && aligned16(B),
                "grouped_gemm_fp8: A/B rows must be 16-byte aligned and K-contiguous");
  CIN_CHECK_ARG(ldc >= N, "grouped_gemm_fp8: bad C stride");
  if (K % big::TK == 0 && T >= big::TM && N >= big::TN && N % 128 == 0 && big_offsets_fit(lda, ldb, K, ssam, ssak)) {
    const int64_t mt = cdiv(T, big::TM) + E;
    const uint32_t tn = (uint32_t)cdiv(N, big::TN);
    CIN_CHECK_ARG(mt * tn < ((int64_t)1 << 31), "grouped_gemm_fp8: grid too large");
    if (E <= pers::kMaxExpertsLds) {
      const int64_t ncu = device_cus();
      const unsigned grid = (unsigned)(mt * tn < ncu ? mt * tn : ncu);
#define CIN_LAUNCH_GROUPED_PERS(EPI_)                                                                \
  hipLaunchKernelGGL(pers::k_grouped_gemm_fp8_pers<EPI_>, grid, big::kThreads, 0,                      \
                     static_cast<hipStream_t>(stream), A, lda, sa, ssam, ssak, B, sbe, ldb, sb, ssbe, ssbn, \
                     ssbk, starts, ends, (int)E, T, N, K, C, c_dtype, ldc, tn)
      const int epi = pers_epi(c_dtype, C, ldc, 0);
      if (epi == pers::kEpiCounted16x4)
        CIN_LAUNCH_GROUPED_PERS(pers::kEpiCounted16x4);
      else if (epi == pers::kEpiCounted16)
        CIN_LAUNCH_GROUPED_PERS(pers::kEpiCounted16);
      else if (epi == pers::kEpiCounted32)
        CIN_LAUNCH_GROUPED_PERS(pers::kEpiCounted32);
      else
        CIN_LAUNCH_GROUPED_PERS(pers::kEpiDirect);
#undef CIN_LAUNCH_GROUPED_PERS
      return cin_check_launch("grouped_gemm_fp8");
    }
    hipLaunchKernelGGL(big::k_grouped_gemm_fp8_256, (unsigned)(mt * tn), big::kThreads, 0,
                       static_cast<hipStream_t>(stream), A, lda, sa, ssam, ssak, B, sbe, ldb, sb,
                       ssbe, ssbn, ssbk, starts, ends, E, T, N, K, C, c_dtype, ldc, tn,
                       (uint32_t)mt);
    return cin_check_launch("grouped_gemm_fp8");
  }
  const int64_t max_tiles = cdiv(T, BM) + E;
  const uint32_t ntn = (uint32_t)cdiv(N, BN);
  CIN_CHECK_ARG(max_tiles * ntn < ((int64_t)1 << 31), "grouped_gemm_fp8: grid too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = (unsigned)(max_tiles * ntn);
  hipLaunchKernelGGL(k_grouped_gemm_fp8, grid, kThreads, 0, s, A, lda, sa, ssam, ssak, B, sbe, ldb,
                     sb, ssbe, ssbn, ssbk, starts, ends, E, T, N, K, C, c_dtype, ldc, ntn);
  return cin_check_launch("grouped_gemm_fp8");
}

int cin_grouped_gemm_fp8_wgrad(const uint8_t* A, int64_t lda, const float* sa, int64_t ssam,
                               int64_t ssak, const uint8_t* B, int64_t ldb, const float* sb, int64_t ssbm,
                               const int64_t* starts, const int64_t* ends, int64_t E, int64_t T,
                               int64_t tcap, int64_t N, int64_t K, void* C, int c_dtype, int64_t ldc,
                               int64_t sce, void* stream) {
  CIN_CHECK_ARG(c_dtype == CIN_DT_BF16 || c_dtype == CIN_DT_F16 || c_dtype == CIN_DT_F32,
                "grouped_wgrad_fp8: C dtype must be bf16, fp16 or fp32");
  CIN_CHECK_ARG(E >= 0 && T >= 0 && N >= 0 && K >= 0, "grouped_wgrad_fp8: negative shape");
  if (E == 0 || N == 0 || K == 0) return CIN_OK;
  CIN_CHECK_ARG(A && B && sa && sb && starts && ends && C, "grouped_wgrad_fp8: null pointer");
  CIN_CHECK_ARG(N >= big::TM && K >= big::TN && K % 128 == 0,
                "grouped_wgrad_fp8: needs N >= 256, K >= 256 and K %% 128 == 0 (N=%lld, K=%lld)",
                (long long)N, (long long)K);
  CIN_CHECK_ARG(lda % 16 == 0 && ldb % 16 == 0 && aligned16(A) && aligned16(B),
                "grouped_wgrad_fp8: A/B rows must be 16-byte aligned");
  // A's scales [N, tcap / 128]: row-major (ssak == 1) or column-major (ssam == 1)
  const bool sa_ok = (ssak == 1 && ssam >= tcap / 128) || (ssam == 1 && ssak >= N);
  CIN_CHECK_ARG(tcap >= 0 && tcap <= lda && tcap <= ldb && sa_ok,
                "grouped_wgrad_fp8: padded capacity exceeds the operand rows, or A-scale strides overlap");
  CIN_CHECK_ARG(ldc >= K && sce >= N * ldc, "grouped_wgrad_fp8: bad C strides");
  CIN_CHECK_ARG(ssbm >= K / 128, "grouped_wgrad_fp8: bad B-scale stride");
  CIN_CHECK_ARG(big_offsets_fit(lda, ldb, tcap, ssam, ssak),
                "grouped_wgrad_fp8: operand rows too long for the 256 x 256 tile's 32-bit offsets");
  const int64_t tm = cdiv(N, big::TM), tn = cdiv(K, big::TN);
  CIN_CHECK_ARG(E * tm * tn < ((int64_t)1 << 31), "grouped_wgrad_fp8: grid too large");
  const uint32_t ntot = (uint32_t)(E * tm * tn);
  if (E <= pers::kMaxWgradExperts) {
    // one workgroup per CU on the persistent walk; the counted epilogues need every expert's
    // dW aligned as the first one (sce a multiple of 4 elements)
    const unsigned ncu = (unsigned)device_cus();
#define CIN_LAUNCH_WGRAD_PERS(EPI_)                                                                   \
  hipLaunchKernelGGL(pers::k_grouped_wgrad_fp8_pers<EPI_>, ncu, big::kThreads, 0,                       \
                     static_cast<hipStream_t>(stream), A, lda, sa, ssam, ssak, B, ldb, sb, ssbm, starts,   \
                     ends, (int)E, T, tcap, N, K, C, c_dtype, ldc, sce, (uint32_t)tm, (uint32_t)tn)
    const int epi = pers_epi(c_dtype, C, ldc, sce);
    if (epi == pers::kEpiCounted16x4)
      CIN_LAUNCH_WGRAD_PERS(pers::kEpiCounted16x4);
    else if (epi == pers::kEpiCounted16)
      CIN_LAUNCH_WGRAD_PERS(pers::kEpiCounted16);
    else if (epi == pers::kEpiCounted32)
      CIN_LAUNCH_WGRAD_PERS(pers::kEpiCounted32);
    else
      CIN_LAUNCH_WGRAD_PERS(pers::kEpiDirect);
#undef CIN_LAUNCH_WGRAD_PERS
    return cin_check_launch("grouped_wgrad_fp8");
  }
  hipLaunchKernelGGL(big::k_grouped_wgrad_fp8_256, ntot, big::kThreads, 0,
                     static_cast<hipStream_t>(stream), A, lda, sa, ssam, ssak, B, ldb, sb, ssbm, starts,
                     ends, T, tcap, N, K, C, c_dtype, ldc, sce, (uint32_t)tm, (uint32_t)tn, ntot);
  return cin_check_launch("grouped_wgrad_fp8");
}

}  // extern "C"
