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
#include "cin_runtime.h"

using namespace cin;

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

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
        const uint32_t b0 = f32_to_bf16_bits(acc[i][j][0]), b1 = f32_to_bf16_bits(acc[i][j][1]);
        const uint32_t b2 = f32_to_bf16_bits(acc[i][j][2]), b3 = f32_to_bf16_bits(acc[i][j][3]);
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

// Workgroup tile 256 x 256 x 128, 8 waves (2 per SIMD: one wave's MFMAs run while
// the other issues its scale-FMAs), wave tile 128 (m) x 64 (n), two LDS stages.
// Operands are staged global -> VGPR -> LDS: the loads of K block kb+1 are issued at
// the start of block kb and written to the free stage in its second half.  (The
// global_load_lds path moves only ~16 bytes per clock per CU on gfx950, half of what
// the MFMAs consume here.)
constexpr int TM = 256, TN = 256, TK = 128;
constexpr int kThreads = 512;
constexpr int kTileBytes = TM * TK;  // 32 KB per operand per stage

struct __attribute__((aligned(16))) Smem {
  uint8_t a[2][kTileBytes];
  uint8_t b[2][kTileBytes];
  float sa[2][TM];
  float sb[2][2];
};

// 16-byte chunk c of tile row r lives at slot c ^ f(r), f(r) = (r % 8) ^ ((r / 8) % 2):
// the 8 rows a 32-bank LDS serves together, and the 8 same-parity rows a 64-bank LDS
// serves together, all hit distinct banks.
__device__ inline int swz_f(int r) { return (r & 7) ^ ((r >> 3) & 1); }
__device__ inline int swz2(int row, int chunk) { return row * TK + ((chunk ^ swz_f(row)) << 4); }

__device__ inline v8i frag(const uint8_t* lds, int row, int kq) {
  const uint4 lo = *reinterpret_cast<const uint4*>(lds + swz2(row, 2 * kq));
  const uint4 hi = *reinterpret_cast<const uint4*>(lds + swz2(row, 2 * kq + 1));
  v8i v;
  v[0] = (int)lo.x; v[1] = (int)lo.y; v[2] = (int)lo.z; v[3] = (int)lo.w;
  v[4] = (int)hi.x; v[5] = (int)hi.y; v[6] = (int)hi.z; v[7] = (int)hi.w;
  return v;
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
};

__device__ __forceinline__ void tile_body(const Tile& T, int64_t lda, int64_t ssam, int64_t ssak,
                                          int64_t ldb, int64_t ssbn, int64_t ssbk, int64_t K,
                                          int c_dtype, int64_t ldc) {
  __shared__ Smem sm;
  const uint8_t* Ab = T.A;
  const uint8_t* Bb = T.B;
  const float* sab = T.sa;
  const float* sbt = T.sb;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int l16 = lane & 15, kq = lane >> 4;

  // Loads: round i covers tile rows i*64 .. i*64+63; thread tid fetches row
  // i*64 + tid/8, chunk (tid % 8) ^ swz_f(row) and stores it to slot i*512 + tid.
  // Addresses are a wave-uniform base (row round, K block) plus a 32-bit lane offset.
  const int r0 = tid >> 3;
  const uint32_t q16 = (uint32_t)(((tid & 7) ^ swz_f(r0)) * 16);
  const uint32_t offA = (uint32_t)(r0 * lda) + q16;
  const uint32_t offB = (uint32_t)(r0 * ldb) + q16;
  const int64_t stepa = 64 * lda, stepb = 64 * ldb;
  // scales: threads 0-255 fetch the A-scale rows, 256-257 the tile's two B-block scales
  const bool has_s = tid < TM + 2;
  const uint32_t offS = tid < TM ? (uint32_t)(tid * ssam * 4) : (uint32_t)(((tid - TM) & 1) * ssbn * 4);
  const uint8_t* sbase = reinterpret_cast<const uint8_t*>(wave < 4 ? sab : sbt);  // uniform
  const int64_t steps = (wave < 4 ? ssak : ssbk) * 4;
  // staging registers for half a K block: the 4 A chunks, later the 4 B chunks + scale
  uint4 r0v, r1v, r2v, r3v;
  float rs = 0.0f;
#define CIN_LOAD_A(kb)                                                                      \
  do {                                                                                      \
    const uint8_t* base = Ab + (int64_t)(kb) * TK;                                          \
    r0v = *reinterpret_cast<const uint4*>(base + offA);                                     \
    r1v = *reinterpret_cast<const uint4*>(base + stepa + offA);                             \
    r2v = *reinterpret_cast<const uint4*>(base + 2 * stepa + offA);                         \
    r3v = *reinterpret_cast<const uint4*>(base + 3 * stepa + offA);                         \
  } while (0)
#define CIN_LOAD_B(kb)                                                                      \
  do {                                                                                      \
    const uint8_t* base = Bb + (int64_t)(kb) * TK;                                          \
    r0v = *reinterpret_cast<const uint4*>(base + offB);                                     \
    r1v = *reinterpret_cast<const uint4*>(base + stepb + offB);                             \
    r2v = *reinterpret_cast<const uint4*>(base + 2 * stepb + offB);                         \
    r3v = *reinterpret_cast<const uint4*>(base + 3 * stepb + offB);                         \
    if (has_s) rs = *reinterpret_cast<const float*>(sbase + (int64_t)(kb) * steps + offS);  \
  } while (0)
#define CIN_STORE(arr, i, rv, st)                                                           \
  *reinterpret_cast<uint4*>(__builtin_assume_aligned(&sm.arr[st][((i) * kThreads + tid) * 16], 16)) = rv
#define CIN_STORE_S(st)                                                                     \
  do {                                                                                      \
    if (tid < TM) sm.sa[st][tid] = rs;                                                      \
    else if (has_s) sm.sb[st][tid - TM] = rs;                                               \
  } while (0)

  v4f acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  const int nk = (int)(K / TK);
  CIN_LOAD_A(0);
  CIN_STORE(a, 0, r0v, 0);
  CIN_STORE(a, 1, r1v, 0);
  CIN_STORE(a, 2, r2v, 0);
  CIN_STORE(a, 3, r3v, 0);
  CIN_LOAD_B(0);
  CIN_STORE(b, 0, r0v, 0);
  CIN_STORE(b, 1, r1v, 0);
  CIN_STORE(b, 2, r2v, 0);
  CIN_STORE(b, 3, r3v, 0);
  CIN_STORE_S(0);

  const v4f zero = {0.f, 0.f, 0.f, 0.f};
  for (int kb = 0; kb < nk; ++kb) {
    const int st = kb & 1;
    __syncthreads();  // stage st is complete; stage st^1 is no longer read
    const bool more = kb + 1 < nk;
    if (more) CIN_LOAD_A(kb + 1);
    const uint8_t* la = sm.a[st];
    const uint8_t* lb = sm.b[st];
    const float* lsa = sm.sa[st];
    const float sbv = sm.sb[st][wn >> 1];
    v8i bf[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) bf[j] = frag(lb, wn * 64 + j * 16 + l16, kq);
    v8i af[2];
    af[0] = frag(la, wm * 128 + l16, kq);
    float cs[2];
    cs[0] = lsa[wm * 128 + l16] * sbv;
    // 32 steps s = 4 i + j (m-tile i, n-tile j): step s issues MFMA(s) into partial
    // ring slot s % 2, then the 4 scale-FMAs of MFMA(s-1), whose result had one MFMA
    // slot of latency to land.  Empty asm statements pin this order (the MFMA builtins
    // are otherwise free to move, and the compiler would cluster them and hold many
    // partials live).
    v4f p[2];
#pragma unroll
    for (int st8 = 0; st8 < 33; ++st8) {
      const int i = st8 >> 2, j = st8 & 3;
      if (st8 < 32) {
        if (j == 0) {
          // staged loads of the next block: A chunks were loaded at the top and are
          // stored in groups 2-3; then the B chunks + scales, stored in groups 6-7
          if (more) {
            if (i == 2) { CIN_STORE(a, 0, r0v, st ^ 1); CIN_STORE(a, 1, r1v, st ^ 1); }
            if (i == 3) { CIN_STORE(a, 2, r2v, st ^ 1); CIN_STORE(a, 3, r3v, st ^ 1); CIN_LOAD_B(kb + 1); }
            if (i == 6) { CIN_STORE(b, 0, r0v, st ^ 1); CIN_STORE(b, 1, r1v, st ^ 1); }
            if (i == 7) { CIN_STORE(b, 2, r2v, st ^ 1); CIN_STORE(b, 3, r3v, st ^ 1); CIN_STORE_S(st ^ 1); }
          }
        }
        asm volatile("" : "+v"(bf[j]));
        p[st8 & 1] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf[j], af[i & 1], zero, 0, 0, 0, 0, 0, 0);
      }
      if (st8 > 0) {
        const int s1 = st8 - 1, i1 = s1 >> 2, j1 = s1 & 3;
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i1][j1][r] = fmaf(p[s1 & 1][r], cs[i1 & 1], acc[i1][j1][r]);
        asm volatile("" : "+v"(acc[i1][j1]));
      }
      // fragment and scale of m-tile i+1 (its slot's previous user, tile i-1, is done)
      if (st8 < 32 && j == 0 && i + 1 < 8) {
        af[(i + 1) & 1] = frag(la, wm * 128 + (i + 1) * 16 + l16, kq);
        cs[(i + 1) & 1] = lsa[wm * 128 + (i + 1) * 16 + l16] * sbv;
      }
    }
  }
#undef CIN_LOAD_A
#undef CIN_LOAD_B
#undef CIN_STORE
#undef CIN_STORE_S

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
        const uint32_t b0 = f32_to_bf16_bits(acc[i][j][0]), b1 = f32_to_bf16_bits(acc[i][j][1]);
        const uint32_t b2 = f32_to_bf16_bits(acc[i][j][2]), b3 = f32_to_bf16_bits(acc[i][j][3]);
        if ((((uintptr_t)cp) & 7) == 0) {
          *reinterpret_cast<uint2*>(cp) = make_uint2(b0 | (b1 << 16), b2 | (b3 << 16));
        } else {
          cp[0] = (uint16_t)b0; cp[1] = (uint16_t)b1; cp[2] = (uint16_t)b2; cp[3] = (uint16_t)b3;
        }
      }
    }
  }
}

// XCD-aware order: workgroup b runs on XCD b % 8; give each XCD a contiguous run of
// tile ids (n fastest) so its CUs share A row panels and B in their L2.
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
  const uint32_t tm = b / tiles_n, tn = b - tm * tiles_n;
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

}  // namespace big

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

extern "C" {

int cin_gemm_fp8_bs(const uint8_t* A, int64_t lda, const float* sa, int64_t ssam, int64_t ssak,
                    const uint8_t* B, int64_t ldb, const float* sb, int64_t ssbn, int64_t ssbk,
                    int64_t M, int64_t N, int64_t K, void* C, int c_dtype, int64_t ldc,
                    void* stream) {
  CIN_CHECK_ARG(c_dtype == CIN_DT_BF16 || c_dtype == CIN_DT_F32,
                "gemm_fp8_bs: C dtype must be bf16 or fp32");
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
    // empty reduction: C = 0 (same as the reference's zero-initialised accumulator)
    hipError_t e = hipMemset2DAsync(C, ldc * (c_dtype == CIN_DT_F32 ? 4 : 2), 0,
                                    N * (c_dtype == CIN_DT_F32 ? 4 : 2), M, s);
    if (e != hipSuccess) return cin_set_error(CIN_ERR_HIP, "gemm_fp8_bs: %s", hipGetErrorString(e));
    return CIN_OK;
  }
  if (K % big::TK == 0 && M >= big::TM && N >= big::TN && N % 128 == 0) {
    const uint32_t tm = (uint32_t)cdiv(M, big::TM), tn = (uint32_t)cdiv(N, big::TN);
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
  CIN_CHECK_ARG(c_dtype == CIN_DT_BF16 || c_dtype == CIN_DT_F32,
                "grouped_gemm_fp8: C dtype must be bf16 or fp32");
  CIN_CHECK_ARG(E >= 0 && T >= 0 && N >= 0 && K >= 0, "grouped_gemm_fp8: negative shape");
  if (E == 0 || T == 0 || N == 0) return CIN_OK;
  CIN_CHECK_ARG(A && B && sa && sb && starts && ends && C, "grouped_gemm_fp8: null pointer");
  CIN_CHECK_ARG(K > 0 && K % 16 == 0, "grouped_gemm_fp8: K=%lld must be a positive multiple of 16",
                (long long)K);
  CIN_CHECK_ARG(lda >= K && ldb >= K && lda % 16 == 0 && ldb % 16 == 0 && sbe % 16 == 0 &&
                    aligned16(A) && aligned16(B),
                "grouped_gemm_fp8: A/B rows must be 16-byte aligned and K-contiguous");
  CIN_CHECK_ARG(ldc >= N, "grouped_gemm_fp8: bad C stride");
  if (K % big::TK == 0 && T >= big::TM && N >= big::TN && N % 128 == 0) {
    const int64_t mt = cdiv(T, big::TM) + E;
    const uint32_t tn = (uint32_t)cdiv(N, big::TN);
    CIN_CHECK_ARG(mt * tn < ((int64_t)1 << 31), "grouped_gemm_fp8: grid too large");
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

}  // extern "C"
