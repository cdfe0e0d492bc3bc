// FP8 e4m3 quantizers, dequantizer, dual (row + transposed) quantizer, row->block
// re-quantizer and byte transpose for gfx950.  All arithmetic follows the
// reference quantizers (src/kernels.py:19-132) as restated in cin_common.h.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cin_common.h"
#include "cin_grouped.h"
#include "cin_runtime.h"

using namespace cin;

namespace {

constexpr int kThreads = 256;

inline int elem_size(int dt) { return dt == CIN_DT_F32 ? 4 : 2; }
inline bool valid_dtype(int dt) { return dt == CIN_DT_BF16 || dt == CIN_DT_F32 || dt == CIN_DT_F16; }
inline bool aligned(const void* p, int a) { return ((uintptr_t)p % (uintptr_t)a) == 0; }

inline unsigned grid_for(int64_t work_items, int64_t per_block, int64_t cap) {
  int64_t g = cdiv(work_items, per_block);
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (unsigned)g;
}

// ---------------------------------------------------------------------------
// Row-wise 1x128, contiguous rows: each 16-lane DPP row owns one 128-element
// tile (8 elements per lane, one 16-byte load for bf16/fp16, two for fp32).
// A group walks tiles t, t + G, t + 2G, ... with U tiles loaded before use so
// several loads are in flight per lane.
// ---------------------------------------------------------------------------
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int DT>
struct Vec8 {
  float v[8];
};

template <int DT>
__device__ inline void load8(const void* base, int64_t off, int64_t ncols, Vec8<DT>& o) {
  // off: element offset of the lane's first element; ncols: valid elements (<= 8)
  if (ncols >= 8) {
    if constexpr (DT == CIN_DT_F32) {
      const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(base) + off);
      f32x4 a = __builtin_nontemporal_load(p);
      f32x4 b = __builtin_nontemporal_load(p + 1);
      o.v[0] = a[0]; o.v[1] = a[1]; o.v[2] = a[2]; o.v[3] = a[3];
      o.v[4] = b[0]; o.v[5] = b[1]; o.v[6] = b[2]; o.v[7] = b[3];
    } else {
      const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + off);
      u32x4 w = __builtin_nontemporal_load(p);
      uint32_t ws[4] = {w[0], w[1], w[2], w[3]};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (DT == CIN_DT_BF16) {
          o.v[2 * i] = bf16_lo(ws[i]);
          o.v[2 * i + 1] = bf16_hi(ws[i]);
        } else {
          _Float16 h0, h1;
          uint16_t b0 = (uint16_t)(ws[i] & 0xffffu), b1 = (uint16_t)(ws[i] >> 16);
          __builtin_memcpy(&h0, &b0, 2);
          __builtin_memcpy(&h1, &b1, 2);
          o.v[2 * i] = (float)h0;
          o.v[2 * i + 1] = (float)h1;
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) o.v[i] = (i < ncols) ? load_elem(base, DT, off + i) : 0.0f;
  }
}

// Max over the 8 lanes of a DPP half-row (lanes 8h..8h+7), maxnum semantics.
__device__ inline float row8_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));  // quad [1,0,3,2]
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));  // quad [2,3,0,1]
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false))); // row_half_mirror
  return v;
}

// Quantize NV (multiple of 4) values with scale s / reciprocal r into packed codes.
// STEPS = correction steps of div_by_scale (1 for bf16/fp16 tiles, 2 for fp32).
template <int NV, int STEPS>
__device__ inline void quant_vals(const float (&v)[NV], float s, float r, uint32_t (&out)[NV / 4]) {
  float y[NV];
  if (s < __builtin_inff()) {
#pragma unroll
    for (int i = 0; i < NV; ++i) y[i] = div_by_scale<STEPS>(v[i], s, r);
  } else {
    // infinite amax: x / inf is a signed zero, inf / inf NaN
#pragma unroll
    for (int i = 0; i < NV; ++i) y[i] = v[i] / s;
  }
#pragma unroll
  for (int i = 0; i < NV / 4; ++i)
    out[i] = cvt4_e4m3(clamp448(y[4 * i]), clamp448(y[4 * i + 1]), clamp448(y[4 * i + 2]),
                       clamp448(y[4 * i + 3]));
}

// Row-wise 1x128 with contiguous rows: LANES lanes (8 or 16, a DPP half-row or
// row) own one tile.  Each lane loads NC 16-byte chunks, chunk c of lane i sitting at
// tile chunk c * LANES + i so every load instruction reads whole 16*LANES-byte runs.
// A group walks tiles t, t + G, ... keeping U tiles in flight; (row, tile) advance
// incrementally instead of by division.
template <int DT, int LANES, int U, bool FULL>
__global__ __launch_bounds__(kThreads) void k_rowwise128(const void* __restrict__ x, int64_t N,
                                                         int64_t sxm, int round_scale,
                                                         uint8_t* __restrict__ q, int64_t sqm,
                                                         float* __restrict__ sc, int64_t ssm,
                                                         uint32_t nb, uint32_t ntiles) {
  constexpr int ES = DT == CIN_DT_F32 ? 4 : 2;  // input element bytes
  constexpr int EPC = 16 / ES;                   // elements per 16-byte chunk
  constexpr int NC = 128 / (LANES * EPC);        // chunks per lane
  constexpr int EPL = NC * EPC;                  // elements per lane
  static_assert(NC >= 1 && EPL % 4 == 0, "tile split");
  const uint32_t li = threadIdx.x & (LANES - 1);
  const uint32_t G = (gridDim.x * kThreads) / LANES;
  const uint32_t g0 = (blockIdx.x * kThreads + threadIdx.x) / LANES;
  const float floor_v = amax_floor(DT);
  const bool rs = round_scale != 0;
  uint32_t row = g0 / nb, cb = g0 - row * nb;
  const uint32_t drow = G / nb, dcb = G - drow * nb;
  for (uint32_t tb = g0; tb < ntiles; tb += G * U) {
    float v[U][EPL];
    uint32_t rows[U], cbs[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      rows[u] = row;
      cbs[u] = cb;
      const bool live = tb + (uint32_t)u * G < ntiles;
      const int64_t base = (int64_t)row * sxm + (int64_t)cb * 128;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int64_t e0 = (int64_t)(c * LANES + li) * EPC;  // element offset in the tile
        const int64_t col = (int64_t)cb * 128 + e0;
        int64_t nv = live ? N - col : 0;
        nv = nv < 0 ? 0 : (nv > EPC ? EPC : nv);
        // FULL only drops the column check: a tile past ntiles (u > 0 on the last
        // iteration) has nv == 0 and loads nothing.
        if ((FULL && live) || nv == EPC) {
          if constexpr (DT == CIN_DT_F32) {
            const f32x4 w = __builtin_nontemporal_load(
                reinterpret_cast<const f32x4*>(static_cast<const float*>(x) + base + e0));
#pragma unroll
            for (int e = 0; e < 4; ++e) v[u][c * 4 + e] = w[e];
          } else {
            const u32x4 w = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(x) + base + e0));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if constexpr (DT == CIN_DT_BF16) {
                v[u][c * 8 + 2 * e] = bf16_lo(w[e]);
                v[u][c * 8 + 2 * e + 1] = bf16_hi(w[e]);
              } else {
                _Float16 h0, h1;
                const uint16_t b0 = (uint16_t)(w[e] & 0xffffu), b1 = (uint16_t)(w[e] >> 16);
                __builtin_memcpy(&h0, &b0, 2);
                __builtin_memcpy(&h1, &b1, 2);
                v[u][c * 8 + 2 * e] = (float)h0;
                v[u][c * 8 + 2 * e + 1] = (float)h1;
              }
            }
          }
        } else {
#pragma unroll
          for (int e = 0; e < EPC; ++e)
            v[u][c * EPC + e] = (e < nv) ? load_elem(x, DT, base + e0 + e) : 0.0f;
        }
      }
      cb += dcb;
      row += drow;
      if (cb >= nb) {
        cb -= nb;
        ++row;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (tb + (uint32_t)u * G >= ntiles) break;  // uniform across the tile's lanes
      float a = 0.0f;
#pragma unroll
      for (int i = 0; i < EPL; ++i) a = fmaxf(a, fabsf(v[u][i]));
      a = LANES == 16 ? row16_max(a) : row8_max(a);
      a = fmaxf(a, floor_v);
      const float s = compute_scale(a, rs);
      uint32_t codes[EPL / 4];
      quant_vals<EPL, kDivSteps<DT>>(v[u], s, 1.0f / s, codes);
      uint8_t* qrow = q + (int64_t)rows[u] * sqm + (int64_t)cbs[u] * 128;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int64_t e0 = (int64_t)(c * LANES + li) * EPC;
        const int64_t col = (int64_t)cbs[u] * 128 + e0;
        if (FULL || col + EPC <= N) {
          if constexpr (EPC == 8)
            *reinterpret_cast<uint2*>(qrow + e0) = make_uint2(codes[2 * c], codes[2 * c + 1]);
          else
            *reinterpret_cast<uint32_t*>(qrow + e0) = codes[c];
        } else {
          for (int e = 0; e < EPC; ++e)
            if (col + e < N)
              qrow[e0 + e] = (uint8_t)((codes[(c * EPC + e) >> 2] >> (8 * (e & 3))) & 0xffu);
        }
      }
      if (li == 0) sc[(int64_t)rows[u] * ssm + cbs[u]] = s;
    }
  }
}

template <int LANES, int U, bool FULL>
void launch_rowwise128_t(const void* x, int dt, int64_t N, int64_t sxm, int rs, uint8_t* q,
                         int64_t sqm, float* sc, int64_t ssm, uint32_t nb, uint32_t ntiles,
                         unsigned grid, hipStream_t st) {
  if (dt == CIN_DT_BF16)
    hipLaunchKernelGGL((k_rowwise128<CIN_DT_BF16, LANES, U, FULL>), grid, kThreads, 0, st, x, N,
                       sxm, rs, q, sqm, sc, ssm, nb, ntiles);
  else if (dt == CIN_DT_F16)
    hipLaunchKernelGGL((k_rowwise128<CIN_DT_F16, LANES, U, FULL>), grid, kThreads, 0, st, x, N,
                       sxm, rs, q, sqm, sc, ssm, nb, ntiles);
  else
    hipLaunchKernelGGL((k_rowwise128<CIN_DT_F32, LANES, U, FULL>), grid, kThreads, 0, st, x, N,
                       sxm, rs, q, sqm, sc, ssm, nb, ntiles);
}

template <int LANES, int U>
void launch_rowwise128(const void* x, int dt, int64_t M, int64_t N, int64_t sxm, int rs,
                       uint8_t* q, int64_t sqm, float* sc, int64_t ssm, int64_t nb, int gridcap,
                       hipStream_t st) {
  const uint32_t ntiles = (uint32_t)(M * nb);
  const unsigned grid = grid_for(ntiles, (kThreads / LANES) * U, gridcap);
  if (N % 128 == 0)
    launch_rowwise128_t<LANES, U, true>(x, dt, N, sxm, rs, q, sqm, sc, ssm, (uint32_t)nb, ntiles, grid, st);
  else
    launch_rowwise128_t<LANES, U, false>(x, dt, N, sxm, rs, q, sqm, sc, ssm, (uint32_t)nb, ntiles, grid, st);
}

// Generic row-wise: one wave per (row, tile), any block size / strides / dtype.
__global__ __launch_bounds__(kThreads) void k_rowwise_generic(const void* __restrict__ x, int dt,
                                                              int64_t M, int64_t N, int64_t sxm,
                                                              int64_t sxn, int64_t block,
                                                              int round_scale, uint8_t* q,
                                                              int64_t sqm, float* sc, int64_t ssm,
                                                              int64_t nb) {
  const int lane = threadIdx.x & 63;
  const int64_t w = ((int64_t)blockIdx.x * kThreads + threadIdx.x) >> 6;
  const int64_t W = ((int64_t)gridDim.x * kThreads) >> 6;
  const float floor_v = amax_floor(dt);
  for (int64_t t = w; t < M * nb; t += W) {
    const int64_t row = t / nb, cb = t - row * nb;
    const int64_t c0 = cb * block;
    const int64_t c1 = (c0 + block < N) ? c0 + block : N;
    float a = 0.0f;
    for (int64_t c = c0 + lane; c < c1; c += 64) a = fmaxf(a, fabsf(load_elem(x, dt, row * sxm + c * sxn)));
    a = wave_max(a);
    a = fmaxf(a, floor_v);
    const float s = compute_scale(a, round_scale != 0);
    for (int64_t c = c0 + lane; c < c1; c += 64) {
      float y = clamp448(load_elem(x, dt, row * sxm + c * sxn) / s);
      q[row * sqm + c] = (uint8_t)cvt2_e4m3(y, 0.0f);
    }
    if (lane == 0) sc[row * ssm + cb] = s;
  }
}

// ---------------------------------------------------------------------------
// Block-wise generic: one workgroup per (bm x bn) block, two passes (the second
// read hits L2).  Optional transposed code output.
// ---------------------------------------------------------------------------
__device__ inline float block_reduce_max(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < kThreads / 64; ++i) r = fmaxf(r, red[i]);
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(kThreads) void k_blockwise_generic(
    const void* __restrict__ x, int dt, int64_t M, int64_t N, int64_t sxm, int64_t sxn, int64_t bm,
    int64_t bn, int round_scale, uint8_t* q, int64_t sqm, uint8_t* qt, int64_t sqtm, float* sc,
    int64_t ssm, int64_t nbn) {
  __shared__ float red[kThreads / 64];
  const int64_t rb = blockIdx.y, cb = blockIdx.x;
  const int64_t r0 = rb * bm, c0 = cb * bn;
  const int64_t nr = (r0 + bm < M ? bm : M - r0), nc = (c0 + bn < N ? bn : N - c0);
  const int64_t n = nr * nc;
  float a = 0.0f;
  for (int64_t i = threadIdx.x; i < n; i += kThreads) {
    const int64_t r = r0 + i / nc, c = c0 + i % nc;
    a = fmaxf(a, fabsf(load_elem(x, dt, r * sxm + c * sxn)));
  }
  a = block_reduce_max(a, red);
  a = fmaxf(a, amax_floor(dt));
  const float s = compute_scale(a, round_scale != 0);
  for (int64_t i = threadIdx.x; i < n; i += kThreads) {
    const int64_t r = r0 + i / nc, c = c0 + i % nc;
    const float y = clamp448(load_elem(x, dt, r * sxm + c * sxn) / s);
    const uint8_t code = (uint8_t)cvt2_e4m3(y, 0.0f);
    if (q) q[r * sqm + c] = code;
    if (qt) qt[c * sqtm + r] = code;
  }
  if (threadIdx.x == 0) sc[rb * ssm + cb] = s;
}

// Block-wise 128x128 with contiguous rows: the block stays in registers
// (8 rows x 8 columns per thread), one HBM read.  The transposed output goes
// through a padded LDS byte tile so both layouts are written coalesced.
// Transposed 128 x 128 byte tiles live in LDS as [col][row] with 136-byte rows (34
// words): a thread owning 8 consecutive rows of a column writes them as one 8-byte store.
constexpr int kTW = 34;
typedef uint32_t TileT[128][kTW];

__device__ inline void put_col8(TileT& t, int col, int rgrp, uint32_t lo, uint32_t hi) {
  *reinterpret_cast<uint2*>(&t[col][rgrp * 2]) = make_uint2(lo, hi);
}

// Write the tile to dst[(n0 + col) * ld + t0 + row] for its first tw rows and cols < ncols.
__device__ inline void store_tile_t(const TileT& tileT, uint8_t* dst_base, int64_t ld, int64_t n0,
                                    int64_t ncols, int64_t t0, int tw) {
  for (int idx = threadIdx.x; idx < 128 * 8; idx += kThreads) {
    const int tc = idx >> 3, seg = idx & 7;
    const int64_t n = n0 + tc;
    const int m0 = seg * 16;
    if (n >= ncols || m0 >= tw) continue;
    const uint2 w0 = *reinterpret_cast<const uint2*>(&tileT[tc][seg * 4]);
    const uint2 w1 = *reinterpret_cast<const uint2*>(&tileT[tc][seg * 4 + 2]);
    const uint32_t src[4] = {w0.x, w0.y, w1.x, w1.y};
    uint8_t* dst = dst_base + n * ld + t0 + m0;
    if (m0 + 16 <= tw && (((uintptr_t)dst) & 15u) == 0) {
      *reinterpret_cast<uint4*>(dst) = make_uint4(src[0], src[1], src[2], src[3]);
    } else {
      for (int k = 0; k < 16; ++k)
        if (m0 + k < tw) dst[k] = (uint8_t)((src[k >> 2] >> (8 * (k & 3))) & 0xffu);
    }
  }
}

// 4 x 4 byte transpose: rows a, b, c, d (byte k = column k) -> columns (byte k = row k).
__device__ inline void t4x4(uint32_t a, uint32_t b, uint32_t c, uint32_t d, uint32_t (&o)[4]) {
  const uint32_t ab_lo = __builtin_amdgcn_perm(b, a, 0x05010400u);  // a0 b0 a1 b1
  const uint32_t ab_hi = __builtin_amdgcn_perm(b, a, 0x07030602u);  // a2 b2 a3 b3
  const uint32_t cd_lo = __builtin_amdgcn_perm(d, c, 0x05010400u);
  const uint32_t cd_hi = __builtin_amdgcn_perm(d, c, 0x07030602u);
  o[0] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x05040100u);  // a0 b0 c0 d0
  o[1] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x07060302u);
  o[2] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x05040100u);
  o[3] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x07060302u);
}

// rows[i] = 8 codes of row i (2 words) -> cols[j] = 8 codes of column j, in row order.
__device__ inline void t8x8(const uint32_t (&rows)[8][2], uint32_t (&cols)[8][2]) {
#pragma unroll
  for (int hr = 0; hr < 2; ++hr)      // rows 4 hr .. 4 hr + 3
#pragma unroll
    for (int hc = 0; hc < 2; ++hc) {  // columns 4 hc .. 4 hc + 3
      uint32_t o[4];
      t4x4(rows[4 * hr][hc], rows[4 * hr + 1][hc], rows[4 * hr + 2][hc], rows[4 * hr + 3][hc], o);
#pragma unroll
      for (int k = 0; k < 4; ++k) cols[4 * hc + k][hr] = o[k];
    }
}

template <int DT>
__global__ __launch_bounds__(kThreads) void k_blockwise128(const void* __restrict__ x, int64_t M,
                                                           int64_t N, int64_t sxm, int round_scale,
                                                           uint8_t* q, int64_t sqm, uint8_t* qt,
                                                           int64_t sqtm, float* sc, int64_t ssm) {
  __shared__ float red[kThreads / 64];
  __shared__ TileT tileT;  // transposed codes
  // thread (lane16, rg): rows 8 rg .. 8 rg + 7, columns 8 lane16 .. 8 lane16 + 7
  const int64_t rb = blockIdx.y, cb = blockIdx.x;
  const int lane16 = threadIdx.x & 15, rg = threadIdx.x >> 4;
  const int64_t c = cb * 128 + lane16 * 8;
  Vec8<DT> d[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t r = rb * 128 + rg * 8 + i;
    const int64_t nc = (r < M) ? N - c : 0;
    load8<DT>(x, r * sxm + c, nc < 0 ? 0 : (nc > 8 ? 8 : nc), d[i]);
  }
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) a = fmaxf(a, fabsf(d[i].v[j]));
  a = block_reduce_max(a, red);
  a = fmaxf(a, amax_floor(DT));
  const float s = compute_scale(a, round_scale != 0);
  const float rcp = 1.0f / s;
  uint32_t codes[8][2];
#pragma unroll
  for (int i = 0; i < 8; ++i) quant_vals<8, kDivSteps<DT>>(d[i].v, s, rcp, codes[i]);
  if (q) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t r = rb * 128 + rg * 8 + i;
      if (r >= M) continue;
      uint8_t* qp = q + r * sqm + c;
      if (c + 8 <= N) {
        *reinterpret_cast<uint2*>(qp) = make_uint2(codes[i][0], codes[i][1]);
      } else {
        for (int j = 0; j < 8; ++j)
          if (c + j < N) qp[j] = (uint8_t)((codes[i][j >> 2] >> (8 * (j & 3))) & 0xffu);
      }
    }
  }
  if (qt) {
    uint32_t cols[8][2];
    t8x8(codes, cols);
#pragma unroll
    for (int j = 0; j < 8; ++j) put_col8(tileT, lane16 * 8 + j, rg, cols[j][0], cols[j][1]);
    __syncthreads();
    const int64_t left = M - rb * 128;
    store_tile_t(tileT, qt, sqtm, cb * 128, N, rb * 128, (int)(left < 128 ? left : 128));
  }
  if (threadIdx.x == 0) sc[rb * ssm + cb] = s;
}

// ---------------------------------------------------------------------------
// Placement of one 128-row tile of the dual and re-quantization kernels.  Dense: tile rb
// covers rows [128 rb, min(128 rb + 128, M)) and its transposed outputs sit at the same
// columns.  Grouped (MoE backward): the tile is one 128-token chunk of an expert, and its
// transposed outputs sit at the chunk's padded position; the columns past the chunk's
// rows are written as code 0, so a GEMM reducing over the padded axis adds nothing there.
// ---------------------------------------------------------------------------
struct RowTile {
  int64_t r0;  // first input row
  int nr;      // valid rows, 1..128
  int64_t t0;  // first column of the transposed outputs
  int tw;      // transposed columns written: nr (dense) or 128 (padded)
  int64_t tb;  // index of the tile's scale along the transposed axis
};

__device__ inline RowTile dense_tile(int64_t rb, int64_t M) {
  const int64_t left = M - rb * 128;
  const int nr = (int)(left < 128 ? left : 128);
  return RowTile{rb * 128, nr, rb * 128, nr, rb};
}

// Grouped tile for block row `id`; false when `id` is past the last chunk or its padded
// position would not fit in `tcap` columns (the caller's transposed row length).
__device__ inline bool grouped_tile(const int64_t* starts, const int64_t* ends, int64_t E,
                                    int64_t T, int64_t id, int64_t tcap, RowTile& rt) {
  Chunk c;
  if (!find_chunk(starts, ends, E, T, id, c) || c.t0 + 128 > tcap) return false;
  rt = RowTile{c.r0, c.nr, c.t0, 128, c.t0 / 128};
  return true;
}

// ---------------------------------------------------------------------------
// Dual quantization of a gradient tile (reference FP8MatmulFunction.backward,
// src/kernels.py:771-782): 1x128 row tiles of dY and 1x128 row tiles of dY^T (= 128x1
// column tiles of dY) from one read.  The transposed codes are written through an
// LDS tile.
// ---------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ void dual_tile(const void* __restrict__ x, int64_t N, int64_t sxm,
                                          int round_scale, uint8_t* q, int64_t sqm, float* s,
                                          int64_t ssm, uint8_t* qt, int64_t sqtm, float* st,
                                          int64_t sstm, const RowTile rt, int64_t cb) {
  __shared__ float colpart[16][128];
  __shared__ float colscale[128];
  __shared__ TileT tileT;
  // thread (lane16, rg): rows 8 rg .. 8 rg + 7, columns 8 lane16 .. 8 lane16 + 7
  const int lane16 = threadIdx.x & 15, rg = threadIdx.x >> 4;
  const int64_t c = cb * 128 + lane16 * 8;
  const bool rs = round_scale != 0;
  const float floor_v = amax_floor(DT);
  Vec8<DT> d[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int ri = rg * 8 + i;
    const int64_t nc = (ri < rt.nr) ? N - c : 0;
    load8<DT>(x, (rt.r0 + ri) * sxm + c, nc < 0 ? 0 : (nc > 8 ? 8 : nc), d[i]);
  }
  // column partial maxima over this thread's 8 rows
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) a = fmaxf(a, fabsf(d[i].v[j]));
    colpart[rg][lane16 * 8 + j] = a;
  }
  // row tiles: quantize and store
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int ri = rg * 8 + i;
    const int64_t r = rt.r0 + ri;
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) a = fmaxf(a, fabsf(d[i].v[j]));
    a = row16_max(a);
    a = fmaxf(a, floor_v);
    const float sr = compute_scale(a, rs);
    uint32_t c2[2];
    quant_vals<8, kDivSteps<DT>>(d[i].v, sr, 1.0f / sr, c2);
    const uint32_t lo = c2[0], hi = c2[1];
    if (ri < rt.nr) {
      uint8_t* qp = q + r * sqm + c;
      if (c + 8 <= N) {
        *reinterpret_cast<uint2*>(qp) = make_uint2(lo, hi);
      } else {
        for (int j = 0; j < 8; ++j)
          if (c + j < N) qp[j] = (uint8_t)(((j < 4 ? lo : hi) >> (8 * (j & 3))) & 0xffu);
      }
      if (lane16 == 0) s[r * ssm + cb] = sr;
    }
  }
  __syncthreads();
  if (threadIdx.x < 128) {
    float a = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) a = fmaxf(a, colpart[k][threadIdx.x]);
    a = fmaxf(a, floor_v);
    const float sc = compute_scale(a, rs);
    colscale[threadIdx.x] = sc;
    const int64_t n = cb * 128 + threadIdx.x;
    if (n < N) st[n * sstm + rt.tb] = sc;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float sc = colscale[lane16 * 8 + j];
    float col[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) col[i] = d[i].v[j];
    uint32_t c2[2];
    quant_vals<8, kDivSteps<DT>>(col, sc, 1.0f / sc, c2);  // rows 8 rg .. 8 rg + 7, in order
    put_col8(tileT, lane16 * 8 + j, rg, c2[0], c2[1]);
  }
  __syncthreads();
  store_tile_t(tileT, qt, sqtm, cb * 128, N, rt.t0, rt.tw);
}

template <int DT>
__global__ __launch_bounds__(kThreads) void k_dual128(const void* __restrict__ x, int64_t M,
                                                      int64_t N, int64_t sxm, int round_scale,
                                                      uint8_t* q, int64_t sqm, float* s,
                                                      int64_t ssm, uint8_t* qt, int64_t sqtm,
                                                      float* st, int64_t sstm) {
  dual_tile<DT>(x, N, sxm, round_scale, q, sqm, s, ssm, qt, sqtm, st, sstm,
                dense_tile(blockIdx.y, M), blockIdx.x);
}

// Grouped: block row = one 128-token chunk of an expert (see cin_grouped.h).  Rows
// outside every expert range are not quantized.
template <int DT>
__global__ __launch_bounds__(kThreads) void k_dual128_grouped(
    const void* __restrict__ x, int64_t T, int64_t N, int64_t sxm, int round_scale, uint8_t* q,
    int64_t sqm, float* s, int64_t ssm, uint8_t* qt, int64_t sqtm, float* st, int64_t sstm,
    const int64_t* __restrict__ starts, const int64_t* __restrict__ ends, int64_t E, int64_t tcap) {
  RowTile rt;
  if (!grouped_tile(starts, ends, E, T, blockIdx.y, tcap, rt)) return;  // before any barrier
  dual_tile<DT>(x, N, sxm, round_scale, q, sqm, s, ssm, qt, sqtm, st, sstm, rt, blockIdx.x);
}

// ---------------------------------------------------------------------------
// Re-quantization row(1x128) -> block(128x128).  x = fp32(code) * srow (fp32
// product, as torch's dequantize_fp8_rowwise), then the block quantizer with
// the fp32 floor and round_scale = False.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void requant_tile(const uint8_t* __restrict__ q, int64_t K, int64_t sqm,
                                             const float* __restrict__ srow, int64_t ssm, uint8_t* qb,
                                             int64_t sqbm, uint8_t* qbt, int64_t sqbtm, float* sblk,
                                             int64_t ssbm, const RowTile rt, int64_t cb) {
  __shared__ float red[kThreads / 64];
  __shared__ TileT tileT;
  // thread (lane16, rg): rows 8 rg .. 8 rg + 7, columns 8 lane16 .. 8 lane16 + 7
  const int lane16 = threadIdx.x & 15, rg = threadIdx.x >> 4;
  const int64_t c = cb * 128 + lane16 * 8;
  float v[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int ri = rg * 8 + i;
    const int64_t r = rt.r0 + ri;
    uint32_t w0 = 0, w1 = 0;
    float sr = 0.0f;
    if (ri < rt.nr) {
      sr = srow[r * ssm + cb];
      const uint8_t* qp = q + r * sqm + c;
      if (c + 8 <= K) {
        uint2 w = *reinterpret_cast<const uint2*>(qp);
        w0 = w.x;
        w1 = w.y;
      } else {
        for (int j = 0; j < 8; ++j)
          if (c + j < K) (j < 4 ? w0 : w1) |= (uint32_t)qp[j] << (8 * (j & 3));
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t code = ((j < 4 ? w0 : w1) >> (8 * (j & 3))) & 0xffu;
      const bool valid = (ri < rt.nr) && (c + j < K);
      v[i][j] = valid ? __fmul_rn(e4m3_to_f32(code), sr) : 0.0f;
    }
  }
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) a = fmaxf(a, fabsf(v[i][j]));
  a = block_reduce_max(a, red);
  a = fmaxf(a, kFloorF32);
  const float s = compute_scale(a, false);
  const float rcp = 1.0f / s;
  uint32_t codes[8][2];
#pragma unroll
  for (int i = 0; i < 8; ++i) quant_vals<8, 2>(v[i], s, rcp, codes[i]);
  if (qb) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int ri = rg * 8 + i;
      if (ri >= rt.nr) continue;
      uint8_t* qp = qb + (rt.r0 + ri) * sqbm + c;
      if (c + 8 <= K) {
        *reinterpret_cast<uint2*>(qp) = make_uint2(codes[i][0], codes[i][1]);
      } else {
        for (int j = 0; j < 8; ++j)
          if (c + j < K) qp[j] = (uint8_t)((codes[i][j >> 2] >> (8 * (j & 3))) & 0xffu);
      }
    }
  }
  if (qbt) {
    uint32_t cols[8][2];
    t8x8(codes, cols);
#pragma unroll
    for (int j = 0; j < 8; ++j) put_col8(tileT, lane16 * 8 + j, rg, cols[j][0], cols[j][1]);
    __syncthreads();
    store_tile_t(tileT, qbt, sqbtm, cb * 128, K, rt.t0, rt.tw);
  }
  if (threadIdx.x == 0) sblk[rt.tb * ssbm + cb] = s;
}

__global__ __launch_bounds__(kThreads) void k_requant128(const uint8_t* __restrict__ q, int64_t M,
                                                         int64_t K, int64_t sqm,
                                                         const float* __restrict__ srow,
                                                         int64_t ssm, uint8_t* qb, int64_t sqbm,
                                                         uint8_t* qbt, int64_t sqbtm, float* sblk,
                                                         int64_t ssbm) {
  requant_tile(q, K, sqm, srow, ssm, qb, sqbm, qbt, sqbtm, sblk, ssbm, dense_tile(blockIdx.y, M),
               blockIdx.x);
}

// Grouped: block row = one 128-token chunk of an expert; block scales are indexed by
// the chunk's padded position, codes by the input row (qb) or the padded column (qbt).
__global__ __launch_bounds__(kThreads) void k_requant128_grouped(
    const uint8_t* __restrict__ q, int64_t T, int64_t K, int64_t sqm, const float* __restrict__ srow,
    int64_t ssm, uint8_t* qb, int64_t sqbm, uint8_t* qbt, int64_t sqbtm, float* sblk, int64_t ssbm,
    const int64_t* __restrict__ starts, const int64_t* __restrict__ ends, int64_t E, int64_t tcap) {
  RowTile rt;
  if (!grouped_tile(starts, ends, E, T, blockIdx.y, tcap, rt)) return;  // before any barrier
  requant_tile(q, K, sqm, srow, ssm, qb, sqbm, qbt, sqbtm, sblk, ssbm, rt, blockIdx.x);
}

// ---------------------------------------------------------------------------
// Dequantization: out = fp32(code) * scale[m / bm, n / bn]  (fp32 product),
// stored as fp32 or as bf16 (round-to-nearest-even).  Thread = 8 columns.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void k_dequant(const uint8_t* __restrict__ q, int64_t M,
                                                      int64_t N, int64_t sqm, int64_t sqn,
                                                      const float* __restrict__ sc, int64_t ssm,
                                                      int64_t ssn, int64_t bm, int64_t bn,
                                                      void* out, int odt, int64_t som) {
  const int64_t nchunk = cdiv(N, 8);
  const int64_t total = M * nchunk;
  for (int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * kThreads) {
    const int64_t m = t / nchunk, c0 = (t - m * nchunk) * 8;
    const float* srow = sc + (m / bm) * ssm;
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t n = c0 + j;
      v[j] = (n < N) ? __fmul_rn(e4m3_to_f32(q[m * sqm + n * sqn]), srow[(n / bn) * ssn]) : 0.0f;
    }
    if (odt == CIN_DT_F32) {
      float* o = static_cast<float*>(out) + m * som + c0;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (c0 + j < N) o[j] = v[j];
    } else {
      uint16_t* o = static_cast<uint16_t*>(out) + m * som + c0;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (c0 + j < N) o[j] = (uint16_t)f32_to_bf16_bits(v[j]);
    }
  }
}

// ---------------------------------------------------------------------------
// Byte transpose through a 64x64 LDS tile.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void k_transpose_u8(const uint8_t* __restrict__ src,
                                                           int64_t R, int64_t C, int64_t lds,
                                                           uint8_t* __restrict__ dst,
                                                           int64_t ldd) {
  __shared__ uint8_t tile[64][65];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  for (int i = threadIdx.x; i < 64 * 64; i += kThreads) {
    const int rr = i >> 6, cc = i & 63;
    if (r0 + rr < R && c0 + cc < C) tile[rr][cc] = src[(r0 + rr) * lds + c0 + cc];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += kThreads) {
    const int cc = i >> 6, rr = i & 63;
    if (r0 + rr < R && c0 + cc < C) dst[(c0 + cc) * ldd + r0 + rr] = tile[rr][cc];
  }
}


}  // namespace

extern "C" {

int cin_quant_rowwise(const void* x, int x_dtype, int64_t M, int64_t N, int64_t sxm, int64_t sxn,
                      int64_t block, int round_scale, uint8_t* q, int64_t sqm, float* scales,
                      int64_t ssm, void* stream) {
  CIN_CHECK_ARG(valid_dtype(x_dtype), "quant_rowwise: unsupported x dtype %d", x_dtype);
  CIN_CHECK_ARG(M >= 0 && N >= 0, "quant_rowwise: negative shape");
  CIN_CHECK_ARG(block >= 1 && block <= 1024, "quant_rowwise: block %lld outside [1, 1024]",
                (long long)block);
  if (M == 0 || N == 0) return CIN_OK;
  CIN_CHECK_ARG(x && q && scales, "quant_rowwise: null pointer");
  const int64_t nb = cdiv(N, block);
  CIN_CHECK_ARG(sqm >= N && ssm >= nb, "quant_rowwise: output row stride too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int es = elem_size(x_dtype);
  const bool fast = block == 128 && sxn == 1 && aligned(x, 16) && ((sxm * es) % 16 == 0) &&
                    aligned(q, 8) && (sqm % 8 == 0) && M * nb < (int64_t)1 << 31;
  if (fast) {
    launch_rowwise128<8, 1>(x, x_dtype, M, N, sxm, round_scale, q, sqm, scales, ssm, nb, 16384, s);
  } else {
    const unsigned grid = grid_for(M * nb, kThreads / 64, 65536);
    hipLaunchKernelGGL(k_rowwise_generic, grid, kThreads, 0, s, x, x_dtype, M, N, sxm, sxn, block,
                       round_scale, q, sqm, scales, ssm, nb);
  }
  return cin_check_launch("quant_rowwise");
}

int cin_quant_blockwise(const void* x, int x_dtype, int64_t M, int64_t N, int64_t sxm, int64_t sxn,
                        int64_t bm, int64_t bn, int round_scale, uint8_t* q, int64_t sqm,
                        uint8_t* qt, int64_t sqtm, float* scales, int64_t ssm, void* stream) {
  CIN_CHECK_ARG(valid_dtype(x_dtype), "quant_blockwise: unsupported x dtype %d", x_dtype);
  CIN_CHECK_ARG(M >= 0 && N >= 0, "quant_blockwise: negative shape");
  CIN_CHECK_ARG(bm >= 1 && bn >= 1 && bm <= 1024 && bn <= 1024 && bm * bn <= 65536,
                "quant_blockwise: block %lldx%lld unsupported", (long long)bm, (long long)bn);
  if (M == 0 || N == 0) return CIN_OK;
  CIN_CHECK_ARG(x && scales && (q || qt), "quant_blockwise: null pointer");
  const int64_t nbm = cdiv(M, bm), nbn = cdiv(N, bn);
  CIN_CHECK_ARG(!q || sqm >= N, "quant_blockwise: q row stride too small");
  CIN_CHECK_ARG(!qt || sqtm >= M, "quant_blockwise: qt row stride too small");
  CIN_CHECK_ARG(ssm >= nbn, "quant_blockwise: scale row stride too small");
  CIN_CHECK_ARG(nbm < 65536 && nbn < ((int64_t)1 << 31), "quant_blockwise: grid too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int es = elem_size(x_dtype);
  const bool fast = bm == 128 && bn == 128 && sxn == 1 && aligned(x, 16) &&
                    ((sxm * es) % 16 == 0) && (!q || (aligned(q, 8) && sqm % 8 == 0));
  dim3 grid((unsigned)nbn, (unsigned)nbm);
  if (fast) {
    if (x_dtype == CIN_DT_BF16)
      hipLaunchKernelGGL(k_blockwise128<CIN_DT_BF16>, grid, kThreads, 0, s, x, M, N, sxm,
                         round_scale, q, sqm, qt, sqtm, scales, ssm);
    else if (x_dtype == CIN_DT_F16)
      hipLaunchKernelGGL(k_blockwise128<CIN_DT_F16>, grid, kThreads, 0, s, x, M, N, sxm,
                         round_scale, q, sqm, qt, sqtm, scales, ssm);
    else
      hipLaunchKernelGGL(k_blockwise128<CIN_DT_F32>, grid, kThreads, 0, s, x, M, N, sxm,
                         round_scale, q, sqm, qt, sqtm, scales, ssm);
  } else {
    hipLaunchKernelGGL(k_blockwise_generic, grid, kThreads, 0, s, x, x_dtype, M, N, sxm, sxn, bm,
                       bn, round_scale, q, sqm, qt, sqtm, scales, ssm, nbn);
  }
  return cin_check_launch("quant_blockwise");
}

int cin_dequant(const uint8_t* q, int64_t M, int64_t N, int64_t sqm, int64_t sqn,
                const float* scales, int64_t ssm, int64_t ssn, int64_t bm, int64_t bn, void* out,
                int out_dtype, int64_t som, void* stream) {
  CIN_CHECK_ARG(out_dtype == CIN_DT_BF16 || out_dtype == CIN_DT_F32,
                "dequant: output dtype must be bf16 or fp32");
  CIN_CHECK_ARG(M >= 0 && N >= 0 && bm >= 1 && bn >= 1, "dequant: bad shape or block");
  if (M == 0 || N == 0) return CIN_OK;
  CIN_CHECK_ARG(q && scales && out, "dequant: null pointer");
  CIN_CHECK_ARG(som >= N, "dequant: output row stride too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = grid_for(M * cdiv(N, 8), kThreads, 65536);
  hipLaunchKernelGGL(k_dequant, grid, kThreads, 0, s, q, M, N, sqm, sqn, scales, ssm, ssn, bm, bn,
                     out, out_dtype, som);
  return cin_check_launch("dequant");
}

int cin_quant_dual(const void* dy, int dy_dtype, int64_t M, int64_t N, int64_t sdm, int64_t sdn,
                   int round_scale, uint8_t* q, int64_t sqm, float* s, int64_t ssm, uint8_t* qt,
                   int64_t sqtm, float* st, int64_t sstm, void* stream) {
  CIN_CHECK_ARG(valid_dtype(dy_dtype), "quant_dual: unsupported dtype %d", dy_dtype);
  CIN_CHECK_ARG(M >= 0 && N >= 0, "quant_dual: negative shape");
  if (M == 0 || N == 0) return CIN_OK;
  CIN_CHECK_ARG(dy && q && s && qt && st, "quant_dual: null pointer");
  CIN_CHECK_ARG(sqm >= N && sqtm >= M && ssm >= cdiv(N, 128) && sstm >= cdiv(M, 128),
                "quant_dual: output row stride too small");
  hipStream_t stream_ = static_cast<hipStream_t>(stream);
  const int es = elem_size(dy_dtype);
  const bool fast = sdn == 1 && aligned(dy, 16) && ((sdm * es) % 16 == 0) && aligned(q, 8) &&
                    sqm % 8 == 0 && cdiv(M, 128) < 65536;
  if (fast) {
    dim3 grid((unsigned)cdiv(N, 128), (unsigned)cdiv(M, 128));
    if (dy_dtype == CIN_DT_BF16)
      hipLaunchKernelGGL(k_dual128<CIN_DT_BF16>, grid, kThreads, 0, stream_, dy, M, N, sdm,
                         round_scale, q, sqm, s, ssm, qt, sqtm, st, sstm);
    else if (dy_dtype == CIN_DT_F16)
      hipLaunchKernelGGL(k_dual128<CIN_DT_F16>, grid, kThreads, 0, stream_, dy, M, N, sdm,
                         round_scale, q, sqm, s, ssm, qt, sqtm, st, sstm);
    else
      hipLaunchKernelGGL(k_dual128<CIN_DT_F32>, grid, kThreads, 0, stream_, dy, M, N, sdm,
                         round_scale, q, sqm, s, ssm, qt, sqtm, st, sstm);
    return cin_check_launch("quant_dual");
  }
  // Strided input: two generic row-wise passes (dy, then dy^T through strides).
  int rc = cin_quant_rowwise(dy, dy_dtype, M, N, sdm, sdn, 128, round_scale, q, sqm, s, ssm, stream);
  if (rc != CIN_OK) return rc;
  return cin_quant_rowwise(dy, dy_dtype, N, M, sdn, sdm, 128, round_scale, qt, sqtm, st, sstm,
                           stream);
}

int cin_quant_dual_grouped(const void* dy, int dy_dtype, int64_t T, int64_t N, int64_t sdm,
                           const int64_t* starts, const int64_t* ends, int64_t E, int round_scale,
                           uint8_t* q, int64_t sqm, float* s, int64_t ssm, uint8_t* qt,
                           int64_t sqtm, float* st, int64_t sstm, void* stream) {
  CIN_CHECK_ARG(valid_dtype(dy_dtype), "quant_dual_grouped: unsupported dtype %d", dy_dtype);
  CIN_CHECK_ARG(T >= 0 && N >= 0 && E >= 0, "quant_dual_grouped: negative shape");
  if (T == 0 || N == 0 || E == 0) return CIN_OK;
  CIN_CHECK_ARG(dy && q && s && qt && st && starts && ends, "quant_dual_grouped: null pointer");
  const int es = elem_size(dy_dtype);
  CIN_CHECK_ARG(aligned(dy, 16) && (sdm * es) % 16 == 0 && sdm >= N,
                "quant_dual_grouped: dy rows must be contiguous and 16-byte aligned");
  CIN_CHECK_ARG(aligned(q, 8) && sqm % 8 == 0 && sqm >= N && ssm >= cdiv(N, 128),
                "quant_dual_grouped: bad row-wise outputs");
  CIN_CHECK_ARG(sqtm >= 128 && sstm >= sqtm / 128,
                "quant_dual_grouped: transposed rows must hold the padded token axis");
  CIN_CHECK_ARG(cdiv(T, 128) + E < 65536, "quant_dual_grouped: too many chunks");
  hipStream_t stream_ = static_cast<hipStream_t>(stream);
  dim3 grid((unsigned)cdiv(N, 128), (unsigned)(cdiv(T, 128) + E));
  if (dy_dtype == CIN_DT_BF16)
    hipLaunchKernelGGL(k_dual128_grouped<CIN_DT_BF16>, grid, kThreads, 0, stream_, dy, T, N, sdm,
                       round_scale, q, sqm, s, ssm, qt, sqtm, st, sstm, starts, ends, E, sqtm);
  else if (dy_dtype == CIN_DT_F16)
    hipLaunchKernelGGL(k_dual128_grouped<CIN_DT_F16>, grid, kThreads, 0, stream_, dy, T, N, sdm,
                       round_scale, q, sqm, s, ssm, qt, sqtm, st, sstm, starts, ends, E, sqtm);
  else
    hipLaunchKernelGGL(k_dual128_grouped<CIN_DT_F32>, grid, kThreads, 0, stream_, dy, T, N, sdm,
                       round_scale, q, sqm, s, ssm, qt, sqtm, st, sstm, starts, ends, E, sqtm);
  return cin_check_launch("quant_dual_grouped");
}

int cin_requant_row_to_block_grouped(const uint8_t* q, int64_t T, int64_t K, int64_t sqm,
                                     const float* srow, int64_t ssm, const int64_t* starts,
                                     const int64_t* ends, int64_t E, uint8_t* qbt, int64_t sqbtm,
                                     float* sblk, int64_t ssbm, void* stream) {
  CIN_CHECK_ARG(T >= 0 && K >= 0 && E >= 0, "requant_grouped: negative shape");
  if (T == 0 || K == 0 || E == 0) return CIN_OK;
  CIN_CHECK_ARG(q && srow && qbt && sblk && starts && ends, "requant_grouped: null pointer");
  CIN_CHECK_ARG(aligned(q, 8) && sqm % 8 == 0 && sqm >= K, "requant_grouped: q must be 8-byte aligned rows");
  CIN_CHECK_ARG(sqbtm >= 128 && ssm >= cdiv(K, 128) && ssbm >= cdiv(K, 128),
                "requant_grouped: bad output strides");
  CIN_CHECK_ARG(cdiv(T, 128) + E < 65536, "requant_grouped: too many chunks");
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 grid((unsigned)cdiv(K, 128), (unsigned)(cdiv(T, 128) + E));
  hipLaunchKernelGGL(k_requant128_grouped, grid, kThreads, 0, s, q, T, K, sqm, srow, ssm,
                     (uint8_t*)nullptr, (int64_t)0, qbt, sqbtm, sblk, ssbm, starts, ends, E, sqbtm);
  return cin_check_launch("requant_row_to_block_grouped");
}

int cin_requant_row_to_block(const uint8_t* q, int64_t M, int64_t K, int64_t sqm,
                             const float* srow, int64_t ssm, uint8_t* qb, int64_t sqbm,
                             uint8_t* qbt, int64_t sqbtm, float* sblk, int64_t ssbm,
                             void* stream) {
  CIN_CHECK_ARG(M >= 0 && K >= 0, "requant: negative shape");
  if (M == 0 || K == 0) return CIN_OK;
  CIN_CHECK_ARG(q && srow && sblk && (qb || qbt), "requant: null pointer");
  CIN_CHECK_ARG(aligned(q, 8) && sqm % 8 == 0, "requant: q must be 8-byte aligned rows");
  CIN_CHECK_ARG(!qb || (aligned(qb, 8) && sqbm % 8 == 0 && sqbm >= K),
                "requant: qb must be 8-byte aligned rows");
  CIN_CHECK_ARG(!qbt || sqbtm >= M, "requant: qbt row stride too small");
  CIN_CHECK_ARG(ssm >= cdiv(K, 128) && ssbm >= cdiv(K, 128) && cdiv(M, 128) < 65536,
                "requant: bad scale stride");
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 grid((unsigned)cdiv(K, 128), (unsigned)cdiv(M, 128));
  hipLaunchKernelGGL(k_requant128, grid, kThreads, 0, s, q, M, K, sqm, srow, ssm, qb, sqbm, qbt,
                     sqbtm, sblk, ssbm);
  return cin_check_launch("requant_row_to_block");
}

int cin_transpose_u8(const uint8_t* src, int64_t R, int64_t C, int64_t lds, uint8_t* dst,
                     int64_t ldd, void* stream) {
  CIN_CHECK_ARG(R >= 0 && C >= 0, "transpose_u8: negative shape");
  if (R == 0 || C == 0) return CIN_OK;
  CIN_CHECK_ARG(src && dst && lds >= C && ldd >= R, "transpose_u8: bad pointer or stride");
  CIN_CHECK_ARG(cdiv(R, 64) < 65536, "transpose_u8: too many rows");
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 grid((unsigned)cdiv(C, 64), (unsigned)cdiv(R, 64));
  hipLaunchKernelGGL(k_transpose_u8, grid, kThreads, 0, s, src, R, C, lds, dst, ldd);
  return cin_check_launch("transpose_u8");
}

}  // extern "C"
