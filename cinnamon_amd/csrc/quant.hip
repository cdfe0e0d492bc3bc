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
// 128 rows of `rowbytes` bytes span less than 2 GiB: 32-bit buffer offsets reach every
// byte of a 128-row tile.
inline bool tile_fits32(int64_t rowbytes) { return rowbytes >= 0 && rowbytes < ((int64_t)1 << 24); }

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

// Row-wise 1x128 with contiguous rows: LANES lanes (8 or 16, a DPP half-row or
// row) own one tile.  Each lane loads NC 16-byte chunks, chunk c of lane i sitting at
// tile chunk c * LANES + i so every load instruction reads whole 16*LANES-byte runs.
// A group walks tiles t, t + G, ... keeping U tiles in flight; (row, tile) advance
// incrementally instead of by division.  MAP selects the MoE dispatch forms:
//   kMapGather : output row r quantizes input row rowmap[r] / rowdiv (int64 map); a map
//                entry that is negative or past src_rows gives a zero row;
//   kMapScatter: input row t is quantized once and its codes and scale go to the output
//                rows rowmap[t * rowdiv + j] (int32 map), j < rowdiv, that lie in
//                [0, src_rows) (src_rows = output rows here);
//   kMapFirstScale: rows as kMapNone, but only each row's first tile scale is written, to
//                sc[row * ssm] (the DSA indexer uses no other, src/attention.py:296-297);
//   kMapScatterTok: codes as kMapScatter, but each scale is written once, by input row, to
//                sc[t * ssm + cb * ssk] (a token-major table that a second pass spreads
//                over the output rows).
constexpr int kMapNone = 0, kMapGather = 1, kMapScatter = 2, kMapFirstScale = 3, kMapScatterTok = 4;
// The body runs as workgroup `bid` of `nblk` (the kernel's own grid, or a share of a fused
// launch's).
template <int DT, int LANES, int U, bool FULL, int MAP = kMapNone>
__device__ __forceinline__ void rowwise128_body(uint32_t bid, uint32_t nblk, const void* __restrict__ x,
                                                int64_t N, int64_t sxm, int round_scale,
                                                uint8_t* __restrict__ q, int64_t sqm,
                                                float* __restrict__ sc, int64_t ssm, int64_t ssk,
                                                uint32_t nb, uint32_t ntiles,
                                                const void* __restrict__ rowmap,
                                                int64_t rowdiv, int64_t src_rows) {
  constexpr int ES = DT == CIN_DT_F32 ? 4 : 2;  // input element bytes
  constexpr int EPC = 16 / ES;                   // elements per 16-byte chunk
  constexpr int NC = 128 / (LANES * EPC);        // chunks per lane
  constexpr int EPL = NC * EPC;                  // elements per lane
  static_assert(NC >= 1 && EPL % 4 == 0, "tile split");
  const uint32_t li = threadIdx.x & (LANES - 1);
  const uint32_t G = (nblk * kThreads) / LANES;
  const uint32_t g0 = (bid * kThreads + threadIdx.x) / LANES;
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
      bool live = tb + (uint32_t)u * G < ntiles;
      int64_t srow = row;
      if constexpr (MAP == kMapGather) {
        const int64_t m = live ? static_cast<const int64_t*>(rowmap)[row] : -1;
        srow = m >= 0 ? m / rowdiv : -1;
        if (srow < 0 || srow >= src_rows) {
          srow = 0;
          live = false;  // loads nothing: the tile quantizes zeros
        }
      }
      const int64_t base = srow * sxm + (int64_t)cb * 128;
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
      constexpr bool kScat = MAP == kMapScatter || MAP == kMapScatterTok;
      const int nout = kScat ? (int)rowdiv : 1;
      for (int j = 0; j < nout; ++j) {
        int64_t orow = rows[u];
        if constexpr (kScat) {
          orow = static_cast<const int32_t*>(rowmap)[(int64_t)rows[u] * rowdiv + j];
          if (orow < 0 || orow >= src_rows) continue;
        }
        uint8_t* qrow = q + orow * sqm + (int64_t)cbs[u] * 128;
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
        if (li == 0) {
          if constexpr (MAP == kMapFirstScale) {
            if (cbs[u] == 0) sc[orow * ssm] = s;
          } else if constexpr (MAP != kMapScatterTok) {
            sc[orow * ssm + (int64_t)cbs[u] * ssk] = s;
          }
        }
      }
      if constexpr (MAP == kMapScatterTok) {
        if (li == 0) sc[(int64_t)rows[u] * ssm + (int64_t)cbs[u] * ssk] = s;
      }
    }
  }
}

// Row-wise 1 x 128 quantization in units of 8 rows x 8 column blocks, 8 lanes per tile,
// whole column blocks only (N % 128 == 0); scales at sc[r * ssm + c * ssk], row- or
// column-major.  Wave w quantizes rows r0 + w and r0 + 4 + w, its eight 8-lane groups column
// blocks cb0 .. cb0 + 7 (2 KB of one row per wave and tile, as in the row walk); the unit's
// 64 scales go through LDS and one wave stores them as eight runs of 8 consecutive floats
// (32 bytes, whole memory sectors) along whichever index is contiguous.  Against the row
// walk (rowwise128_body, kept for partial column blocks and the MoE forms) on config-2 X
// [8192, 7168] bf16: 31.5 -> 29.8 us with row-major scales; with column-major ones the row
// walk's 4-byte stores land in separate sectors (forward pair 41.9 us, 36.1 here).  Units
// advance along the 8 rows first, so a workgroup's reads stay in the same rows.  Same
// per-tile arithmetic as rowwise128_body, so the same codes and scales.
struct RowCmSmem {
  float s[2][8][8];  // [unit parity][column block][row] of a unit
};
template <int DT>
__device__ __forceinline__ void rowwise128_cm_body(uint32_t bid, uint32_t nblk, const void* __restrict__ x,
                                                   int64_t M, int64_t sxm, int round_scale,
                                                   uint8_t* __restrict__ q, int64_t sqm,
                                                   float* __restrict__ sc, int64_t ssm, int64_t ssk,
                                                   uint32_t nb, RowCmSmem& sm) {
  constexpr int ES = DT == CIN_DT_F32 ? 4 : 2;
  constexpr int EPC = 16 / ES;
  constexpr int NC = 128 / (8 * EPC);
  constexpr int EPL = NC * EPC;
  const uint32_t li = threadIdx.x & 7, g8 = (threadIdx.x >> 3) & 7, w = threadIdx.x >> 6;
  const float floor_v = amax_floor(DT);
  const bool rs = round_scale != 0;
  const uint32_t ncb = (nb + 7) >> 3;
  const uint32_t nunits = (uint32_t)((M + 7) >> 3) * ncb;
  uint32_t par = 0;
  for (uint32_t un = bid; un < nunits; un += nblk, par ^= 1u) {
    const uint32_t rb = un / ncb, cbb = un - rb * ncb;
    const uint32_t cb = cbb * 8 + g8;
    float v[2][EPL];
    int64_t rows[2];
    bool live[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      rows[u] = (int64_t)rb * 8 + w + 4 * u;
      live[u] = rows[u] < M && cb < nb;
      const int64_t base = (live[u] ? rows[u] : 0) * sxm + (int64_t)cb * 128;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int64_t e0 = (int64_t)(c * 8 + li) * EPC;
        if constexpr (DT == CIN_DT_F32) {
          f32x4 wv = {0.f, 0.f, 0.f, 0.f};
          if (live[u]) wv = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(static_cast<const float*>(x) + base + e0));
#pragma unroll
          for (int e = 0; e < 4; ++e) v[u][c * 4 + e] = wv[e];
        } else {
          u32x4 wv = {0u, 0u, 0u, 0u};
          if (live[u]) wv = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(x) + base + e0));
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if constexpr (DT == CIN_DT_BF16) {
              v[u][c * 8 + 2 * e] = bf16_lo(wv[e]);
              v[u][c * 8 + 2 * e + 1] = bf16_hi(wv[e]);
            } else {
              _Float16 h0, h1;
              const uint16_t b0 = (uint16_t)(wv[e] & 0xffffu), b1 = (uint16_t)(wv[e] >> 16);
              __builtin_memcpy(&h0, &b0, 2);
              __builtin_memcpy(&h1, &b1, 2);
              v[u][c * 8 + 2 * e] = (float)h0;
              v[u][c * 8 + 2 * e + 1] = (float)h1;
            }
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      float a = 0.0f;
#pragma unroll
      for (int i = 0; i < EPL; ++i) a = fmaxf(a, fabsf(v[u][i]));
      a = fmaxf(row8_max(a), floor_v);
      const float s = compute_scale(a, rs);
      uint32_t codes[EPL / 4];
      quant_vals<EPL, kDivSteps<DT>>(v[u], s, 1.0f / s, codes);
      if (live[u]) {
        uint8_t* qrow = q + rows[u] * sqm + (int64_t)cb * 128;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int64_t e0 = (int64_t)(c * 8 + li) * EPC;
          if constexpr (EPC == 8)
            *reinterpret_cast<uint2*>(qrow + e0) = make_uint2(codes[2 * c], codes[2 * c + 1]);
          else
            *reinterpret_cast<uint32_t*>(qrow + e0) = codes[c];
        }
      }
      if (li == 0) sm.s[par][g8][w + 4 * u] = s;
    }
    __syncthreads();  // the unit's 64 scales are in LDS (the other parity's are being reused
                      // two units later, after the next barrier)
    if (threadIdx.x < 64) {
      // consecutive threads along the contiguous index (rows if column-major)
      const bool cm = ssm == 1;
      const uint32_t cl = cm ? threadIdx.x >> 3 : threadIdx.x & 7;
      const uint32_t rl = cm ? threadIdx.x & 7 : threadIdx.x >> 3;
      const int64_t r = (int64_t)rb * 8 + rl;
      if (r < M && cbb * 8 + cl < nb) sc[r * ssm + (int64_t)(cbb * 8 + cl) * ssk] = sm.s[par][cl][rl];
    }
  }
}

template <int DT>
__global__ __launch_bounds__(kThreads) void k_rowwise128_cm(const void* __restrict__ x, int64_t M,
                                                            int64_t sxm, int round_scale,
                                                            uint8_t* __restrict__ q, int64_t sqm,
                                                            float* __restrict__ sc, int64_t ssm,
                                                            int64_t ssk, uint32_t nb) {
  __shared__ RowCmSmem sm;
  rowwise128_cm_body<DT>(blockIdx.x, gridDim.x, x, M, sxm, round_scale, q, sqm, sc, ssm, ssk, nb, sm);
}

template <int DT, int LANES, int U, bool FULL, int MAP = kMapNone>
__global__ __launch_bounds__(kThreads) void k_rowwise128(const void* __restrict__ x, int64_t N,
                                                         int64_t sxm, int round_scale,
                                                         uint8_t* __restrict__ q, int64_t sqm,
                                                         float* __restrict__ sc, int64_t ssm,
                                                         int64_t ssk, uint32_t nb, uint32_t ntiles,
                                                         const void* __restrict__ rowmap = nullptr,
                                                         int64_t rowdiv = 1, int64_t src_rows = 0) {
  rowwise128_body<DT, LANES, U, FULL, MAP>(blockIdx.x, gridDim.x, x, N, sxm, round_scale, q, sqm, sc,
                                           ssm, ssk, nb, ntiles, rowmap, rowdiv, src_rows);
}

template <int LANES, int U, bool FULL, int MAP = kMapNone>
void launch_rowwise128_t(const void* x, int dt, int64_t N, int64_t sxm, int rs, uint8_t* q,
                         int64_t sqm, float* sc, int64_t ssm, int64_t ssk, uint32_t nb, uint32_t ntiles,
                         unsigned grid, hipStream_t st, const void* rowmap = nullptr,
                         int64_t rowdiv = 1, int64_t src_rows = 0) {
  if (dt == CIN_DT_BF16)
    hipLaunchKernelGGL((k_rowwise128<CIN_DT_BF16, LANES, U, FULL, MAP>), grid, kThreads, 0, st,
                       x, N, sxm, rs, q, sqm, sc, ssm, ssk, nb, ntiles, rowmap, rowdiv, src_rows);
  else if (dt == CIN_DT_F16)
    hipLaunchKernelGGL((k_rowwise128<CIN_DT_F16, LANES, U, FULL, MAP>), grid, kThreads, 0, st,
                       x, N, sxm, rs, q, sqm, sc, ssm, ssk, nb, ntiles, rowmap, rowdiv, src_rows);
  else
    hipLaunchKernelGGL((k_rowwise128<CIN_DT_F32, LANES, U, FULL, MAP>), grid, kThreads, 0, st,
                       x, N, sxm, rs, q, sqm, sc, ssm, ssk, nb, ntiles, rowmap, rowdiv, src_rows);
}

template <int LANES, int U>
void launch_rowwise128(const void* x, int dt, int64_t M, int64_t N, int64_t sxm, int rs,
                       uint8_t* q, int64_t sqm, float* sc, int64_t ssm, int64_t ssk, int64_t nb,
                       int gridcap, hipStream_t st) {
  const uint32_t ntiles = (uint32_t)(M * nb);
  const unsigned grid = grid_for(ntiles, (kThreads / LANES) * U, gridcap);
  if (N % 128 == 0)
    launch_rowwise128_t<LANES, U, true>(x, dt, N, sxm, rs, q, sqm, sc, ssm, ssk, (uint32_t)nb, ntiles, grid, st);
  else
    launch_rowwise128_t<LANES, U, false>(x, dt, N, sxm, rs, q, sqm, sc, ssm, ssk, (uint32_t)nb, ntiles, grid, st);
}

// Generic row-wise: one wave per (row, tile), any block size / strides / dtype.
__global__ __launch_bounds__(kThreads) void k_rowwise_generic(const void* __restrict__ x, int dt,
                                                              int64_t M, int64_t N, int64_t sxm,
                                                              int64_t sxn, int64_t block,
                                                              int round_scale, uint8_t* q,
                                                              int64_t sqm, float* sc, int64_t ssm,
                                                              int64_t ssk, int64_t nb) {
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
    if (lane == 0) sc[row * ssm + cb * ssk] = s;
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

// ---------------------------------------------------------------------------
// 128 x 128 tile kernels: block quantization, dual quantization and row -> block
// re-quantization, dense and grouped.  A workgroup of 256 threads walks tiles
// t, t + G, t + 2G, ... (G = workgroups resident on the device at once).  Thread
// (lane16, rg) owns rows 8 rg .. 8 rg + 7 and columns 8 lane16 .. 8 lane16 + 7 of a tile.
// The raw input of the next tile is loaded into a second register set while the current
// one is quantized; the two sets alternate, so no register copy waits on a load.
//
// Column blocks that run past the last column (N % 128 != 0) go to a second launch with
// EDGE = true, whose element-wise loads and stores are masked.  The main launch addresses
// a tile through buffer descriptors whose range ends after the tile's last valid row:
// rows past it read as zero and are not written, with no per-row test.
// ---------------------------------------------------------------------------
struct TileGeo {
  int64_t r0;   // first input row
  int64_t t0;   // first column of the transposed outputs; t0 / 128 indexes their scales
  uint32_t cb;  // column block
  int nr;       // valid rows, 1..128; 0 = no tile (nothing written)
  int tw;       // transposed columns written: nr (dense) or 128 (padded axis)
};

// Dense tiles: t -> (row block t / nbc, column block cb0 + t % nbc).
struct DenseTiles {
  int64_t M;
  uint32_t nbc, cb0;
  __device__ void operator()(uint32_t t, TileGeo& g) const {
    const uint32_t rb = t / nbc;
    g.cb = cb0 + (t - rb * nbc);
    g.r0 = (int64_t)rb * 128;
    const int64_t left = M - g.r0;
    g.nr = (int)(left < 128 ? left : 128);
    g.t0 = g.r0;
    g.tw = g.nr;
  }
};

// Dense tiles in column-block-major order: t -> (row block t % nrb, column block
// cb0 + t / nrb).  The re-quantizer walks its tiles this way: the workgroups in flight
// then write whole rows of the transposed output together, which measured 8% faster on
// the config-4 shape than the row-block-major walk (the dual quantizer, with a
// row-wise output as well, measured slower in this order and keeps the other).
struct DenseTilesCM {
  int64_t M;
  uint32_t nrb, cb0;
  __device__ void operator()(uint32_t t, TileGeo& g) const {
    const uint32_t cbl = t / nrb;
    const uint32_t rb = t - cbl * nrb;
    g.cb = cb0 + cbl;
    g.r0 = (int64_t)rb * 128;
    const int64_t left = M - g.r0;
    g.nr = (int)(left < 128 ? left : 128);
    g.t0 = g.r0;
    g.tw = g.nr;
  }
};

// Grouped tiles (MoE backward): t -> (128-token chunk t / nbc of the expert-sorted rows,
// column block cb0 + t % nbc); the chunk's transposed outputs sit at its padded position
// (cin_grouped.h).  A workgroup visits increasing t, so the expert cursor only moves
// forward.  Chunks past the last one, or whose padded position does not fit in tcap
// columns, are no tile.
struct GroupedTiles {
  const int64_t* starts;
  const int64_t* ends;
  int64_t T, tcap;
  int32_t E;
  uint32_t nbc, cb0;
  // cursor: expert e owns rows [s0, s1), chunks [seen, seen + n) and padded columns from pad
  int32_t e;
  uint32_t seen, n;
  int64_t pad, s0, s1;
  __device__ void start() {
    e = 0;
    seen = 0;
    pad = 0;
    load_expert();
  }
  __device__ void load_expert() {
    // The ranges are read through the constant address space: they do not change during
    // the kernel, so the loads are scalar and wait on nothing but themselves (a vector
    // load would wait behind the tile loads and stores in flight).
    typedef __attribute__((address_space(4))) const int64_t cint64;
    int64_t a = 0, b = 0;
    if (e < E) {
      a = ((const cint64*)starts)[e];
      b = ((const cint64*)ends)[e];
      if (a < 0) a = 0;
      if (b > T) b = T;
      if (b < a) b = a;
    }
    s0 = a;
    s1 = b;
    n = (uint32_t)((b - a + 127) / 128);
  }
  __device__ void operator()(uint32_t t, TileGeo& g) {
    const uint32_t id = t / nbc;
    g.cb = cb0 + (t - id * nbc);
    while (e < E && id >= seen + n) {
      seen += n;
      pad += 128 * (int64_t)n;
      ++e;
      load_expert();
    }
    const int64_t k = (int64_t)(id - seen);
    g.r0 = s0 + 128 * k;
    g.t0 = pad + 128 * k;
    g.tw = 128;
    const int64_t left = s1 - g.r0;
    g.nr = (e < E && g.t0 + 128 <= tcap) ? (int)(left < 128 ? left : 128) : 0;
    if (g.nr == 0) g.r0 = g.t0 = 0;  // nothing is read or written for it
  }
};

__device__ inline GroupedTiles grouped_tiles(const int64_t* starts, const int64_t* ends, int64_t E,
                                             int64_t T, int64_t tcap, uint32_t nbc, uint32_t cb0) {
  GroupedTiles g;
  g.starts = starts;
  g.ends = ends;
  g.E = (int32_t)E;
  g.T = T;
  g.tcap = tcap;
  g.nbc = nbc;
  g.cb0 = cb0;
  g.start();
  return g;
}

// Walk the workgroup's tiles with the next tile's raw input loaded ahead.  The ahead
// load is unconditional, so every path issues the same loads and the wait before a
// tile's use covers that tile only; when no tile is left it loads an empty one (no valid
// rows: the main launch's buffer range is empty and nothing is read from memory).
template <typename Raw, typename Geo, typename Load, typename Proc>
__device__ __forceinline__ void tile_loop_from(uint32_t t, uint32_t G, uint32_t ntiles, Geo& geo,
                                               Load load, Proc proc) {
  if (t >= ntiles) return;
  Raw ra, rb;
  TileGeo ga, gb;
  geo(t, ga);
  load(ga, ra);
  for (;;) {
    const uint32_t t1 = t + G;
    const bool h1 = t1 < ntiles;
    if (h1) {
      geo(t1, gb);
    } else {
      gb = ga;
      gb.nr = 0;
    }
    load(gb, rb);
    proc(ga, ra);
    if (!h1) break;
    const uint32_t t2 = t1 + G;
    const bool h2 = t2 < ntiles;
    if (h2) {
      geo(t2, ga);
    } else {
      ga = gb;
      ga.nr = 0;
    }
    load(ga, ra);
    proc(gb, rb);
    if (!h2) break;
    t = t2;
  }
}

// The walk over the kernel's own grid.
template <typename Raw, typename Geo, typename Load, typename Proc>
__device__ __forceinline__ void tile_loop(uint32_t ntiles, Geo& geo, Load load, Proc proc) {
  tile_loop_from<Raw>(blockIdx.x, gridDim.x, ntiles, geo, load, proc);
}

// The same walk with one register set: each tile is loaded, then processed.  For inputs
// whose raw tile is large (fp32: 64 registers a lane), where a second set would halve the
// resident waves; the other resident workgroups' loads overlap this one's processing.
template <typename Raw, typename Geo, typename Load, typename Proc>
__device__ __forceinline__ void tile_loop_single(uint32_t ntiles, Geo& geo, Load load, Proc proc) {
  Raw r;
  TileGeo g;
  for (uint32_t t = blockIdx.x; t < ntiles; t += gridDim.x) {
    geo(t, g);
    load(g, r);
    proc(g, r);
  }
}

// Bytes from a tile's first row to the end of its last valid row (128 elements of
// `es` bytes in), in a row-major operand with rows `rowb` bytes apart.
__device__ inline int64_t tile_extent(int nr, int64_t rowb, int es) {
  return nr > 0 ? (int64_t)(nr - 1) * rowb + 128 * es : 0;
}

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
constexpr int kNT = 2;  // buffer cache policy: non-temporal (streamed through once)

// Raw input bits of a thread's 8 x 8 piece (bf16/fp16: 4 words per row, fp32: 8).
template <int DT>
struct RawIn {
  uint32_t w[8][DT == CIN_DT_F32 ? 8 : 4];
};

// Load a thread's piece of a tile.  Main launch: one 16-byte buffer load per row (two
// for fp32); rows past the tile read zero.  EDGE: element loads at clamped (in-bounds)
// addresses, zeroed outside the tile.
template <int DT, bool EDGE>
__device__ __forceinline__ void load_in(const void* __restrict__ x, int64_t sxm, int64_t N,
                                        const TileGeo& g, RawIn<DT>& o) {
  constexpr int ES = DT == CIN_DT_F32 ? 4 : 2;
  const int lane16 = threadIdx.x & 15, rg = threadIdx.x >> 4;
  if constexpr (!EDGE) {
    const int64_t rowb = sxm * ES;
    const __amdgpu_buffer_rsrc_t r = make_rsrc(
        static_cast<const char*>(x) + (g.r0 * sxm + (int64_t)g.cb * 128) * ES, tile_extent(g.nr, rowb, ES));
    const uint32_t v0 = (uint32_t)(rg * 8) * (uint32_t)rowb + (uint32_t)(lane16 * 8 * ES);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t off = v0 + (uint32_t)i * (uint32_t)rowb;
      const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kNT);
#pragma unroll
      for (int k = 0; k < 4; ++k) o.w[i][k] = a[k];
      if constexpr (DT == CIN_DT_F32) {
        const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16, 0, kNT);
#pragma unroll
        for (int k = 0; k < 4; ++k) o.w[i][4 + k] = b[k];
      }
    }
  } else {
    const int64_t c = (int64_t)g.cb * 128 + lane16 * 8;
    const int lastr = g.nr > 0 ? g.nr - 1 : 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int ri = rg * 8 + i;
      const int64_t row = g.r0 + (ri < lastr ? ri : lastr);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const bool ok = ri < g.nr && c + j < N;
        const int64_t off = row * sxm + (c + j < N ? c + j : N - 1);
        if constexpr (DT == CIN_DT_F32) {
          const uint32_t b = static_cast<const uint32_t*>(x)[off];
          o.w[i][j] = ok ? b : 0u;
        } else {
          const uint32_t b = static_cast<const uint16_t*>(x)[off];
          const uint32_t v = ok ? b : 0u;
          if (j & 1)
            o.w[i][j >> 1] |= v << 16;
          else
            o.w[i][j >> 1] = v;
        }
      }
    }
  }
}

template <int DT>
__device__ __forceinline__ float in_val(const RawIn<DT>& r, int i, int j) {
  if constexpr (DT == CIN_DT_F32) {
    return __uint_as_float(r.w[i][j]);
  } else if constexpr (DT == CIN_DT_BF16) {
    const uint32_t w = r.w[i][j >> 1];
    return (j & 1) ? bf16_hi(w) : bf16_lo(w);
  } else {
    const uint32_t w = r.w[i][j >> 1];
    const uint16_t b = (uint16_t)((j & 1) ? (w >> 16) : (w & 0xffffu));
    _Float16 h;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
  }
}

// The 8 values of row i of a piece.
template <int DT>
__device__ __forceinline__ void row_vals(const RawIn<DT>& r, int i, float (&v)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = in_val<DT>(r, i, j);
}

// Divisor for quant8: an infinite scale (infinite amax) divides by 1 with reciprocal
// 1 / inf = 0, which yields x / inf (signed zeros; NaN for an inf or NaN x).
__device__ __forceinline__ float divisor(float s) { return s == __builtin_inff() ? 1.0f : s; }

// Quantize 8 values with divisor d = divisor(s) and reciprocal r = 1 / s into two packed
// code words.
template <int STEPS>
__device__ __forceinline__ void quant8(const float (&v)[8], float d, float r, uint32_t (&out)[2]) {
  float y[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) y[i] = clamp448(div_by_scale<STEPS>(v[i], d, r));
  out[0] = cvt4_e4m3(y[0], y[1], y[2], y[3]);
  out[1] = cvt4_e4m3(y[4], y[5], y[6], y[7]);
}

// Hide a value's origin from the compiler: what is computed from it after this point is
// computed again rather than kept in registers across the barriers between, and it is
// not treated as a load from an array.
__device__ __forceinline__ void opaque(uint32_t& w) { asm volatile("" : "+v"(w)); }
__device__ __forceinline__ void opaquef(float& w) { asm volatile("" : "+v"(w)); }

template <int L>
__device__ __forceinline__ float row_bcast(float v) {  // lane L of each 16-lane DPP row
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x150 + L, 0xF, 0xF, true));
}

// Divisors and reciprocals of a thread's 8 rows from their amax values, which are equal
// across each 16-lane row: lane l computes row l % 8 once and the results are broadcast.
// Returns the scale of row l % 8 (for the scale store).
__device__ __forceinline__ float row_scales8(const float (&ra)[8], float floor_v, bool rs,
                                             float (&d)[8], float (&r)[8]) {
  // ra[l % 8] as a tree of selects on the bits of l.  The values pass through opaque()
  // first: selects between loads of one array would be folded into an indexed load,
  // which puts the array in scratch memory.
  float x0 = ra[0], x1 = ra[1], x2 = ra[2], x3 = ra[3], x4 = ra[4], x5 = ra[5], x6 = ra[6], x7 = ra[7];
  opaquef(x0); opaquef(x1); opaquef(x2); opaquef(x3);
  opaquef(x4); opaquef(x5); opaquef(x6); opaquef(x7);
  const bool b0 = threadIdx.x & 1, b1 = threadIdx.x & 2, b2 = threadIdx.x & 4;
  const float a01 = b0 ? x1 : x0, a23 = b0 ? x3 : x2, a45 = b0 ? x5 : x4, a67 = b0 ? x7 : x6;
  const float a = b2 ? (b1 ? a67 : a45) : (b1 ? a23 : a01);
  const float sv = compute_scale(fmaxf(a, floor_v), rs);
  const float dv = divisor(sv), rv = 1.0f / sv;
  d[0] = row_bcast<0>(dv); r[0] = row_bcast<0>(rv);
  d[1] = row_bcast<1>(dv); r[1] = row_bcast<1>(rv);
  d[2] = row_bcast<2>(dv); r[2] = row_bcast<2>(rv);
  d[3] = row_bcast<3>(dv); r[3] = row_bcast<3>(rv);
  d[4] = row_bcast<4>(dv); r[4] = row_bcast<4>(rv);
  d[5] = row_bcast<5>(dv); r[5] = row_bcast<5>(rv);
  d[6] = row_bcast<6>(dv); r[6] = row_bcast<6>(rv);
  d[7] = row_bcast<7>(dv); r[7] = row_bcast<7>(rv);
  return sv;
}

// Row-major code output of a tile: main launch through a buffer descriptor (rows past
// the tile are out of range), EDGE through masked byte stores.
template <bool EDGE>
struct RowOut {
  __amdgpu_buffer_rsrc_t r;
  uint32_t v0, step;
  uint8_t* base;
  int64_t ld, c, N;
  int nr, rg;
  __device__ RowOut(uint8_t* q, int64_t sqm, int64_t N_, const TileGeo& g) {
    const int lane16 = threadIdx.x & 15;
    rg = threadIdx.x >> 4;
    if constexpr (!EDGE) {
      r = make_rsrc(q + g.r0 * sqm + (int64_t)g.cb * 128, tile_extent(g.nr, sqm, 1));
      v0 = (uint32_t)(rg * 8) * (uint32_t)sqm + (uint32_t)(lane16 * 8);
      step = (uint32_t)sqm;
    } else {
      base = q + g.r0 * sqm;
      ld = sqm;
      c = (int64_t)g.cb * 128 + lane16 * 8;
      N = N_;
      nr = g.nr;
    }
  }
  __device__ void put(int i, const uint32_t (&w)[2]) const {
    if constexpr (!EDGE) {
      u32x2 x;
      x[0] = w[0];
      x[1] = w[1];
      __builtin_amdgcn_raw_buffer_store_b64(x, r, v0 + (uint32_t)i * step, 0, kNT);
    } else {
      const int ri = rg * 8 + i;
      if (ri >= nr) return;
      uint8_t* d = base + ri * ld + c;
      for (int j = 0; j < 8; ++j)
        if (c + j < N) d[j] = (uint8_t)((w[j >> 2] >> (8 * (j & 3))) & 0xffu);
    }
  }
};

// Write the transposed LDS tile: whole 16-byte pieces through a buffer descriptor when
// the tile is complete (128 x 128) and the output rows are 16-byte aligned, else the
// masked writer.
template <bool EDGE>
__device__ __forceinline__ void put_tile_t(const TileT& tileT, uint8_t* qt, int64_t sqtm, int64_t N,
                                           const TileGeo& g, bool vec_t) {
  if (!EDGE && vec_t && g.tw == 128) {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(qt + (int64_t)g.cb * 128 * sqtm + g.t0, 127 * sqtm + 128);
    const int tc0 = threadIdx.x >> 3, seg = threadIdx.x & 7;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int tc = tc0 + 32 * k;
      const uint2 w0 = *reinterpret_cast<const uint2*>(&tileT[tc][seg * 4]);
      const uint2 w1 = *reinterpret_cast<const uint2*>(&tileT[tc][seg * 4 + 2]);
      u32x4 x;
      x[0] = w0.x;
      x[1] = w0.y;
      x[2] = w1.x;
      x[3] = w1.y;
      __builtin_amdgcn_raw_buffer_store_b128(x, r, (uint32_t)tc * (uint32_t)sqtm + (uint32_t)(seg * 16), 0,
                                             kNT);
    }
  } else {
    store_tile_t(tileT, qt, sqtm, (int64_t)g.cb * 128, N, g.t0, g.tw);
  }
}

// Block amax over the workgroup (two barriers); v >= 0 and not NaN.
__device__ __forceinline__ float block_max_pos(float v, float* red) {
  v = wave_max_pos(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  uint32_t r = __float_as_uint(red[0]);
#pragma unroll
  for (int i = 1; i < kThreads / 64; ++i) r = max(r, __float_as_uint(red[i]));
  __syncthreads();
  return __uint_as_float(r);
}


// ----------------------------- block 128 x 128 -----------------------------
// Reference quantize_fp8_blockwise (src/kernels.py:94-132) for 128 x 128 blocks; the
// transposed codes serve the dgrad operand (src/kernels.py:784-788).
struct BlockSmem {
  float red[kThreads / 64];
  TileT tileT;
};

template <int DT, bool EDGE>
__device__ __forceinline__ void block_body(RawIn<DT>& raw, const TileGeo& g, int64_t N, bool rs,
                                           uint8_t* q, int64_t sqm, uint8_t* qt, int64_t sqtm,
                                           bool vec_t, float* sc, int64_t ssm, BlockSmem& sm) {
  const int lane16 = threadIdx.x & 15, rg = threadIdx.x >> 4;
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float v[8];
    row_vals<DT>(raw, i, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) a = fmaxf(a, fabsf(v[j]));
  }
  a = fmaxf(block_max_pos(a, sm.red), amax_floor(DT));
  const float s = compute_scale(a, rs);
  const float d = divisor(s), r = 1.0f / s;
  uint32_t codes[8][2];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
#pragma unroll
    for (int k = 0; k < (int)(sizeof(raw.w[0]) / sizeof(raw.w[0][0])); ++k) opaque(raw.w[i][k]);
    float v[8];
    row_vals<DT>(raw, i, v);
    quant8<kDivSteps<DT>>(v, d, r, codes[i]);
  }
  if (q) {
    const RowOut<EDGE> out(q, sqm, N, g);
#pragma unroll
    for (int i = 0; i < 8; ++i) out.put(i, codes[i]);
  }
  if (qt) {
    uint32_t cols[8][2];
    t8x8(codes, cols);
#pragma unroll
    for (int j = 0; j < 8; ++j) put_col8(sm.tileT, lane16 * 8 + j, rg, cols[j][0], cols[j][1]);
    __syncthreads();
    put_tile_t<EDGE>(sm.tileT, qt, sqtm, N, g, vec_t);
  }
  if (threadIdx.x == 0) sc[(g.t0 >> 7) * ssm + g.cb] = s;
}

// (4 waves per SIMD fit the main kernel without spills: bf16/fp16 with two register sets,
// fp32 with one, which measured 3-7% faster than two sets at 2 waves per SIMD)
template <int DT, bool EDGE>
__global__ __launch_bounds__(kThreads, EDGE ? 1 : 4) void k_blockwise128(const void* __restrict__ x, int64_t M,
                                                           int64_t N, int64_t sxm, int round_scale,
                                                           uint8_t* q, int64_t sqm, uint8_t* qt,
                                                           int64_t sqtm, int vec_t, float* sc,
                                                           int64_t ssm, uint32_t nbc, uint32_t cb0,
                                                           uint32_t ntiles) {
  __shared__ BlockSmem sm;
  DenseTiles geo{M, nbc, cb0};
  const bool rs = round_scale != 0;
  auto ld = [&](const TileGeo& g, RawIn<DT>& r) { load_in<DT, EDGE>(x, sxm, N, g, r); };
  auto pr = [&](const TileGeo& g, RawIn<DT>& r) {
    block_body<DT, EDGE>(r, g, N, rs, q, sqm, qt, sqtm, vec_t != 0, sc, ssm, sm);
  };
  if constexpr (DT == CIN_DT_F32 && !EDGE)
    tile_loop_single<RawIn<DT>>(ntiles, geo, ld, pr);
  else
    tile_loop<RawIn<DT>>(ntiles, geo, ld, pr);
}

// ----------------------------- forward-step pair -----------------------------
// The two quantizations of the reference forward (src/kernels.py:742-747) in one launch:
// workgroups [0, gw) quantize W's 128 x 128 blocks (one block each; with qt also the
// transposed codes), the others X's 1 x 128 row tiles.  W's blocks are dispatched first
// and their load latency overlaps X's streaming, instead of W paying it in a launch of its
// own (a single round of ~900 blocks).  Same code paths, same results, as
// k_blockwise128 and k_rowwise128.  W is 16-bit (the register budget of 4 waves per SIMD).
// X tiles in flight per 8-lane group: the W share's registers hold the launch at 4 waves
// per SIMD (the row-wise kernel alone runs 8), so each group keeps two tiles' loads out --
// the two rows of a unit of rowwise128_cm_body (64 tiles per workgroup and unit).
constexpr int kFwdXU = 2;
template <int XDT, int WDT>
__global__ __launch_bounds__(kThreads, 4) void k_quant_fwd(
    const void* __restrict__ x, int64_t xN, int64_t sxm, int xrs, uint8_t* xq, int64_t sxqm, float* xsc,
    int64_t sxsm, int64_t sxsk, uint32_t xnb, uint32_t xtiles, const void* __restrict__ w, int64_t wM, int64_t wN,
    int64_t swm, uint8_t* wq, int64_t swqm, uint8_t* wqt, int64_t swqtm, int wvec_t, float* wsc,
    int64_t swsm, uint32_t wnbc, uint32_t wtiles, uint32_t gw) {
  static_assert(WDT != CIN_DT_F32, "16-bit W only");
  __shared__ BlockSmem sm;
  if (blockIdx.x < gw) {  // uniform per workgroup
    DenseTiles geo{wM, wnbc, 0};
    tile_loop_from<RawIn<WDT>>(
        blockIdx.x, gw, wtiles, geo, [&](const TileGeo& g, RawIn<WDT>& r) { load_in<WDT, false>(w, swm, wN, g, r); },
        [&](const TileGeo& g, RawIn<WDT>& r) {
          block_body<WDT, false>(r, g, wN, false, wq, swqm, wqt, swqtm, wvec_t != 0, wsc, swsm, sm);
        });
  } else {
    __shared__ RowCmSmem smx;
    rowwise128_cm_body<XDT>(blockIdx.x - gw, gridDim.x - gw, x, (int64_t)(xtiles / xnb), sxm, xrs, xq, sxqm,
                            xsc, sxsm, sxsk, xnb, smx);
  }
}

// ----------------------------- dual 1x128 / 128x1 -----------------------------
// Dual quantization of a gradient tile (reference FP8MatmulFunction.backward,
// src/kernels.py:771-782): 1x128 row tiles of dY and 1x128 row tiles of dY^T (= 128x1
// column tiles of dY) from one read.  Column amax goes through LDS partials; the
// transposed codes through an LDS tile.
struct DualSmem {
  float colpart[16][128];
  float coldiv[128];
  float colrcp[128];
  TileT tileT;
};

struct NoOp {
  __device__ void operator()() const {}
};

// after_raw() runs once the raw tile is no longer read (its registers may take the next
// tile's load), before the transposed tile leaves LDS.
template <int DT, bool EDGE, typename After = NoOp>
__device__ __forceinline__ void dual_body(RawIn<DT>& raw, const TileGeo& g, int64_t N, bool rs,
                                          uint8_t* q, int64_t sqm, float* s, int64_t ssm,
                                          int64_t ssk, uint8_t* qt, int64_t sqtm, bool vec_t,
                                          float* st, int64_t sstm, int64_t sstk, DualSmem& sm,
                                          After after_raw = After()) {
  constexpr int NW = (int)(sizeof(raw.w[0]) / sizeof(raw.w[0][0]));
  const int lane16 = threadIdx.x & 15, rg = threadIdx.x >> 4;
  const float floor_v = amax_floor(DT);
  // Values are widened from the raw bits at each of their three uses (maxima, row codes,
  // column codes) rather than held as 64 floats across the barriers.
  float ra[8];
  {
    float cm[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) cm[j] = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float v[8];
      row_vals<DT>(raw, i, v);
      float a = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        a = fmaxf(a, fabsf(v[j]));
        cm[j] = fmaxf(cm[j], fabsf(v[j]));
      }
      ra[i] = a;
    }
    // column partial maxima over this thread's 8 rows
    *reinterpret_cast<float4*>(&sm.colpart[rg][lane16 * 8]) = make_float4(cm[0], cm[1], cm[2], cm[3]);
    *reinterpret_cast<float4*>(&sm.colpart[rg][lane16 * 8 + 4]) = make_float4(cm[4], cm[5], cm[6], cm[7]);
  }
  // row tiles
  {
    float dr[8], rr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) ra[i] = row16_max_pos(ra[i]);
    const float own = row_scales8(ra, floor_v, rs, dr, rr);
    const RowOut<EDGE> out(q, sqm, N, g);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int k = 0; k < NW; ++k) opaque(raw.w[i][k]);
      float v[8];
      row_vals<DT>(raw, i, v);
      uint32_t w[2];
      quant8<kDivSteps<DT>>(v, dr[i], rr[i], w);
      out.put(i, w);
    }
    const int ro = rg * 8 + (lane16 & 7);
    if (lane16 < 8 && ro < g.nr) s[(g.r0 + ro) * ssm + (int64_t)g.cb * ssk] = own;
  }
  __syncthreads();
  if (threadIdx.x < 128) {
    uint32_t a = 0u;
#pragma unroll
    for (int k = 0; k < 16; ++k) a = max(a, __float_as_uint(sm.colpart[k][threadIdx.x]));
    const float sc = compute_scale(fmaxf(__uint_as_float(a), floor_v), rs);
    sm.coldiv[threadIdx.x] = divisor(sc);
    sm.colrcp[threadIdx.x] = 1.0f / sc;
    const int64_t n = (int64_t)g.cb * 128 + threadIdx.x;
    if (!EDGE || n < N) st[n * sstm + (int64_t)(g.t0 >> 7) * sstk] = sc;
  }
  __syncthreads();
  {
    const float4 d0 = *reinterpret_cast<const float4*>(&sm.coldiv[lane16 * 8]);
    const float4 d1 = *reinterpret_cast<const float4*>(&sm.coldiv[lane16 * 8 + 4]);
    const float4 r0 = *reinterpret_cast<const float4*>(&sm.colrcp[lane16 * 8]);
    const float4 r1 = *reinterpret_cast<const float4*>(&sm.colrcp[lane16 * 8 + 4]);
    const float cd[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
    const float cr[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int k = 0; k < NW; ++k) opaque(raw.w[i][k]);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float col[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) col[i] = in_val<DT>(raw, i, j);
      uint32_t w[2];
      quant8<kDivSteps<DT>>(col, cd[j], cr[j], w);  // rows 8 rg .. 8 rg + 7, in order
      put_col8(sm.tileT, lane16 * 8 + j, rg, w[0], w[1]);
    }
  }
  after_raw();
  __syncthreads();
  put_tile_t<EDGE>(sm.tileT, qt, sqtm, N, g, vec_t);
}

template <int DT, bool EDGE, typename Geo>
__device__ __forceinline__ void dual_run(Geo& geo, uint32_t ntiles, const void* __restrict__ x,
                                         int64_t N, int64_t sxm, bool rs, uint8_t* q, int64_t sqm,
                                         float* s, int64_t ssm, int64_t ssk, uint8_t* qt, int64_t sqtm,
                                         bool vec_t, float* st, int64_t sstm, int64_t sstk,
                                         DualSmem& sm) {
  auto ld = [&](const TileGeo& g, RawIn<DT>& r) { load_in<DT, EDGE>(x, sxm, N, g, r); };
  auto pr = [&](const TileGeo& g, RawIn<DT>& r) {
    if (g.nr == 0) return;  // uniform over the workgroup
    dual_body<DT, EDGE>(r, g, N, rs, q, sqm, s, ssm, ssk, qt, sqtm, vec_t, st, sstm, sstk, sm);
  };
  // fp32: one register set at 3 waves per SIMD (two sets hold it to 2); measured 2-8%
  // faster, and 4 waves per SIMD slower on large inputs.  The next tile's load is issued
  // from inside dual_body, once the set is free (1% faster than loading after it).
  if constexpr (DT == CIN_DT_F32 && !EDGE) {
    // one register set; the next tile's load starts once this tile's values are coded
    uint32_t t = blockIdx.x;
    if (t >= ntiles) return;
    RawIn<DT> r;
    TileGeo g, gn;
    geo(t, g);
    ld(g, r);
    for (;;) {
      const uint32_t t1 = t + gridDim.x;
      const bool more = t1 < ntiles;
      if (more) {
        geo(t1, gn);
      } else {
        gn = g;
        gn.nr = 0;
      }
      if (g.nr != 0)  // uniform over the workgroup
        dual_body<DT, EDGE>(r, g, N, rs, q, sqm, s, ssm, ssk, qt, sqtm, vec_t, st, sstm, sstk, sm,
                            [&]() { ld(gn, r); });
      else
        ld(gn, r);
      if (!more) break;
      g = gn;
      t = t1;
    }
  } else {
    tile_loop<RawIn<DT>>(ntiles, geo, ld, pr);
  }
}

template <int DT, bool EDGE>
__global__ __launch_bounds__(kThreads, (DT == CIN_DT_F32 && !EDGE) ? 3 : 1) void k_dual128(const void* __restrict__ x, int64_t M,
                                                      int64_t N, int64_t sxm, int round_scale,
                                                      uint8_t* q, int64_t sqm, float* s,
                                                      int64_t ssm, int64_t ssk, uint8_t* qt,
                                                      int64_t sqtm, int vec_t, float* st,
                                                      int64_t sstm, int64_t sstk, uint32_t nbc,
                                                      uint32_t cb0, uint32_t ntiles) {
  __shared__ DualSmem sm;
  DenseTiles geo{M, nbc, cb0};
  dual_run<DT, EDGE>(geo, ntiles, x, N, sxm, round_scale != 0, q, sqm, s, ssm, ssk, qt, sqtm,
                     vec_t != 0, st, sstm, sstk, sm);
}

// Grouped: tiles are 128-token chunks of the experts (cin_grouped.h).  Rows outside
// every expert range are not quantized.
template <int DT, bool EDGE>
__global__ __launch_bounds__(kThreads, (DT == CIN_DT_F32 && !EDGE) ? 3 : 1) void k_dual128_grouped(
    const void* __restrict__ x, int64_t T, int64_t N, int64_t sxm, int round_scale, uint8_t* q,
    int64_t sqm, float* s, int64_t ssm, int64_t ssk, uint8_t* qt, int64_t sqtm, int vec_t, float* st,
    int64_t sstm, int64_t sstk, const int64_t* __restrict__ starts, const int64_t* __restrict__ ends,
    int64_t E, int64_t tcap, uint32_t nbc, uint32_t cb0, uint32_t ntiles) {
  __shared__ DualSmem sm;
  GroupedTiles geo = grouped_tiles(starts, ends, E, T, tcap, nbc, cb0);
  dual_run<DT, EDGE>(geo, ntiles, x, N, sxm, round_scale != 0, q, sqm, s, ssm, ssk, qt, sqtm,
                     vec_t != 0, st, sstm, sstk, sm);
}

// ----------------------------- SwiGLU backward + grouped dual -----------------------------
// The experts' backward computes dh12 = [dh * h2 * silu'(h1), dh * silu(h1)] ([h1 h2] = h12)
// and quantizes it both ways (k_swiglu_backward, then k_dual128_grouped).  This kernel does
// both in registers, so the fp32 dh12 [T, 2H] is never written or read back: a tile is a
// 128-token chunk x 128 columns of the first half; its pieces of dh, h1 and h2 give the
// dh12 tile of column block cb (first half) and of cb + H / 128 (second half, the same dh and
// h1), each quantized by dual_body.  The arithmetic is k_swiglu_backward's, operation for
// operation, and the tiles are k_dual128_grouped's, so the codes and scales are the same.
// H % 128 == 0 (a column block never straddles the halves).
template <int IT>
struct SwiRaw {
  RawIn<CIN_DT_F32> dh;
  RawIn<IT> a, b;  // h1, h2
};

template <int IT>
__device__ __forceinline__ void swiglu_dual_vals(const SwiRaw<IT>& r, RawIn<CIN_DT_F32>& d1,
                                                 RawIn<CIN_DT_F32>& d2) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float gv = in_val<CIN_DT_F32>(r.dh, i, j);
      const float a = in_val<IT>(r.a, i, j), b = in_val<IT>(r.b, i, j);
      const float sig = recip_ge1(1.0f + expf(-a));
      const float t = sig * (1.0f + a * (1.0f - sig));
      d1.w[i][j] = __float_as_uint(gv * b * t);
      d2.w[i][j] = __float_as_uint(gv * (a * sig));
      // both values held as computed: otherwise the second is formed after the first
      // tile's quantization, keeping dh, h1 and the sigmoid live across it
      opaque(d1.w[i][j]);
      opaque(d2.w[i][j]);
    }
  }
}

template <int IT>
__global__ __launch_bounds__(kThreads, 2) void k_swiglu_dual128_grouped(
    const float* __restrict__ dh, int64_t sdm, const void* __restrict__ h12, int64_t s12, int64_t T,
    int64_t H, int round_scale, uint8_t* q, int64_t sqm, float* s, int64_t ssm, int64_t ssk, uint8_t* qt,
    int64_t sqtm, int vec_t, float* st, int64_t sstm, int64_t sstk, const int64_t* __restrict__ starts,
    const int64_t* __restrict__ ends, int64_t E, int64_t tcap, uint32_t nbh, uint32_t ntiles) {
  __shared__ DualSmem sm;
  GroupedTiles geo = grouped_tiles(starts, ends, E, T, tcap, nbh, 0);
  const int64_t N = 2 * H;
  const bool rs = round_scale != 0, vt = vec_t != 0;
  uint32_t t = blockIdx.x;
  if (t >= ntiles) return;
  SwiRaw<IT> r;
  TileGeo g, gn;
  geo(t, g);
  load_in<CIN_DT_F32, false>(dh, sdm, H, g, r.dh);
  load_in<IT, false>(h12, s12, N, g, r.a);
  {
    TileGeo gb = g;
    gb.cb += nbh;
    load_in<IT, false>(h12, s12, N, gb, r.b);
  }
  // The next tile's inputs load while this tile is quantized: dh after the first half's
  // tile, h1 and h2 after the second's (their registers are free then: the values live
  // in d1 and d2).  Measured 1.29 -> 0.78 ms at 131072 x 2048.
  for (;;) {
    RawIn<CIN_DT_F32> d1, d2;
    swiglu_dual_vals<IT>(r, d1, d2);
    const uint32_t t1 = t + gridDim.x;
    const bool more = t1 < ntiles;
    if (more) {
      geo(t1, gn);
    } else {
      gn = g;
      gn.nr = 0;
    }
    TileGeo g2 = g;
    g2.cb += nbh;
    if (g.nr != 0)  // uniform over the workgroup
      dual_body<CIN_DT_F32, false>(d1, g, N, rs, q, sqm, s, ssm, ssk, qt, sqtm, vt, st, sstm, sstk, sm);
    load_in<CIN_DT_F32, false>(dh, sdm, H, gn, r.dh);
    if (g.nr != 0)
      dual_body<CIN_DT_F32, false>(d2, g2, N, rs, q, sqm, s, ssm, ssk, qt, sqtm, vt, st, sstm, sstk, sm);
    load_in<IT, false>(h12, s12, N, gn, r.a);
    {
      TileGeo gb = gn;
      gb.cb += nbh;
      load_in<IT, false>(h12, s12, N, gb, r.b);
    }
    if (!more) break;
    g = gn;
    t = t1;
  }
}

// ----------------------------- row -> block re-quantization -----------------------------
// x = fp32(code) * srow (fp32 product, as the reference's dequantize_fp8_rowwise), then
// the block quantizer with the fp32 floor and round_scale = False (reference
// src/kernels.py:784-788 re-quantizes the saved row-wise X this way).
struct RawQ {
  uint32_t w[8][2];  // 8 codes per row
  float sr[8];       // row scale of each row (0 for rows past the tile)
};

template <bool EDGE>
__device__ __forceinline__ void load_q(const uint8_t* __restrict__ q, int64_t sqm, int64_t K,
                                       const float* __restrict__ srow, int64_t ssm, int64_t ssk,
                                       const TileGeo& g, RawQ& o) {
  const int lane16 = threadIdx.x & 15, rg = threadIdx.x >> 4;
  if constexpr (!EDGE) {
    const __amdgpu_buffer_rsrc_t r =
        make_rsrc(q + g.r0 * sqm + (int64_t)g.cb * 128, tile_extent(g.nr, sqm, 1));
    const __amdgpu_buffer_rsrc_t rsc =
        make_rsrc(srow + g.r0 * ssm + (int64_t)g.cb * ssk, g.nr > 0 ? ((int64_t)(g.nr - 1) * ssm + 1) * 4 : 0);
    const uint32_t v0 = (uint32_t)(rg * 8) * (uint32_t)sqm + (uint32_t)(lane16 * 8);
    const uint32_t s0 = (uint32_t)(rg * 8) * (uint32_t)(ssm * 4);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(r, v0 + (uint32_t)i * (uint32_t)sqm, 0, kNT);
      o.w[i][0] = w[0];
      o.w[i][1] = w[1];
      o.sr[i] = __uint_as_float(
          __builtin_amdgcn_raw_buffer_load_b32(rsc, s0 + (uint32_t)i * (uint32_t)(ssm * 4), 0, 0));
    }
  } else {
    const int64_t c = (int64_t)g.cb * 128 + lane16 * 8;
    const int lastr = g.nr > 0 ? g.nr - 1 : 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int ri = rg * 8 + i;
      const bool rok = ri < g.nr;
      const int64_t row = g.r0 + (ri < lastr ? ri : lastr);
      const float sv = srow[row * ssm + (int64_t)g.cb * ssk];
      o.sr[i] = rok ? sv : 0.0f;
      o.w[i][0] = o.w[i][1] = 0u;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const bool ok = rok && c + j < K;
        const uint32_t b = q[row * sqm + (c + j < K ? c + j : K - 1)];
        o.w[i][j >> 2] |= (ok ? b : 0u) << (8 * (j & 3));
      }
    }
  }
}

// fp32(code) of the 8 codes of a row (hardware e4m3fn -> fp32, exact).
__device__ __forceinline__ void codes_f32(const uint32_t (&w)[2], float (&f)[8]) {
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[k], false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[k], true);
    f[4 * k] = lo[0];
    f[4 * k + 1] = lo[1];
    f[4 * k + 2] = hi[0];
    f[4 * k + 3] = hi[1];
  }
}

struct RequantSmem {
  float red[kThreads / 64];
  TileT tileT;
};

template <bool EDGE>
__device__ __forceinline__ void requant_body(RawQ& raw, const TileGeo& g, int64_t K, uint8_t* qb,
                                             int64_t sqbm, uint8_t* qbt, int64_t sqbtm, bool vec_t,
                                             float* sblk, int64_t ssbm, RequantSmem& sm) {
  const int lane16 = threadIdx.x & 15, rg = threadIdx.x >> 4;
  const int64_t c = (int64_t)g.cb * 128 + lane16 * 8;
  // Block amax.  |fl(c sr)| = fl(|c| |sr|) is monotone in |c|, so a row's largest
  // magnitude is fl(max |c| * |sr|); NaN products are skipped either way.
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float f[8];
    codes_f32(raw.w[i], f);
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(f[j]));
    a = fmaxf(a, __fmul_rn(m, fabsf(raw.sr[i])));
  }
  a = fmaxf(block_max_pos(a, sm.red), kFloorF32);
  const float s = compute_scale(a, false);
  const float d = divisor(s), r = 1.0f / s;
  uint32_t codes[8][2];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    opaque(raw.w[i][0]);
    opaque(raw.w[i][1]);
    float v[8];
    codes_f32(raw.w[i], v);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v[j] = __fmul_rn(v[j], raw.sr[i]);
      if (EDGE && !(rg * 8 + i < g.nr && c + j < K)) v[j] = 0.0f;  // not 0 * srow: srow may be inf
    }
    quant8<2>(v, d, r, codes[i]);
  }
  if (qb) {
    const RowOut<EDGE> out(qb, sqbm, K, g);
#pragma unroll
    for (int i = 0; i < 8; ++i) out.put(i, codes[i]);
  }
  if (qbt) {
    uint32_t cols[8][2];
    t8x8(codes, cols);
#pragma unroll
    for (int j = 0; j < 8; ++j) put_col8(sm.tileT, lane16 * 8 + j, rg, cols[j][0], cols[j][1]);
    __syncthreads();
    put_tile_t<EDGE>(sm.tileT, qbt, sqbtm, K, g, vec_t);
  }
  if (threadIdx.x == 0) sblk[(g.t0 >> 7) * ssbm + g.cb] = s;
}

template <bool EDGE, typename Geo>
__device__ __forceinline__ void requant_run(Geo& geo, uint32_t ntiles, const uint8_t* __restrict__ q,
                                            int64_t K, int64_t sqm, const float* __restrict__ srow,
                                            int64_t ssm, int64_t ssk, uint8_t* qb, int64_t sqbm, uint8_t* qbt,
                                            int64_t sqbtm, bool vec_t, float* sblk, int64_t ssbm,
                                            RequantSmem& sm) {
  // One register set: without the second the dense kernel holds 5 waves per SIMD (96
  // VGPRs, no spills), and the VALU-heavy tiles of more workgroups overlap each other's
  // loads.  Measured on config-4 X: 27.8 against 30.9 us with two sets at 4 waves; the
  // grouped kernel (more geometry in registers) at 4 waves: 454 against 463 us on config 3.
  tile_loop_single<RawQ>(
      ntiles, geo, [&](const TileGeo& g, RawQ& r) { load_q<EDGE>(q, sqm, K, srow, ssm, ssk, g, r); },
      [&](const TileGeo& g, RawQ& r) {
        if (g.nr == 0) return;  // uniform over the workgroup
        requant_body<EDGE>(r, g, K, qb, sqbm, qbt, sqbtm, vec_t, sblk, ssbm, sm);
      });
}

template <bool EDGE>
__global__ __launch_bounds__(kThreads, 5) void k_requant128(const uint8_t* __restrict__ q, int64_t M,
                                                         int64_t K, int64_t sqm,
                                                         const float* __restrict__ srow,
                                                         int64_t ssm, int64_t ssk, uint8_t* qb, int64_t sqbm,
                                                         uint8_t* qbt, int64_t sqbtm, int vec_t,
                                                         float* sblk, int64_t ssbm, uint32_t nbc,
                                                         uint32_t cb0, uint32_t ntiles) {
  __shared__ RequantSmem sm;
  (void)nbc;
  DenseTilesCM geo{M, (uint32_t)((M + 127) >> 7), cb0};
  requant_run<EDGE>(geo, ntiles, q, K, sqm, srow, ssm, ssk, qb, sqbm, qbt, sqbtm, vec_t != 0, sblk,
                    ssbm, sm);
}

// Grouped: tiles are 128-token chunks of the experts; block scales are indexed by the
// chunk's padded position, codes by the input row (qb) or the padded column (qbt).
template <bool EDGE>
__global__ __launch_bounds__(kThreads) void k_requant128_grouped(
    const uint8_t* __restrict__ q, int64_t T, int64_t K, int64_t sqm, const float* __restrict__ srow,
    int64_t ssm, int64_t ssk, uint8_t* qb, int64_t sqbm, uint8_t* qbt, int64_t sqbtm, int vec_t, float* sblk,
    int64_t ssbm, const int64_t* __restrict__ starts, const int64_t* __restrict__ ends, int64_t E,
    int64_t tcap, uint32_t nbc, uint32_t cb0, uint32_t ntiles) {
  __shared__ RequantSmem sm;
  GroupedTiles geo = grouped_tiles(starts, ends, E, T, tcap, nbc, cb0);
  requant_run<EDGE>(geo, ntiles, q, K, sqm, srow, ssm, ssk, qb, sqbm, qbt, sqbtm, vec_t != 0, sblk,
                    ssbm, sm);
}

// ----------------------------- backward pair in one launch -----------------------------
// FP8MatmulFunction.backward needs both quantizations of dY (src/kernels.py:771, :781-783)
// and the 128 x 128 re-quantization of the saved X codes (:784-787).  One launch walks both
// tile sets: walk index t < nd is dual tile t of dY (row-block major, as k_dual128), the rest
// are re-quantization tiles of X (column-block major, as k_requant128).  With the dual tiles
// first, the first round of workgroups holds both kinds, so the memory-bound dual tiles and
// the VALU-heavy re-quantization tiles share the CUs, and the second launch's ramp is gone.
// Each tile is loaded, then processed (one register set); the other resident workgroups'
// loads overlap a tile's arithmetic.  Same tile bodies as the two kernels, so the same bits.
union BwdSmem {
  DualSmem d;
  RequantSmem r;
};

template <int DT>
__global__ __launch_bounds__(kThreads, 5) void k_quant_bwd(
    const void* __restrict__ dy, int64_t M, int64_t N, int64_t sdm, int round_scale, uint8_t* q,
    int64_t sqm, float* s, int64_t ssm, int64_t ssk, uint8_t* qt, int64_t sqtm, int dvec_t, float* st,
    int64_t sstm, int64_t sstk, const uint8_t* __restrict__ xq, int64_t K, int64_t sxqm,
    const float* __restrict__ srow, int64_t ssrm, int64_t ssrk, uint8_t* xbt, int64_t sxbtm, int rvec_t, float* sblk, int64_t ssbm, uint32_t nd,
    uint32_t ntiles) {
  static_assert(DT != CIN_DT_F32, "the pair launch takes 16-bit dY");
  __shared__ BwdSmem sm;
  uint32_t t = blockIdx.x;
  {
    const DenseTiles dgeo{M, (uint32_t)(N >> 7), 0};
    for (; t < nd; t += gridDim.x) {
      TileGeo g;
      dgeo(t, g);
      RawIn<DT> r;
      load_in<DT, false>(dy, sdm, N, g, r);
      dual_body<DT, false>(r, g, N, round_scale != 0, q, sqm, s, ssm, ssk, qt, sqtm, dvec_t != 0, st, sstm,
                           sstk, sm.d);
    }
  }
  __syncthreads();  // the union's other member: every thread is past its dual tiles
  const DenseTilesCM rgeo{M, (uint32_t)((M + 127) >> 7), 0};
  for (; t < ntiles; t += gridDim.x) {
    TileGeo g;
    rgeo(t - nd, g);
    RawQ r;
    load_q<false>(xq, sxqm, K, srow, ssrm, ssrk, g, r);
    requant_body<false>(r, g, K, nullptr, 0, xbt, sxbtm, rvec_t != 0, sblk, ssbm, sm.r);
  }
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


// ---------------------------------------------------------------------------
// SwiGLU activation fused into the row-wise quantizer (reference GroupedExperts.forward,
// src/layers.py:72-74): h = silu(h12[:, :H]) * h12[:, H:] in fp32, rounded to the
// activation dtype OT, then the 1x128 tiles of h exactly as quantize_fp8_rowwise(h)
// (src/kernels.py:19-71).  silu(a) = a / (1 + exp(-a)) with an IEEE division: the
// operations of torch's GPU silu, so the codes equal quantizing torch's h.  A 16-lane DPP
// row owns one tile, 8 consecutive elements per lane.
// ---------------------------------------------------------------------------
template <int OT>
__device__ __forceinline__ float round_to(float h) {
  if constexpr (OT == CIN_DT_BF16) return __uint_as_float(f32_to_bf16_bits(h) << 16);
  // through the pinned conversion: a bare (_Float16)(silu * b) lets the compiler fuse the
  // product and the conversion into v_fma_mixlo_f16 with a +0 addend, which rounds the
  // exact product once and turns a -0 product (an exactly zero input) into +0
  else if constexpr (OT == CIN_DT_F16) return half_bits_to_f32(CIN_DT_F16, f32_to_f16_bits(h));
  else return h;
}

template <int IT, int OT>
__global__ __launch_bounds__(kThreads) void k_silu_mul_rowwise128(
    const void* __restrict__ h12, int64_t s12, int64_t H, int round_scale, uint8_t* __restrict__ q,
    int64_t sqm, float* __restrict__ sc, int64_t ssm, int64_t ssk, uint32_t nb, uint32_t ntiles) {
  const int li = threadIdx.x & 15;
  const uint32_t G = (gridDim.x * kThreads) / 16;
  const bool rs = round_scale != 0;
  for (uint32_t t = (blockIdx.x * kThreads + threadIdx.x) / 16; t < ntiles; t += G) {
    const uint32_t row = t / nb, cb = t - row * nb;
    const int64_t c = (int64_t)cb * 128 + li * 8;
    int64_t nv = H - c;
    nv = nv < 0 ? 0 : (nv > 8 ? 8 : nv);
    Vec8<IT> a, b;
    load8<IT>(h12, (int64_t)row * s12 + c, nv, a);
    load8<IT>(h12, (int64_t)row * s12 + H + c, nv, b);
    float v[8];
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float x = a.v[j];
      const float silu = x / (1.0f + expf(-x));
      v[j] = j < nv ? round_to<OT>(silu * b.v[j]) : 0.0f;
      m = fmaxf(m, fabsf(v[j]));
    }
    m = row16_max_pos(m);
    const float sv = compute_scale(fmaxf(m, amax_floor(OT)), rs);
    uint32_t w[2];
    quant8<kDivSteps<OT>>(v, divisor(sv), 1.0f / sv, w);
    uint8_t* qp = q + (int64_t)row * sqm + c;
    if (nv == 8) {
      *reinterpret_cast<uint2*>(qp) = make_uint2(w[0], w[1]);
    } else {
      for (int j = 0; j < nv; ++j) qp[j] = (uint8_t)((w[j >> 2] >> (8 * (j & 3))) & 0xffu);
    }
    if (li == 0) sc[(int64_t)row * ssm + (int64_t)cb * ssk] = sv;
  }
}

// ---------------------------------------------------------------------------
// SwiGLU backward in one pass: for h = silu(h1) * h2 with [h1 h2] = h12,
//   dh12[:, :H] = dh * h2 * (sig * (1 + h1 * (1 - sig))),  dh12[:, H:] = dh * (h1 * sig),
// sig = 1 / (1 + exp(-h1)), every product and sum rounded to fp32 in that order (the
// elementwise chain it replaces computes the same way, one rounding per operation).
// A thread owns 4 consecutive columns of a row.
// ---------------------------------------------------------------------------
template <int IT>
__global__ __launch_bounds__(kThreads) void k_swiglu_backward(
    const float* __restrict__ dh, int64_t sdm, const void* __restrict__ h12, int64_t s12,
    int64_t M, int64_t H, float* __restrict__ dh12, int64_t som) {
  const int64_t nq = H / 4;
  const int64_t total = M * nq;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kThreads) {
    const int64_t r = i / nq, j = (i - r * nq) * 4;
    const f32x4 g = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(dh + r * sdm + j));
    const float gv[4] = {g[0], g[1], g[2], g[3]};
    float a[4], b[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      a[k] = load_elem(h12, IT, r * s12 + j + k);
      b[k] = load_elem(h12, IT, r * s12 + H + j + k);
    }
    float d1[4], d2[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float sig = recip_ge1(1.0f + expf(-a[k]));
      const float t = sig * (1.0f + a[k] * (1.0f - sig));
      d1[k] = gv[k] * b[k] * t;
      d2[k] = gv[k] * (a[k] * sig);
    }
    *reinterpret_cast<float4*>(dh12 + r * som + j) = make_float4(d1[0], d1[1], d1[2], d1[3]);
    *reinterpret_cast<float4*>(dh12 + r * som + H + j) = make_float4(d2[0], d2[1], d2[2], d2[3]);
  }
}

// ---------------------------------------------------------------------------
// Zero the rows of a [T, ncols] matrix that lie outside every expert range: the grouped
// kernels never write them, and with ranges that cover all rows (a router's counts)
// this reads the ranges and writes nothing.  A thread owns a row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void k_zero_uncovered(uint8_t* __restrict__ C, int64_t ldc_bytes,
                                                             int64_t row_bytes, int64_t T,
                                                             const int64_t* __restrict__ starts,
                                                             const int64_t* __restrict__ ends,
                                                             int64_t E) {
  typedef __attribute__((address_space(4))) const int64_t cint64;
  const int64_t r = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (r >= T) return;
  bool covered = false;
  for (int64_t e = 0; e < E && !covered; ++e)
    covered = r >= ((const cint64*)starts)[e] && r < ((const cint64*)ends)[e];
  if (covered) return;
  uint8_t* p = C + r * ldc_bytes;
  int64_t i = 0;
  if ((((uintptr_t)p) & 15) == 0)
    for (; i + 16 <= row_bytes; i += 16) *reinterpret_cast<uint4*>(p + i) = make_uint4(0, 0, 0, 0);
  for (; i < row_bytes; ++i) p[i] = 0;
}

// Workgroups for a persistent tile kernel: as many as the device holds at once (from the
// kernel's occupancy and the device's CU count), at most one per tile.
template <auto Kernel>
unsigned resident_grid(uint32_t ntiles) {
  static int per_cu = 0;
  if (per_cu == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(Kernel),
                                                     kThreads, 0) != hipSuccess || n < 1)
      n = 1;
    per_cu = n;
  }
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
      n = 256;
    cus[dev] = n;
  }
  const int64_t g = (int64_t)per_cu * cus[dev];
  return (unsigned)(g < (int64_t)ntiles ? g : (int64_t)ntiles);
}

// Output rows that no assignment reaches (perm[r] < 0: the tail after dropped ids) get the
// quantization of a zero row: codes 0 and the scale of the amax floor.  A thread owns a
// row; routed rows (all of them when no id was dropped) return at once, or, with a
// token-major scale table tok [T, nb] (kMapScatterTok), copy their token's scales: row r's
// scales are tok[perm[r] / k], and threads of consecutive rows store consecutive addresses
// in either layout (column-major: one run per column block; row-major: whole rows).
__global__ __launch_bounds__(kThreads) void k_zero_unrouted(const int64_t* __restrict__ perm,
                                                            int64_t rows, int64_t N, int dt,
                                                            int round_scale, uint8_t* q,
                                                            int64_t sqm, float* sc, int64_t ssm,
                                                            int64_t ssk, const float* __restrict__ tok = nullptr,
                                                            int64_t k = 1, int64_t ntok = 0) {
  const int64_t r = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (r >= rows) return;
  const int64_t a = perm[r];
  const int64_t nb = (N + 127) / 128;
  if (a >= 0) {
    const int64_t t = a / k;
    if (tok == nullptr || t >= ntok) return;  // (an assignment past the tokens: left as is)
    const float* src = tok + t * nb;
    if ((nb & 3) == 0) {  // 16-byte rows of the table (it is 16-byte aligned)
      for (int64_t b = 0; b < nb; b += 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(src + b);
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[r * ssm + (b + e) * ssk] = v[e];
      }
    } else {
      for (int64_t b = 0; b < nb; ++b) sc[r * ssm + b * ssk] = src[b];
    }
    return;
  }
  const float s = compute_scale(amax_floor(dt), round_scale != 0);
  for (int64_t b = 0; b < nb; ++b) sc[r * ssm + b * ssk] = s;
  uint8_t* p = q + r * sqm;  // 8-byte aligned (q and sqm are)
  int64_t c = 0;
  for (; c + 8 <= N; c += 8) *reinterpret_cast<uint2*>(p + c) = make_uint2(0u, 0u);
  for (; c < N; ++c) p[c] = 0;
}

// An R x C matrix of scales at strides (sr, sc) whose elements do not overlap: row-major
// (sc == 1, sr >= C) or column-major (sr == 1, sc >= R); a single row or column takes any
// positive stride.
inline bool scale_layout_ok(int64_t R, int64_t C, int64_t sr, int64_t sc) {
  if (R <= 1 && C <= 1) return true;
  if (R <= 1) return sc >= 1;
  if (C <= 1) return sr >= 1;
  return (sc == 1 && sr >= C) || (sr == 1 && sc >= R);
}

}  // namespace

// The indexer's two quantizations in one launch: workgroups [0, gk) quantize k's rows (16
// lanes per tile: a small, latency-bound set), the others q's (8 lanes per tile), each
// keeping the first scale of a row only.  Against two launches (config 5: q [16, 1024, 4,
// 128], k [16, 1024, 128] bf16): the quantize call 22 -> 20 us, the scoring call with it
// 44 -> 41 us, same codes and scales.
template <int DT, bool FULL>
__global__ __launch_bounds__(kThreads) void k_indexer_quant2(const void* __restrict__ q, const void* __restrict__ k,
                                                             int64_t d, uint8_t* __restrict__ q8,
                                                             float* __restrict__ qs, uint8_t* __restrict__ k8,
                                                             float* __restrict__ ks, uint32_t nb, uint32_t ntq,
                                                             uint32_t ntk, uint32_t gk) {
  if (blockIdx.x < gk)
    rowwise128_body<DT, 16, 1, FULL, kMapFirstScale>(blockIdx.x, gk, k, d, d, 0, k8, d, ks, 1, 0, nb, ntk,
                                                     nullptr, 1, 0);
  else
    rowwise128_body<DT, 8, 1, FULL, kMapFirstScale>(blockIdx.x - gk, gridDim.x - gk, q, d, d, 0, q8, d, qs, 1, 0,
                                                    nb, ntq, nullptr, 1, 0);
}

extern "C" {

int cin_quant_rowwise(const void* x, int x_dtype, int64_t M, int64_t N, int64_t sxm, int64_t sxn,
                      int64_t block, int round_scale, uint8_t* q, int64_t sqm, float* scales,
                      int64_t ssm, int64_t ssk, void* stream) {
  CIN_CHECK_ARG(valid_dtype(x_dtype), "quant_rowwise: unsupported x dtype %d", x_dtype);
  CIN_CHECK_ARG(M >= 0 && N >= 0, "quant_rowwise: negative shape");
  CIN_CHECK_ARG(block >= 1 && block <= 1024, "quant_rowwise: block %lld outside [1, 1024]",
                (long long)block);
  if (M == 0 || N == 0) return CIN_OK;
  CIN_CHECK_ARG(x && q && scales, "quant_rowwise: null pointer");
  const int64_t nb = cdiv(N, block);
  CIN_CHECK_ARG(sqm >= N, "quant_rowwise: output row stride too small");
  CIN_CHECK_ARG(scale_layout_ok(M, nb, ssm, ssk), "quant_rowwise: scale strides overlap");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int es = elem_size(x_dtype);
  const bool fast = block == 128 && sxn == 1 && aligned(x, 16) && ((sxm * es) % 16 == 0) &&
                    aligned(q, 8) && (sqm % 8 == 0) && M * nb < (int64_t)1 << 31;
  if (fast && N % 128 == 0) {
    // whole column blocks: the unit walk (rowwise128_cm_body), either scale layout
    const int64_t units = cdiv(M, 8) * cdiv(nb, 8);
    const unsigned grid = grid_for(units * 64, 64, 16384);
    if (x_dtype == CIN_DT_BF16)
      hipLaunchKernelGGL(k_rowwise128_cm<CIN_DT_BF16>, grid, kThreads, 0, s, x, M, sxm, round_scale, q, sqm, scales, ssm, ssk, (uint32_t)nb);
    else if (x_dtype == CIN_DT_F16)
      hipLaunchKernelGGL(k_rowwise128_cm<CIN_DT_F16>, grid, kThreads, 0, s, x, M, sxm, round_scale, q, sqm, scales, ssm, ssk, (uint32_t)nb);
    else
      hipLaunchKernelGGL(k_rowwise128_cm<CIN_DT_F32>, grid, kThreads, 0, s, x, M, sxm, round_scale, q, sqm, scales, ssm, ssk, (uint32_t)nb);
  } else if (fast) {
    launch_rowwise128<8, 1>(x, x_dtype, M, N, sxm, round_scale, q, sqm, scales, ssm, ssk, nb, 16384, s);
  } else {
    const unsigned grid = grid_for(M * nb, kThreads / 64, 65536);
    hipLaunchKernelGGL(k_rowwise_generic, grid, kThreads, 0, s, x, x_dtype, M, N, sxm, sxn, block,
                       round_scale, q, sqm, scales, ssm, ssk, nb);
  }
  return cin_check_launch("quant_rowwise");
}

int cin_indexer_quantize(const void* q, int q_dtype, const void* k, int k_dtype, int64_t B,
                         int64_t L, int64_t S, int64_t H, int64_t d, uint8_t* q8, float* q_scale,
                         uint8_t* k8, float* k_scale, void* stream) {
  CIN_CHECK_ARG(valid_dtype(q_dtype) && valid_dtype(k_dtype), "indexer_quantize: unsupported dtype");
  CIN_CHECK_ARG(B >= 0 && L >= 0 && S >= 0 && H >= 1, "indexer_quantize: bad sizes");
  CIN_CHECK_ARG(d >= 32 && d <= 256 && d % 32 == 0,
                "indexer_quantize: head dim %lld must be a multiple of 32 in [32, 256]", (long long)d);
  const int64_t mq = B * L * H, mk = B * S, nb = cdiv(d, 128);
  CIN_CHECK_ARG(mq * nb < ((int64_t)1 << 31) && mk * nb < ((int64_t)1 << 31), "indexer_quantize: too many rows");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool full = d % 128 == 0;
  if (q_dtype == k_dtype && mq > 0 && mk > 0) {
    CIN_CHECK_ARG(q && q8 && q_scale && k && k8 && k_scale, "indexer_quantize: null pointer");
    CIN_CHECK_ARG(aligned(q, 16) && aligned(q8, 8) && aligned(k, 16) && aligned(k8, 8),
                  "indexer_quantize: inputs must be 16-byte and codes 8-byte aligned");
    const uint32_t ntq = (uint32_t)(mq * nb), ntk = (uint32_t)(mk * nb);
    const unsigned gk = grid_for(ntk, kThreads / 16, 16384), gq = grid_for(ntq, kThreads / 8, 16384);
#define CIN_IQ2(DT, FULL)                                                                             \
  hipLaunchKernelGGL((k_indexer_quant2<DT, FULL>), gk + gq, kThreads, 0, st, q, k, d, q8, q_scale, k8, \
                     k_scale, (uint32_t)nb, ntq, ntk, gk)
    if (q_dtype == CIN_DT_BF16) {
      if (full) CIN_IQ2(CIN_DT_BF16, true); else CIN_IQ2(CIN_DT_BF16, false);
    } else if (q_dtype == CIN_DT_F16) {
      if (full) CIN_IQ2(CIN_DT_F16, true); else CIN_IQ2(CIN_DT_F16, false);
    } else {
      if (full) CIN_IQ2(CIN_DT_F32, true); else CIN_IQ2(CIN_DT_F32, false);
    }
#undef CIN_IQ2
    return cin_check_launch("indexer_quantize");
  }
  struct Side { const void* x; int dt; int64_t rows; uint8_t* codes; float* scales; };
  const Side sides[2] = {{q, q_dtype, mq, q8, q_scale}, {k, k_dtype, mk, k8, k_scale}};
  for (const Side& sd : sides) {
    if (sd.rows == 0) continue;
    CIN_CHECK_ARG(sd.x && sd.codes && sd.scales, "indexer_quantize: null pointer");
    CIN_CHECK_ARG(aligned(sd.x, 16) && aligned(sd.codes, 8),
                  "indexer_quantize: inputs must be 16-byte and codes 8-byte aligned");
    const uint32_t ntiles = (uint32_t)(sd.rows * nb);
    // (q and k of different dtypes.)  Below ~32K tiles the launch is latency-bound: 16
    // lanes per tile halve each lane's loads (16384 k rows of 128: 4.6 -> 3.5 us); above, 8
    // lanes per tile are faster (65536 q rows: 5.5 us against 6.5).
    if (ntiles < 32768) {
      const unsigned grid = grid_for(ntiles, kThreads / 16, 16384);
      if (full)
        launch_rowwise128_t<16, 1, true, kMapFirstScale>(sd.x, sd.dt, d, d, 0, sd.codes, d, sd.scales, 1, 0,
                                                         (uint32_t)nb, ntiles, grid, st);
      else
        launch_rowwise128_t<16, 1, false, kMapFirstScale>(sd.x, sd.dt, d, d, 0, sd.codes, d, sd.scales, 1, 0,
                                                          (uint32_t)nb, ntiles, grid, st);
    } else {
      const unsigned grid = grid_for(ntiles, kThreads / 8, 16384);
      if (full)
        launch_rowwise128_t<8, 1, true, kMapFirstScale>(sd.x, sd.dt, d, d, 0, sd.codes, d, sd.scales, 1, 0,
                                                        (uint32_t)nb, ntiles, grid, st);
      else
        launch_rowwise128_t<8, 1, false, kMapFirstScale>(sd.x, sd.dt, d, d, 0, sd.codes, d, sd.scales, 1, 0,
                                                         (uint32_t)nb, ntiles, grid, st);
    }
  }
  return cin_check_launch("indexer_quantize");
}

int cin_moe_gather_quant_rowwise(const void* x, int x_dtype, int64_t src_rows, int64_t N,
                                 int64_t sxm, const int64_t* rowmap, int64_t rows, int64_t rowdiv,
                                 int round_scale, uint8_t* q, int64_t sqm, float* scales,
                                 int64_t ssm, int64_t ssk, void* stream) {
  CIN_CHECK_ARG(valid_dtype(x_dtype), "moe_gather_quant: unsupported x dtype %d", x_dtype);
  CIN_CHECK_ARG(src_rows >= 0 && N >= 0 && rows >= 0 && rowdiv >= 1,
                "moe_gather_quant: negative shape or row divisor < 1");
  if (rows == 0 || N == 0) return CIN_OK;
  CIN_CHECK_ARG(x && rowmap && q && scales, "moe_gather_quant: null pointer");
  const int64_t nb = cdiv(N, 128);
  CIN_CHECK_ARG(sqm >= N, "moe_gather_quant: output row stride too small");
  CIN_CHECK_ARG(scale_layout_ok(rows, nb, ssm, ssk), "moe_gather_quant: scale strides overlap");
  const int es = elem_size(x_dtype);
  CIN_CHECK_ARG(aligned(x, 16) && (sxm * es) % 16 == 0 && sxm >= N && aligned(q, 8) && sqm % 8 == 0,
                "moe_gather_quant: x rows must be contiguous and 16-byte aligned, q rows 8-byte aligned");
  CIN_CHECK_ARG(rows * nb < (int64_t)1 << 31, "moe_gather_quant: too many tiles");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint32_t ntiles = (uint32_t)(rows * nb);
  const unsigned grid = grid_for(ntiles, kThreads / 8, 16384);
  if (N % 128 == 0)
    launch_rowwise128_t<8, 1, true, kMapGather>(x, x_dtype, N, sxm, round_scale, q, sqm, scales,
                                                ssm, ssk, (uint32_t)nb, ntiles, grid, s, rowmap, rowdiv,
                                                src_rows);
  else
    launch_rowwise128_t<8, 1, false, kMapGather>(x, x_dtype, N, sxm, round_scale, q, sqm, scales,
                                                 ssm, ssk, (uint32_t)nb, ntiles, grid, s, rowmap,
                                                 rowdiv, src_rows);
  return cin_check_launch("moe_gather_quant_rowwise");
}

int cin_moe_scatter_quant_rowwise(const void* x, int x_dtype, int64_t T, int64_t N, int64_t sxm,
                                  const int32_t* inv, int64_t k, const int64_t* perm, int64_t rows,
                                  int round_scale, uint8_t* q, int64_t sqm, float* scales,
                                  int64_t ssm, int64_t ssk, void* stream) {
  CIN_CHECK_ARG(valid_dtype(x_dtype), "moe_scatter_quant: unsupported x dtype %d", x_dtype);
  CIN_CHECK_ARG(T >= 0 && N >= 0 && rows >= 0 && k >= 1, "moe_scatter_quant: bad sizes");
  if (N == 0 || (T == 0 && rows == 0)) return CIN_OK;
  CIN_CHECK_ARG(x && inv && perm && q && scales, "moe_scatter_quant: null pointer");
  const int64_t nb = cdiv(N, 128);
  CIN_CHECK_ARG(sqm >= N, "moe_scatter_quant: output row stride too small");
  CIN_CHECK_ARG(scale_layout_ok(rows, nb, ssm, ssk), "moe_scatter_quant: scale strides overlap");
  const int es = elem_size(x_dtype);
  CIN_CHECK_ARG(aligned(x, 16) && (sxm * es) % 16 == 0 && sxm >= N && aligned(q, 8) && sqm % 8 == 0,
                "moe_scatter_quant: x rows must be contiguous and 16-byte aligned, q rows 8-byte aligned");
  CIN_CHECK_ARG(T * nb < (int64_t)1 << 31 && cdiv(rows, kThreads) < (int64_t)1 << 31,
                "moe_scatter_quant: too many tiles");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (T > 0) {
    const uint32_t ntiles = (uint32_t)(T * nb);
    const unsigned grid = grid_for(ntiles, kThreads / 8, 16384);
    if (N % 128 == 0)
      launch_rowwise128_t<8, 1, true, kMapScatter>(x, x_dtype, N, sxm, round_scale, q, sqm, scales,
                                                   ssm, ssk, (uint32_t)nb, ntiles, grid, s, inv, k, rows);
    else
      launch_rowwise128_t<8, 1, false, kMapScatter>(x, x_dtype, N, sxm, round_scale, q, sqm, scales,
                                                    ssm, ssk, (uint32_t)nb, ntiles, grid, s, inv, k, rows);
  }
  if (rows > 0)
    hipLaunchKernelGGL(k_zero_unrouted, (unsigned)cdiv(rows, kThreads), kThreads, 0, s, perm, rows, N,
                       x_dtype, round_scale, q, sqm, scales, ssm, ssk);
  return cin_check_launch("moe_scatter_quant_rowwise");
}

int cin_moe_scatter_quant_rowwise_ws(const void* x, int x_dtype, int64_t T, int64_t N, int64_t sxm,
                                     const int32_t* inv, int64_t k, const int64_t* perm, int64_t rows,
                                     int round_scale, uint8_t* q, int64_t sqm, float* scales,
                                     int64_t ssm, int64_t ssk, float* ws, void* stream) {
  CIN_CHECK_ARG(valid_dtype(x_dtype), "moe_scatter_quant_ws: unsupported x dtype %d", x_dtype);
  CIN_CHECK_ARG(T >= 0 && N >= 0 && rows >= 0 && k >= 1, "moe_scatter_quant_ws: bad sizes");
  if (N == 0 || (T == 0 && rows == 0)) return CIN_OK;
  CIN_CHECK_ARG(x && inv && perm && q && scales && ws, "moe_scatter_quant_ws: null pointer");
  CIN_CHECK_ARG(aligned(ws, 16), "moe_scatter_quant_ws: ws must be 16-byte aligned");
  const int64_t nb = cdiv(N, 128);
  CIN_CHECK_ARG(sqm >= N, "moe_scatter_quant_ws: output row stride too small");
  CIN_CHECK_ARG(scale_layout_ok(rows, nb, ssm, ssk), "moe_scatter_quant_ws: scale strides overlap");
  const int es = elem_size(x_dtype);
  CIN_CHECK_ARG(aligned(x, 16) && (sxm * es) % 16 == 0 && sxm >= N && aligned(q, 8) && sqm % 8 == 0,
                "moe_scatter_quant_ws: x rows must be contiguous and 16-byte aligned, q rows 8-byte aligned");
  CIN_CHECK_ARG(T * nb < (int64_t)1 << 31 && cdiv(rows, kThreads) < (int64_t)1 << 31,
                "moe_scatter_quant_ws: too many tiles");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (T > 0) {
    const uint32_t ntiles = (uint32_t)(T * nb);
    const unsigned grid = grid_for(ntiles, kThreads / 8, 16384);
    if (N % 128 == 0)
      launch_rowwise128_t<8, 1, true, kMapScatterTok>(x, x_dtype, N, sxm, round_scale, q, sqm, ws, nb, 1,
                                                      (uint32_t)nb, ntiles, grid, s, inv, k, rows);
    else
      launch_rowwise128_t<8, 1, false, kMapScatterTok>(x, x_dtype, N, sxm, round_scale, q, sqm, ws, nb, 1,
                                                       (uint32_t)nb, ntiles, grid, s, inv, k, rows);
  }
  if (rows > 0)
    hipLaunchKernelGGL(k_zero_unrouted, (unsigned)cdiv(rows, kThreads), kThreads, 0, s, perm, rows, N,
                       x_dtype, round_scale, q, sqm, scales, ssm, ssk, ws, k, T);
  return cin_check_launch("moe_scatter_quant_rowwise_ws");
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
  CIN_CHECK_ARG(nbm < 65536 && nbm * nbn < ((int64_t)1 << 31), "quant_blockwise: grid too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int es = elem_size(x_dtype);
  const bool fast = bm == 128 && bn == 128 && sxn == 1 && aligned(x, 16) &&
                    ((sxm * es) % 16 == 0) && tile_fits32(sxm * es) &&
                    (!q || (aligned(q, 8) && sqm % 8 == 0 && tile_fits32(sqm)));
  if (fast) {
    const int vec_t = qt && aligned(qt, 16) && sqtm % 16 == 0 && tile_fits32(sqtm);
    // column blocks 0 .. nfull-1 whole; the last one, when partial, in an EDGE launch
    const uint32_t nfull = (uint32_t)(N / 128), nrb = (uint32_t)nbm;
#define CIN_BLOCK128(DT, EDGE, NBC, CB0)                                                   \
  do {                                                                                     \
    const uint32_t nt = nrb * (NBC);                                                       \
    const unsigned grid_ = resident_grid<k_blockwise128<DT, EDGE>>(nt);                  \
    hipLaunchKernelGGL((k_blockwise128<DT, EDGE>), grid_,                                  \
                       kThreads, 0, s, x, M, N, sxm, round_scale, q, sqm, qt, sqtm, vec_t, scales, \
                       ssm,                                                                \
                       (uint32_t)(NBC), (uint32_t)(CB0), nt);                             \
  } while (0)
#define CIN_BLOCK128_ALL(DT)                                         \
  do {                                                               \
    if (nfull > 0) CIN_BLOCK128(DT, false, nfull, 0);                \
    if (N % 128 != 0) CIN_BLOCK128(DT, true, 1, nfull);              \
  } while (0)
    if (x_dtype == CIN_DT_BF16)
      CIN_BLOCK128_ALL(CIN_DT_BF16);
    else if (x_dtype == CIN_DT_F16)
      CIN_BLOCK128_ALL(CIN_DT_F16);
    else
      CIN_BLOCK128_ALL(CIN_DT_F32);
#undef CIN_BLOCK128_ALL
#undef CIN_BLOCK128
  } else {
    dim3 grid((unsigned)nbn, (unsigned)nbm);
    hipLaunchKernelGGL(k_blockwise_generic, grid, kThreads, 0, s, x, x_dtype, M, N, sxm, sxn, bm,
                       bn, round_scale, q, sqm, qt, sqtm, scales, ssm, nbn);
  }
  return cin_check_launch("quant_blockwise");
}

int cin_quant_fwd(const void* x, int x_dtype, int64_t M, int64_t K, int64_t sxm, int round_scale,
                  uint8_t* xq, int64_t sxqm, float* xs, int64_t sxsm, int64_t sxsk, const void* w,
                  int w_dtype, int64_t N, int64_t swm, uint8_t* wq, int64_t swqm, uint8_t* wqt,
                  int64_t swqtm, float* ws, int64_t swsm, void* stream) {
  CIN_CHECK_ARG(valid_dtype(x_dtype) && valid_dtype(w_dtype), "quant_fwd: unsupported dtype (x %d, w %d)",
                x_dtype, w_dtype);
  CIN_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "quant_fwd: negative shape");
  const int64_t nbk = cdiv(K, 128), nbn = cdiv(N, 128);
  // both halves are validated before anything is launched, so a rejected call writes nothing
  if (M > 0 && K > 0) {
    CIN_CHECK_ARG(x && xq && xs, "quant_fwd: null activation pointer");
    CIN_CHECK_ARG(sxqm >= K, "quant_fwd: activation output row stride too small");
    CIN_CHECK_ARG(scale_layout_ok(M, nbk, sxsm, sxsk), "quant_fwd: activation scale strides overlap");
  }
  if (N > 0 && K > 0) {
    CIN_CHECK_ARG(w && ws && (wq || wqt), "quant_fwd: null weight pointer");
    CIN_CHECK_ARG((!wq || swqm >= K) && (!wqt || swqtm >= N) && swsm >= nbk,
                  "quant_fwd: weight output row stride too small");
    CIN_CHECK_ARG(nbn < 65536 && nbn * nbk < ((int64_t)1 << 31), "quant_fwd: weight grid too large");
  }
  const int xes = elem_size(x_dtype), wes = elem_size(w_dtype);
  const bool fuse = M > 0 && N > 0 && K > 0 && K % 128 == 0 && w_dtype != CIN_DT_F32 && x && xq && xs &&
                    w && ws && (wq || wqt) && aligned(x, 16) && (sxm * xes) % 16 == 0 && sxm >= K &&
                    aligned(xq, 8) && sxqm % 8 == 0 && sxqm >= K && M * nbk < ((int64_t)1 << 31) &&
                    aligned(w, 16) && (swm * wes) % 16 == 0 && swm >= K && tile_fits32(swm * wes) &&
                    (!wq || (aligned(wq, 8) && swqm % 8 == 0 && swqm >= K && tile_fits32(swqm))) &&
                    (!wqt || swqtm >= N) && swsm >= nbk && nbn < 65536 && nbn * nbk <= ((int64_t)1 << 22);
  if (!fuse) {
    // any other shape, dtype or layout: the two quantizers one after the other
    const int rc = cin_quant_rowwise(x, x_dtype, M, K, sxm, 1, 128, round_scale, xq, sxqm, xs, sxsm, sxsk,
                                     stream);
    if (rc != CIN_OK) return rc;
    return cin_quant_blockwise(w, w_dtype, N, K, swm, 1, 128, 128, 0, wq, swqm, wqt, swqtm, ws, swsm, stream);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint32_t xtiles = (uint32_t)(M * nbk), wtiles = (uint32_t)(nbn * nbk);
  const int wvec_t = wqt && aligned(wqt, 16) && swqtm % 16 == 0 && tile_fits32(swqtm);
  const unsigned gx = grid_for(xtiles, (kThreads / 8) * kFwdXU, 16384);
  const unsigned grid = gx + wtiles;
#define CIN_QFWD(XT, WT)                                                                                   \
  hipLaunchKernelGGL((k_quant_fwd<XT, WT>), grid, kThreads, 0, s, x, K, sxm, round_scale, xq, sxqm, xs, sxsm, sxsk, \
                     (uint32_t)nbk, xtiles, w, N, K, swm, wq, swqm, wqt, swqtm, wvec_t, ws, swsm,            \
                     (uint32_t)nbk, wtiles, wtiles)
#define CIN_QFWD_X(WT)                                    \
  if (x_dtype == CIN_DT_BF16) CIN_QFWD(CIN_DT_BF16, WT);  \
  else if (x_dtype == CIN_DT_F16) CIN_QFWD(CIN_DT_F16, WT); \
  else CIN_QFWD(CIN_DT_F32, WT);
  if (w_dtype == CIN_DT_BF16) {
    CIN_QFWD_X(CIN_DT_BF16)
  } else {
    CIN_QFWD_X(CIN_DT_F16)
  }
#undef CIN_QFWD_X
#undef CIN_QFWD
  return cin_check_launch("quant_fwd");
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
                   int round_scale, uint8_t* q, int64_t sqm, float* s, int64_t ssm, int64_t ssk,
                   uint8_t* qt, int64_t sqtm, float* st, int64_t sstm, int64_t sstk, void* stream) {
  CIN_CHECK_ARG(valid_dtype(dy_dtype), "quant_dual: unsupported dtype %d", dy_dtype);
  CIN_CHECK_ARG(M >= 0 && N >= 0, "quant_dual: negative shape");
  if (M == 0 || N == 0) return CIN_OK;
  CIN_CHECK_ARG(dy && q && s && qt && st, "quant_dual: null pointer");
  CIN_CHECK_ARG(sqm >= N && sqtm >= M, "quant_dual: output row stride too small");
  CIN_CHECK_ARG(scale_layout_ok(M, cdiv(N, 128), ssm, ssk) && scale_layout_ok(N, cdiv(M, 128), sstm, sstk),
                "quant_dual: scale strides overlap");
  hipStream_t stream_ = static_cast<hipStream_t>(stream);
  const int es = elem_size(dy_dtype);
  const bool fast = sdn == 1 && aligned(dy, 16) && ((sdm * es) % 16 == 0) && aligned(q, 8) &&
                    sqm % 8 == 0 && tile_fits32(sdm * es) && tile_fits32(sqm) &&
                    cdiv(M, 128) * cdiv(N, 128) < ((int64_t)1 << 31);
  if (fast) {
    const int vec_t = aligned(qt, 16) && sqtm % 16 == 0 && tile_fits32(sqtm);
    const uint32_t nfull = (uint32_t)(N / 128), nrb = (uint32_t)cdiv(M, 128);
#define CIN_DUAL128(DT, EDGE, NBC, CB0)                                                        \
  do {                                                                                         \
    const uint32_t nt = nrb * (NBC);                                                           \
    const unsigned grid_ = resident_grid<k_dual128<DT, EDGE>>(nt);                             \
    hipLaunchKernelGGL((k_dual128<DT, EDGE>), grid_, kThreads, 0,                              \
                       stream_, dy, M, N, sdm, round_scale, q, sqm, s, ssm, ssk, qt, sqtm, vec_t, \
                       st, sstm, sstk,                                                         \
                       (uint32_t)(NBC), (uint32_t)(CB0), nt);                                  \
  } while (0)
#define CIN_DUAL128_ALL(DT)                                   \
  do {                                                        \
    if (nfull > 0) CIN_DUAL128(DT, false, nfull, 0);          \
    if (N % 128 != 0) CIN_DUAL128(DT, true, 1, nfull);        \
  } while (0)
    if (dy_dtype == CIN_DT_BF16)
      CIN_DUAL128_ALL(CIN_DT_BF16);
    else if (dy_dtype == CIN_DT_F16)
      CIN_DUAL128_ALL(CIN_DT_F16);
    else
      CIN_DUAL128_ALL(CIN_DT_F32);
#undef CIN_DUAL128_ALL
#undef CIN_DUAL128
    return cin_check_launch("quant_dual");
  }
  // Strided input: two generic row-wise passes (dy, then dy^T through strides).
  int rc = cin_quant_rowwise(dy, dy_dtype, M, N, sdm, sdn, 128, round_scale, q, sqm, s, ssm, ssk, stream);
  if (rc != CIN_OK) return rc;
  return cin_quant_rowwise(dy, dy_dtype, N, M, sdn, sdm, 128, round_scale, qt, sqtm, st, sstm, sstk,
                           stream);
}

int cin_quant_dual_grouped(const void* dy, int dy_dtype, int64_t T, int64_t N, int64_t sdm,
                           const int64_t* starts, const int64_t* ends, int64_t E, int round_scale,
                           uint8_t* q, int64_t sqm, float* s, int64_t ssm, int64_t ssk, uint8_t* qt,
                           int64_t sqtm, float* st, int64_t sstm, int64_t sstk, void* stream) {
  CIN_CHECK_ARG(valid_dtype(dy_dtype), "quant_dual_grouped: unsupported dtype %d", dy_dtype);
  CIN_CHECK_ARG(T >= 0 && N >= 0 && E >= 0, "quant_dual_grouped: negative shape");
  if (T == 0 || N == 0 || E == 0) return CIN_OK;
  CIN_CHECK_ARG(dy && q && s && qt && st && starts && ends, "quant_dual_grouped: null pointer");
  const int es = elem_size(dy_dtype);
  CIN_CHECK_ARG(aligned(dy, 16) && (sdm * es) % 16 == 0 && sdm >= N,
                "quant_dual_grouped: dy rows must be contiguous and 16-byte aligned");
  CIN_CHECK_ARG(aligned(q, 8) && sqm % 8 == 0 && sqm >= N && scale_layout_ok(T, cdiv(N, 128), ssm, ssk),
                "quant_dual_grouped: bad row-wise outputs");
  CIN_CHECK_ARG(sqtm >= 128 && scale_layout_ok(N, sqtm / 128, sstm, sstk),
                "quant_dual_grouped: transposed rows must hold the padded token axis");
  CIN_CHECK_ARG((cdiv(T, 128) + E) * cdiv(N, 128) < ((int64_t)1 << 31),
                "quant_dual_grouped: too many tiles");
  CIN_CHECK_ARG(tile_fits32(sdm * es) && tile_fits32(sqm) && tile_fits32(sqtm),
                "quant_dual_grouped: row strides too large");
  const int vec_t = aligned(qt, 16) && sqtm % 16 == 0;
  hipStream_t stream_ = static_cast<hipStream_t>(stream);
  const uint32_t nfull = (uint32_t)(N / 128), nch = (uint32_t)(cdiv(T, 128) + E);
#define CIN_DUALG(DT, EDGE, NBC, CB0)                                                           \
  do {                                                                                          \
    const uint32_t nt = nch * (NBC);                                                            \
    const unsigned grid_ = resident_grid<k_dual128_grouped<DT, EDGE>>(nt);                      \
    hipLaunchKernelGGL((k_dual128_grouped<DT, EDGE>), grid_,                                    \
                       kThreads, 0, stream_, dy, T, N, sdm, round_scale, q, sqm, s, ssm, ssk, qt,  \
                       sqtm, vec_t, st, sstm, sstk, starts, ends, E, sqtm, (uint32_t)(NBC),        \
                       (uint32_t)(CB0), nt);                                                       \
  } while (0)
#define CIN_DUALG_ALL(DT)                                   \
  do {                                                      \
    if (nfull > 0) CIN_DUALG(DT, false, nfull, 0);          \
    if (N % 128 != 0) CIN_DUALG(DT, true, 1, nfull);        \
  } while (0)
  if (dy_dtype == CIN_DT_BF16)
    CIN_DUALG_ALL(CIN_DT_BF16);
  else if (dy_dtype == CIN_DT_F16)
    CIN_DUALG_ALL(CIN_DT_F16);
  else
    CIN_DUALG_ALL(CIN_DT_F32);
#undef CIN_DUALG_ALL
#undef CIN_DUALG
  return cin_check_launch("quant_dual_grouped");
}

int cin_swiglu_dual_grouped(const float* dh, int64_t sdm, const void* h12, int h12_dtype, int64_t s12,
                            int64_t T, int64_t H, const int64_t* starts, const int64_t* ends, int64_t E,
                            int round_scale, uint8_t* q, int64_t sqm, float* s, int64_t ssm, int64_t ssk,
                            uint8_t* qt, int64_t sqtm, float* st, int64_t sstm, int64_t sstk, void* stream) {
  CIN_CHECK_ARG(valid_dtype(h12_dtype), "swiglu_dual_grouped: unsupported h12 dtype %d", h12_dtype);
  CIN_CHECK_ARG(T >= 0 && H >= 0 && E >= 0, "swiglu_dual_grouped: negative shape");
  if (T == 0 || H == 0 || E == 0) return CIN_OK;
  CIN_CHECK_ARG(dh && h12 && q && s && qt && st && starts && ends, "swiglu_dual_grouped: null pointer");
  CIN_CHECK_ARG(H % 128 == 0, "swiglu_dual_grouped: H (%lld) must be a multiple of 128", (long long)H);
  const int es = elem_size(h12_dtype);
  const int64_t N = 2 * H;
  CIN_CHECK_ARG(aligned(dh, 16) && (sdm * 4) % 16 == 0 && sdm >= H && aligned(h12, 16) &&
                    (s12 * es) % 16 == 0 && s12 >= N,
                "swiglu_dual_grouped: dh and h12 rows must be contiguous and 16-byte aligned");
  CIN_CHECK_ARG(aligned(q, 8) && sqm % 8 == 0 && sqm >= N && scale_layout_ok(T, N / 128, ssm, ssk),
                "swiglu_dual_grouped: bad row-wise outputs");
  CIN_CHECK_ARG(sqtm >= 128 && scale_layout_ok(N, sqtm / 128, sstm, sstk),
                "swiglu_dual_grouped: transposed rows must hold the padded token axis");
  CIN_CHECK_ARG((cdiv(T, 128) + E) * (H / 128) < ((int64_t)1 << 31), "swiglu_dual_grouped: too many tiles");
  CIN_CHECK_ARG(tile_fits32(sdm * 4) && tile_fits32(s12 * es) && tile_fits32(sqm) && tile_fits32(sqtm),
                "swiglu_dual_grouped: row strides too large");
  const int vec_t = aligned(qt, 16) && sqtm % 16 == 0;
  const uint32_t nbh = (uint32_t)(H / 128), nt = (uint32_t)(cdiv(T, 128) + E) * nbh;
  hipStream_t stream_ = static_cast<hipStream_t>(stream);
#define CIN_SWID(IT)                                                                                   \
  hipLaunchKernelGGL((k_swiglu_dual128_grouped<IT>), resident_grid<k_swiglu_dual128_grouped<IT>>(nt),  \
                     kThreads, 0, stream_, dh, sdm, h12, s12, T, H, round_scale, q, sqm, s, ssm, ssk, qt,  \
                     sqtm, vec_t, st, sstm, sstk, starts, ends, E, sqtm, nbh, nt)
  if (h12_dtype == CIN_DT_BF16)
    CIN_SWID(CIN_DT_BF16);
  else if (h12_dtype == CIN_DT_F16)
    CIN_SWID(CIN_DT_F16);
  else
    CIN_SWID(CIN_DT_F32);
#undef CIN_SWID
  return cin_check_launch("swiglu_dual_grouped");
}

int cin_requant_row_to_block_grouped(const uint8_t* q, int64_t T, int64_t K, int64_t sqm,
                                     const float* srow, int64_t ssm, int64_t ssk,
                                     const int64_t* starts, const int64_t* ends, int64_t E,
                                     uint8_t* qbt, int64_t sqbtm, float* sblk, int64_t ssbm,
                                     void* stream) {
  CIN_CHECK_ARG(T >= 0 && K >= 0 && E >= 0, "requant_grouped: negative shape");
  if (T == 0 || K == 0 || E == 0) return CIN_OK;
  CIN_CHECK_ARG(q && srow && qbt && sblk && starts && ends, "requant_grouped: null pointer");
  CIN_CHECK_ARG(aligned(q, 8) && sqm % 8 == 0 && sqm >= K, "requant_grouped: q must be 8-byte aligned rows");
  CIN_CHECK_ARG(sqbtm >= 128 && scale_layout_ok(T, cdiv(K, 128), ssm, ssk) && ssbm >= cdiv(K, 128),
                "requant_grouped: bad output strides");
  CIN_CHECK_ARG((cdiv(T, 128) + E) * cdiv(K, 128) < ((int64_t)1 << 31),
                "requant_grouped: too many tiles");
  CIN_CHECK_ARG(tile_fits32(sqm) && tile_fits32(ssm * 4) && tile_fits32(sqbtm),
                "requant_grouped: row strides too large");
  const int vec_t = aligned(qbt, 16) && sqbtm % 16 == 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint32_t nfull = (uint32_t)(K / 128), nch = (uint32_t)(cdiv(T, 128) + E);
#define CIN_REQG(EDGE, NBC, CB0)                                                                  \
  do {                                                                                            \
    const uint32_t nt = nch * (NBC);                                                              \
    const unsigned grid_ = resident_grid<k_requant128_grouped<EDGE>>(nt);                         \
    hipLaunchKernelGGL(k_requant128_grouped<EDGE>, grid_,                                         \
                       kThreads, 0, s, q, T, K, sqm, srow, ssm, ssk, (uint8_t*)nullptr, (int64_t)0, qbt, \
                       sqbtm, vec_t, sblk, ssbm, starts, ends, E, sqbtm, (uint32_t)(NBC),         \
                       (uint32_t)(CB0), nt);                                                        \
  } while (0)
  if (nfull > 0) CIN_REQG(false, nfull, 0);
  if (K % 128 != 0) CIN_REQG(true, 1, nfull);
#undef CIN_REQG
  return cin_check_launch("requant_row_to_block_grouped");
}

int cin_requant_row_to_block(const uint8_t* q, int64_t M, int64_t K, int64_t sqm,
                             const float* srow, int64_t ssm, int64_t ssk, uint8_t* qb,
                             int64_t sqbm, uint8_t* qbt, int64_t sqbtm, float* sblk, int64_t ssbm,
                             void* stream) {
  CIN_CHECK_ARG(M >= 0 && K >= 0, "requant: negative shape");
  if (M == 0 || K == 0) return CIN_OK;
  CIN_CHECK_ARG(q && srow && sblk && (qb || qbt), "requant: null pointer");
  CIN_CHECK_ARG(aligned(q, 8) && sqm % 8 == 0, "requant: q must be 8-byte aligned rows");
  CIN_CHECK_ARG(!qb || (aligned(qb, 8) && sqbm % 8 == 0 && sqbm >= K),
                "requant: qb must be 8-byte aligned rows");
  CIN_CHECK_ARG(!qbt || sqbtm >= M, "requant: qbt row stride too small");
  CIN_CHECK_ARG(scale_layout_ok(M, cdiv(K, 128), ssm, ssk) && ssbm >= cdiv(K, 128), "requant: bad scale stride");
  CIN_CHECK_ARG(cdiv(M, 128) * cdiv(K, 128) < ((int64_t)1 << 31), "requant: too many tiles");
  CIN_CHECK_ARG(tile_fits32(sqm) && tile_fits32(ssm * 4) && (!qb || tile_fits32(sqbm)),
                "requant: row strides too large");
  const int vec_t = qbt && aligned(qbt, 16) && sqbtm % 16 == 0 && tile_fits32(sqbtm);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint32_t nfull = (uint32_t)(K / 128), nrb = (uint32_t)cdiv(M, 128);
#define CIN_REQ(EDGE, NBC, CB0)                                                                 \
  do {                                                                                          \
    const uint32_t nt = nrb * (NBC);                                                            \
    const unsigned grid_ = resident_grid<k_requant128<EDGE>>(nt);                               \
    hipLaunchKernelGGL(k_requant128<EDGE>, grid_, kThreads, 0, s, q,                            \
                       M, K, sqm, srow, ssm, ssk, qb, sqbm, qbt, sqbtm, vec_t, sblk, ssbm, (uint32_t)(NBC), \
                       (uint32_t)(CB0), nt);                                                    \
  } while (0)
  if (nfull > 0) CIN_REQ(false, nfull, 0);
  if (K % 128 != 0) CIN_REQ(true, 1, nfull);
#undef CIN_REQ
  return cin_check_launch("requant_row_to_block");
}

int cin_quant_backward(const void* dy, int dy_dtype, int64_t M, int64_t N, int64_t sdm,
                       int round_scale, uint8_t* q, int64_t sqm, float* s, int64_t ssm, int64_t ssk,
                       uint8_t* qt, int64_t sqtm, float* st, int64_t sstm, int64_t sstk,
                       const uint8_t* xq, int64_t K, int64_t sxqm, const float* xs, int64_t sxsm,
                       int64_t sxsk, uint8_t* xbt, int64_t sxbtm, float* sblk, int64_t ssbm,
                       void* stream) {
  CIN_CHECK_ARG(valid_dtype(dy_dtype), "quant_backward: unsupported dtype %d", dy_dtype);
  CIN_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "quant_backward: negative shape");
  if (M == 0 || (N == 0 && K == 0)) return CIN_OK;
  CIN_CHECK_ARG(dy && q && s && qt && st && xq && xs && xbt && sblk, "quant_backward: null pointer");
  CIN_CHECK_ARG(sqm >= N && sqtm >= M && scale_layout_ok(M, cdiv(N, 128), ssm, ssk) &&
                    scale_layout_ok(N, cdiv(M, 128), sstm, sstk),
                "quant_backward: dY output row stride too small or scale strides overlap");
  CIN_CHECK_ARG(aligned(xq, 8) && sxqm % 8 == 0 && sxqm >= K && scale_layout_ok(M, cdiv(K, 128), sxsm, sxsk) &&
                    sxbtm >= M && ssbm >= cdiv(K, 128),
                "quant_backward: bad X codes, scales or outputs");
  const int es = elem_size(dy_dtype);
  // one launch: 16-bit dY and both widths whole 128-column blocks, with the layouts the two
  // kernels' fast paths take
  const bool pair = (dy_dtype == CIN_DT_BF16 || dy_dtype == CIN_DT_F16) && N > 0 && K > 0 &&
                    N % 128 == 0 && K % 128 == 0 && aligned(dy, 16) && (sdm * es) % 16 == 0 &&
                    sdm >= N && aligned(q, 8) && sqm % 8 == 0 && tile_fits32(sdm * es) &&
                    tile_fits32(sqm) && tile_fits32(sxqm) && tile_fits32(sxsm * 4) &&
                    cdiv(M, 128) * (N / 128 + K / 128) < ((int64_t)1 << 31);
  if (!pair) {
    int rc = cin_quant_dual(dy, dy_dtype, M, N, sdm, 1, round_scale, q, sqm, s, ssm, ssk, qt, sqtm, st,
                            sstm, sstk, stream);
    if (rc != CIN_OK) return rc;
    return cin_requant_row_to_block(xq, M, K, sxqm, xs, sxsm, sxsk, nullptr, 0, xbt, sxbtm, sblk, ssbm,
                                    stream);
  }
  const int dvec_t = aligned(qt, 16) && sqtm % 16 == 0 && tile_fits32(sqtm);
  const int rvec_t = aligned(xbt, 16) && sxbtm % 16 == 0 && tile_fits32(sxbtm);
  const uint32_t nrb = (uint32_t)cdiv(M, 128);
  const uint32_t nd = nrb * (uint32_t)(N / 128), nt = nd + nrb * (uint32_t)(K / 128);
  hipStream_t stream_ = static_cast<hipStream_t>(stream);
#define CIN_QBWD(DT)                                                                               \
  hipLaunchKernelGGL((k_quant_bwd<DT>), resident_grid<k_quant_bwd<DT>>(nt), kThreads, 0, stream_, dy, \
                     M, N, sdm, round_scale, q, sqm, s, ssm, ssk, qt, sqtm, dvec_t, st, sstm, sstk, xq, K, \
                     sxqm, xs, sxsm, sxsk, xbt, sxbtm, rvec_t, sblk, ssbm, nd, nt)
  if (dy_dtype == CIN_DT_BF16)
    CIN_QBWD(CIN_DT_BF16);
  else
    CIN_QBWD(CIN_DT_F16);
#undef CIN_QBWD
  return cin_check_launch("quant_backward");
}

int cin_silu_mul_quant_rowwise(const void* h12, int in_dtype, int64_t M, int64_t H, int64_t s12,
                               int out_dtype, int round_scale, uint8_t* q, int64_t sqm,
                               float* scales, int64_t ssm, int64_t ssk, void* stream) {
  CIN_CHECK_ARG(valid_dtype(in_dtype) && valid_dtype(out_dtype), "silu_mul_quant: unsupported dtype");
  CIN_CHECK_ARG(M >= 0 && H >= 0, "silu_mul_quant: negative shape");
  if (M == 0 || H == 0) return CIN_OK;
  CIN_CHECK_ARG(h12 && q && scales, "silu_mul_quant: null pointer");
  const int es = elem_size(in_dtype);
  CIN_CHECK_ARG(aligned(h12, 16) && (s12 * es) % 16 == 0 && (H * es) % 16 == 0 && s12 >= 2 * H,
                "silu_mul_quant: h12 rows must hold 2H elements at 16-byte aligned offsets");
  CIN_CHECK_ARG(aligned(q, 8) && sqm % 8 == 0 && sqm >= H && scale_layout_ok(M, cdiv(H, 128), ssm, ssk),
                "silu_mul_quant: bad outputs");
  const int64_t nb = cdiv(H, 128);
  CIN_CHECK_ARG(M * nb < ((int64_t)1 << 31), "silu_mul_quant: too many tiles");
  const uint32_t ntiles = (uint32_t)(M * nb);
  const unsigned grid = grid_for(ntiles, kThreads / 16, 16384);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define CIN_SILU(IT, OT)                                                                        \
  hipLaunchKernelGGL((k_silu_mul_rowwise128<IT, OT>), grid, kThreads, 0, s, h12, s12, H,         \
                     round_scale, q, sqm, scales, ssm, ssk, (uint32_t)nb, ntiles)
#define CIN_SILU_OT(IT)                                                                         \
  do {                                                                                          \
    if (out_dtype == CIN_DT_BF16) CIN_SILU(IT, CIN_DT_BF16);                                    \
    else if (out_dtype == CIN_DT_F16) CIN_SILU(IT, CIN_DT_F16);                                 \
    else CIN_SILU(IT, CIN_DT_F32);                                                              \
  } while (0)
  if (in_dtype == CIN_DT_BF16)
    CIN_SILU_OT(CIN_DT_BF16);
  else if (in_dtype == CIN_DT_F16)
    CIN_SILU_OT(CIN_DT_F16);
  else
    CIN_SILU_OT(CIN_DT_F32);
#undef CIN_SILU_OT
#undef CIN_SILU
  return cin_check_launch("silu_mul_quant_rowwise");
}

int cin_swiglu_backward(const float* dh, int64_t sdm, const void* h12, int h12_dtype, int64_t s12,
                        int64_t M, int64_t H, float* dh12, int64_t som, void* stream) {
  CIN_CHECK_ARG(valid_dtype(h12_dtype), "swiglu_backward: unsupported h12 dtype %d", h12_dtype);
  CIN_CHECK_ARG(M >= 0 && H >= 0, "swiglu_backward: negative shape");
  if (M == 0 || H == 0) return CIN_OK;
  CIN_CHECK_ARG(dh && h12 && dh12, "swiglu_backward: null pointer");
  CIN_CHECK_ARG(H % 4 == 0 && aligned(dh, 16) && sdm % 4 == 0 && sdm >= H && aligned(dh12, 16) &&
                    som % 4 == 0 && som >= 2 * H && s12 >= 2 * H,
                "swiglu_backward: H must be a multiple of 4 with 16-byte aligned fp32 rows");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = grid_for(M * (H / 4), kThreads, 65536);
  if (h12_dtype == CIN_DT_BF16)
    hipLaunchKernelGGL(k_swiglu_backward<CIN_DT_BF16>, grid, kThreads, 0, s, dh, sdm, h12, s12, M, H,
                       dh12, som);
  else if (h12_dtype == CIN_DT_F16)
    hipLaunchKernelGGL(k_swiglu_backward<CIN_DT_F16>, grid, kThreads, 0, s, dh, sdm, h12, s12, M, H,
                       dh12, som);
  else
    hipLaunchKernelGGL(k_swiglu_backward<CIN_DT_F32>, grid, kThreads, 0, s, dh, sdm, h12, s12, M, H,
                       dh12, som);
  return cin_check_launch("swiglu_backward");
}

int cin_zero_rows_outside_ranges(void* C, int64_t ldc_bytes, int64_t row_bytes, int64_t T,
                                 const int64_t* starts, const int64_t* ends, int64_t E,
                                 void* stream) {
  CIN_CHECK_ARG(T >= 0 && E >= 0 && row_bytes >= 0 && ldc_bytes >= row_bytes,
                "zero_rows_outside_ranges: bad shape");
  if (T == 0 || row_bytes == 0) return CIN_OK;
  CIN_CHECK_ARG(C && (E == 0 || (starts && ends)), "zero_rows_outside_ranges: null pointer");
  CIN_CHECK_ARG(cdiv(T, kThreads) < ((int64_t)1 << 31), "zero_rows_outside_ranges: too many rows");
  hipLaunchKernelGGL(k_zero_uncovered, (unsigned)cdiv(T, kThreads), kThreads, 0,
                     static_cast<hipStream_t>(stream), static_cast<uint8_t*>(C), ldc_bytes,
                     row_bytes, T, starts, ends, E);
  return cin_check_launch("zero_rows_outside_ranges");
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
