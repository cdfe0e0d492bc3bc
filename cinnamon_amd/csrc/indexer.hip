// DSA indexer scoring on FP8 q / k codes (reference src/attention.py:288-300):
//
//   scores[b, t, s] = k_scale[b, s] * sum_h relu(sum_d q8[b, t, h, d] k8[b, s, d]) * w'[b, t, h]
//   w'[b, t, h]     = (q_scale[b, t, h] * weights[b, t, h]) * softmax_scale
//
// The reference materialises the fp32 logits [B, L, H, S] (einsum of the dequantised codes)
// before the ReLU, the weighting and the head sum.  Here nothing but the scores leaves the
// chip.  A workgroup owns 64 tokens x 512 keys (4 waves of 16 tokens):
//   - the keys stream through LDS in sub-tiles of 128 rows, double buffered: the next
//     sub-tile's global loads (codes and k_scale) are in flight while the current one is
//     multiplied; rows are padded to d + 16 bytes so the 16 lanes of a 16-byte LDS read hit
//     16 distinct bank groups (d / 16 + 1 is odd for every d that is a multiple of 32);
//   - each wave keeps its tokens' q fragments for up to HG heads in registers for the whole
//     key range;
//   - one v_mfma_f32_16x16x128_f8f6f4 per (16 keys x 16 tokens, head, 128-byte slice of d)
//     is issued keys-first, so a lane ends up with 4 consecutive keys of one token; the
//     ReLU, the head weight and the head sum happen in registers (no cross-lane traffic),
//     the head sum in increasing head order;
//   - the 16 x 128 fp32 block of a wave is staged through LDS and written as 512-byte row
//     segments with non-temporal stores (the scores are consumed by a later top-k, not by
//     this kernel's caches).
// Consecutive workgroups share a batch row of keys; the tile order is rotated so that the
// eight XCDs (round-robin workgroup placement) each get a contiguous range of tiles, and a
// batch's keys stay in one XCD's L2.
// The products of two e4m3 codes are exact; the 128-product sums of the MFMA are not exact
// fp32 sums (measured within 2.2e-5 of the largest score at the indexer's shapes).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cin_common.h"
#include "cin_runtime.h"

using namespace cin;

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));

constexpr int kThreads = 256;  // 4 waves, 16 tokens each
constexpr int kTT = 64;        // tokens per workgroup
constexpr int kKT = 128;       // keys per LDS sub-tile
constexpr int64_t kKPW = 512;  // keys per workgroup

// 32 bytes at byte offset 128 c + 32 kq of a d-byte row, zero past d or when !ok.
template <int D>
__device__ inline v8i frag32(const uint8_t* row, bool ok, int kq, int c) {
  v8i v = {0, 0, 0, 0, 0, 0, 0, 0};
  const int off = c * 128 + 32 * kq;
  if (ok && off < D) {
    const uint4 lo = *reinterpret_cast<const uint4*>(row + off);
    const uint4 hi = *reinterpret_cast<const uint4*>(row + off + 16);
    v[0] = (int)lo.x; v[1] = (int)lo.y; v[2] = (int)lo.z; v[3] = (int)lo.w;
    v[4] = (int)hi.x; v[5] = (int)hi.y; v[6] = (int)hi.z; v[7] = (int)hi.w;
  }
  return v;
}

// Waves per SIMD the register allocation aims for: two workgroups per CU fit in LDS up to
// d = 160 (2 x (2 key buffers + staging) <= 160 KB), one beyond.
template <int D>
constexpr int kMinWaves = D <= 160 ? 2 : 1;

// Workgroup -> (batch, 64-token tile, 512-key range).  With xcd_rotate (grid a multiple of
// 8) XCD x = blockIdx % 8 runs the contiguous tiles [x n/8, (x+1) n/8).
struct Tile {
  int64_t b, tt, sw, s_begin, s_end;
  int nsub;
};

__device__ inline Tile tile_of(int64_t S, int64_t tiles_t, int64_t tiles_s, int xcd_rotate) {
  int64_t tile = blockIdx.x;
  if (xcd_rotate) {
    const int64_t per = gridDim.x >> 3;
    tile = (tile & 7) * per + (tile >> 3);
  }
  Tile t;
  t.b = tile / (tiles_t * tiles_s);
  const int64_t rem = tile - t.b * tiles_t * tiles_s;
  t.tt = rem / tiles_s;
  t.sw = rem - t.tt * tiles_s;
  t.s_begin = t.sw * kKPW;
  t.s_end = t.s_begin + kKPW < S ? t.s_begin + kKPW : S;
  t.nsub = (int)((t.s_end - t.s_begin + kKT - 1) / kKT);
  return t;
}

// One 128-key sub-tile of codes and k_scale: global -> registers (issued early) -> LDS rows
// of d + 16 bytes (the 16 lanes of a 16-byte fragment read hit 16 distinct bank groups,
// d / 16 + 1 being odd).  Keys past the range read as zero.
template <int D>
struct KeyStage {
  static constexpr int RS = D + 16;
  static constexpr int CH = D / 16;
  static constexpr int PER = (kKT * CH + kThreads - 1) / kThreads;
  uint4 pre[PER];
  v4f kpre;

  __device__ void load(const uint8_t* k8, const float* ks, int64_t b, int64_t S, int64_t s_sub,
                       int64_t s_end, int vec, int tid = -1) {
    if (tid < 0) tid = threadIdx.x;  // tid: this thread's index among the 256 that share the stage
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int idx = tid + u * kThreads;
      const int row = idx / CH, c = idx - row * CH;
      const int64_t s = s_sub + row;
      pre[u] = uint4{0u, 0u, 0u, 0u};
      if (idx < kKT * CH && s < s_end) pre[u] = *reinterpret_cast<const uint4*>(k8 + (b * S + s) * D + 16 * c);
    }
    kpre = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    if (tid < kKT / 4) {
      const int64_t s0 = s_sub + 4 * tid;
      if (vec && s0 + 4 <= s_end) {
        kpre = *reinterpret_cast<const v4f*>(ks + b * S + s0);
      } else {
        for (int r = 0; r < 4; ++r)
          if (s0 + r < s_end) kpre[r] = ks[b * S + s0 + r];
      }
    }
  }
  __device__ void store(uint8_t* kl, float* ksl, int tid = -1) const {
    if (tid < 0) tid = threadIdx.x;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int idx = tid + u * kThreads;
      const int row = idx / CH, c = idx - row * CH;
      if (idx < kKT * CH) *reinterpret_cast<uint4*>(&kl[row * RS + 16 * c]) = pre[u];
    }
    if (tid < kKT / 4) *reinterpret_cast<v4f*>(&ksl[4 * tid]) = kpre;
  }
};

// D = head dim (multiple of 32, <= 256), HG = heads whose q fragments are held at once.
// vec: k_scale and scores rows are 16-byte aligned (S % 4 == 0 and aligned bases).
// max(x, 0) as one integer max of the bits (negative floats, -0 included, are negative
// int32s, so they become +0; non-negative ones keep their bits): fmaxf also quiets a
// signalling NaN first, two instructions per value.  The logits here are finite.
__device__ __forceinline__ float relu1(float x) {
  return __int_as_float(max(__float_as_int(x), 0));
}

// The fused form's q quantization.  Lane (l16, kq) holds bytes [128 c + 32 kq, + 32) of each
// of its token's head rows (the MFMA's B-operand layout), so a 1 x 128 tile of a row lies in
// the four lanes l16, l16 + 16, l16 + 32, l16 + 48.  The arithmetic is the row-wise
// quantizer's (k_rowwise128 with 1 x 128 tiles: maxnum of |x| from 0, the fp32(1e-4) floor,
// amax / 448, RN(x / scale) clamped to +-448, e4m3 RNE), so codes and scales are the ones
// cin_indexer_quantize writes.  QDT is the input dtype.
template <int QDT>
struct RawSlice {
  static constexpr int ES = QDT == CIN_DT_F32 ? 4 : 2;
  static constexpr int NW = 32 * ES / 16;  // 16-byte words for 32 elements
  uint4 w[NW];
};

// 32 input elements at element offset 128 c + 32 kq of a d-element row, zero past d or when
// !ok (a zero slice leaves the tile's amax as it is).
template <int D, int QDT>
__device__ inline void load_slice(const void* row, bool ok, int kq, int c, RawSlice<QDT>& r) {
  const int off = c * 128 + 32 * kq;
#pragma unroll
  for (int i = 0; i < RawSlice<QDT>::NW; ++i) r.w[i] = uint4{0u, 0u, 0u, 0u};
  if (ok && off < D) {
    const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(row) +
                                                    (int64_t)off * RawSlice<QDT>::ES);
#pragma unroll
    for (int i = 0; i < RawSlice<QDT>::NW; ++i) r.w[i] = p[i];
  }
}

// Codes of a lane's 32 elements as the MFMA fragment, and the tile's scale.  Every lane of
// the wave calls it (the tile's amax is exchanged across lanes).
template <int QDT>
__device__ inline v8i quant_slice(const RawSlice<QDT>& r, float& scale) {
  float v[32];
#pragma unroll
  for (int i = 0; i < RawSlice<QDT>::NW; ++i) {
    const uint4 w = r.w[i];
    const uint32_t e[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (QDT == CIN_DT_F32) {
        v[4 * i + j] = __uint_as_float(e[j]);
      } else if constexpr (QDT == CIN_DT_BF16) {
        v[8 * i + 2 * j] = bf16_lo(e[j]);
        v[8 * i + 2 * j + 1] = bf16_hi(e[j]);
      } else {
        v[8 * i + 2 * j] = half_bits_to_f32(CIN_DT_F16, (uint16_t)(e[j] & 0xffffu));
        v[8 * i + 2 * j + 1] = half_bits_to_f32(CIN_DT_F16, (uint16_t)(e[j] >> 16));
      }
    }
  }
  float a = 0.0f;
  if constexpr (QDT == CIN_DT_F32) {
#pragma unroll
    for (int i = 0; i < 32; ++i) a = fmaxf(a, fabsf(v[i]));
  } else {
    // 16-bit inputs: the magnitudes' bit patterns order as unsigned integers (infinity
    // above every finite value, NaN above infinity), so two at a time with a packed 16-bit
    // max; a NaN among them sends the lane to maxnum, which skips NaNs.  Widening to fp32 is
    // exact and keeps the order, so the result is maxnum's.
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    u16x2 m = {0, 0};
#pragma unroll
    for (int i = 0; i < RawSlice<QDT>::NW; ++i) {
      const uint32_t e[4] = {r.w[i].x, r.w[i].y, r.w[i].z, r.w[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, e[j] & 0x7fff7fffu));
    }
    const uint32_t mag = m[0] > m[1] ? m[0] : m[1];
    constexpr uint32_t kInf = QDT == CIN_DT_BF16 ? 0x7f80u : 0x7c00u;
    if (mag <= kInf) {
      a = QDT == CIN_DT_BF16 ? __uint_as_float(mag << 16) : half_bits_to_f32(CIN_DT_F16, (uint16_t)mag);
    } else {
#pragma unroll
      for (int i = 0; i < 32; ++i) a = fmaxf(a, fabsf(v[i]));
    }
  }
  // a >= 0 and never NaN (maxnum from 0): the bit patterns order as unsigned integers
  uint32_t u = __float_as_uint(a);
  u = max(u, (uint32_t)__shfl_xor((int)u, 16));
  u = max(u, (uint32_t)__shfl_xor((int)u, 32));
  const float s = compute_scale(fmaxf(__uint_as_float(u), amax_floor(QDT)), false);
  uint32_t out[8];
  quant_vals<32, kDivSteps<QDT>>(v, s, 1.0f / s, out);
  scale = s;
  return v8i{(int)out[0], (int)out[1], (int)out[2], (int)out[3],
             (int)out[4], (int)out[5], (int)out[6], (int)out[7]};
}

// QDT < 0: q arrives as codes q8 with first scales qs.  QDT = an input dtype (the fused form):
// q arrives unquantized and each wave quantizes its own tokens' rows (H <= HG, so once per
// workgroup); when q8_out is not null the codes go to q8_out and the first scales to qs_out,
// each head's by one of the workgroups that share the tokens.
template <int D, int HG, int QDT = -1>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(kMinWaves<D>, 8))) void k_indexer_scores_fp8(
    const void* __restrict__ qin, const float* __restrict__ qs, const uint8_t* __restrict__ k8,
    const float* __restrict__ ks, const float* __restrict__ w, int64_t L, int64_t S, int64_t H,
    float softmax_scale, float* __restrict__ out, int64_t tiles_t, int64_t tiles_s, int xcd_rotate,
    int vec, uint8_t* __restrict__ q8_out = nullptr, float* __restrict__ qs_out = nullptr) {
  constexpr int NC = (D + 127) / 128;           // 128-byte slices of d
  constexpr int RS = KeyStage<D>::RS;
  constexpr int OS = kKT + 4;                   // staging row stride (floats)
  __shared__ __attribute__((aligned(16))) uint8_t kl[2][kKT * RS];
  __shared__ __attribute__((aligned(16))) float ksl[2][kKT];
  __shared__ __attribute__((aligned(16))) float ost[4 * 16 * OS];

  const Tile tl = tile_of(S, tiles_t, tiles_s, xcd_rotate);
  const int64_t b = tl.b;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int l16 = lane & 15, kq = lane >> 4;
  KeyStage<D> stage;

  // the wave's tokens: q fragments and head weights for HG heads
  const int64_t tok = tl.tt * kTT + wave * 16 + l16;
  const bool tok_ok = tok < L;
  const int64_t orow = (b * L + (tok_ok ? tok : 0)) * H;
  v8i qf[HG][NC];
  float wr[HG];
  auto load_q = [&](int64_t h0) {
    if constexpr (QDT < 0) {
      const uint8_t* qrow = static_cast<const uint8_t*>(qin) + orow * D;
#pragma unroll
      for (int g = 0; g < HG; ++g) {
        const bool ok = tok_ok && h0 + g < H;
#pragma unroll
        for (int c = 0; c < NC; ++c) qf[g][c] = frag32<D>(qrow + (h0 + g) * D, ok, kq, c);
        wr[g] = ok ? (qs[orow + h0 + g] * w[orow + h0 + g]) * softmax_scale : 0.0f;
      }
    }
  };
  // The fused form: q's rows as loaded (after the first key sub-tile's loads: issuing them
  // first measured slower), then quantized.
  constexpr int RW = QDT < 0 ? 1 : HG;
  constexpr int RC = QDT < 0 ? 1 : NC;
  RawSlice<QDT < 0 ? CIN_DT_BF16 : QDT> raw[RW][RC];
  float wv[RW];
  auto load_q_raw = [&]() {
    if constexpr (QDT >= 0) {
      const uint8_t* qrow = static_cast<const uint8_t*>(qin) + orow * D * RawSlice<QDT>::ES;
#pragma unroll
      for (int g = 0; g < HG; ++g) {
        const bool ok = tok_ok && g < H;
#pragma unroll
        for (int c = 0; c < NC; ++c)
          load_slice<D, QDT>(qrow + g * D * RawSlice<QDT>::ES, ok, kq, c, raw[g][c]);
        wv[g] = ok ? w[orow + g] : 0.0f;
      }
    }
  };
  auto quant_q = [&]() {
    if constexpr (QDT >= 0) {
      float s0[HG];
#pragma unroll
      for (int g = 0; g < HG; ++g) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          float sc;
          qf[g][c] = quant_slice<QDT>(raw[g][c], sc);
          if (c == 0) s0[g] = sc;
        }
        const bool ok = tok_ok && g < H;
        wr[g] = ok ? (s0[g] * wv[g]) * softmax_scale : 0.0f;
      }
      if (q8_out != nullptr) {
        // every workgroup of the 64 tokens holds all their codes: head h is written by the
        // one of key range h % tiles_s, so the writes spread over the ranges
#pragma unroll
        for (int g = 0; g < HG; ++g) {
          if (!(tok_ok && g < H) || g % tiles_s != tl.sw) continue;
          uint8_t* dst = q8_out + (orow + g) * D;
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const int off = c * 128 + 32 * kq;
            if (off < D) {
              const v8i f = qf[g][c];
              *reinterpret_cast<uint4*>(dst + off) = uint4{(uint32_t)f[0], (uint32_t)f[1], (uint32_t)f[2], (uint32_t)f[3]};
              *reinterpret_cast<uint4*>(dst + off + 16) = uint4{(uint32_t)f[4], (uint32_t)f[5], (uint32_t)f[6], (uint32_t)f[7]};
            }
          }
          if (kq == 0) qs_out[orow + g] = s0[g];
        }
      }
    }
  };
  const bool one_group = H <= HG;

  if constexpr (QDT < 0) {
    stage.load(k8, ks, b, S, tl.s_begin, tl.s_end, vec);
    load_q(0);
  } else {
    stage.load(k8, ks, b, S, tl.s_begin, tl.s_end, vec);
    load_q_raw();
    quant_q();
  }
  stage.store(kl[0], ksl[0]);
  __syncthreads();
  float* my = ost + wave * 16 * OS;
  for (int i = 0; i < tl.nsub; ++i) {
    const int buf = i & 1;
    if (i + 1 < tl.nsub) stage.load(k8, ks, b, S, tl.s_begin + (int64_t)(i + 1) * kKT, tl.s_end, vec);
    // Each 16-key tile's head sum goes straight to the wave's staging rows; a later head
    // group continues the sum from there (same increasing head order).  The staging rows
    // belong to this wave alone and a wave's LDS accesses complete in order, so no
    // workgroup barrier is needed around them.
    for (int64_t h0 = 0; h0 < H; h0 += HG) {
      if constexpr (QDT < 0) {
        if (!one_group) load_q(h0);
      }
      const bool first = h0 == 0, last = h0 + HG >= H;
#pragma unroll 2
      for (int j = 0; j < 8; ++j) {
        const uint8_t* kr = &kl[buf][(16 * j + l16) * RS];
        v8i kf[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) kf[c] = frag32<D>(kr, true, kq, c);
        v4f* slot = reinterpret_cast<v4f*>(&my[l16 * OS + 16 * j + 4 * kq]);
        v4f a = first ? v4f{0.0f, 0.0f, 0.0f, 0.0f} : *slot;
        // every head's MFMAs first, then the head sum in increasing head order: the MFMAs
        // run back to back instead of each waiting for its own result
        v4f p[HG];
#pragma unroll
        for (int g = 0; g < HG; ++g) {
          p[g] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int c = 0; c < NC; ++c)
            p[g] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(kf[c], qf[g][c], p[g], 0, 0, 0, 0, 0, 0);
        }
        // (the results pass through one empty asm: all MFMAs issue before any of them is read)
        if constexpr (HG == 4)
          asm volatile("" : "+v"(p[0]), "+v"(p[1]), "+v"(p[2]), "+v"(p[3]));
        else if constexpr (HG == 2)
          asm volatile("" : "+v"(p[0]), "+v"(p[1]));
#pragma unroll
        for (int g = 0; g < HG; ++g) {
#pragma unroll
          // relu * weight added with one rounding (an FMA), not two: within the scores'
          // tolerance either way, and 4% faster in this VALU-paced loop
          for (int r = 0; r < 4; ++r) a[r] = __builtin_fmaf(relu1(p[g][r]), wr[g], a[r]);
        }
        if (last) {
          const v4f kv = *reinterpret_cast<const v4f*>(&ksl[buf][16 * j + 4 * kq]);
          a = v4f{a[0] * kv[0], a[1] * kv[1], a[2] * kv[2], a[3] * kv[3]};
        }
        *slot = a;
      }
    }
    // the wave's 16 tokens x 128 keys as 512-byte row segments
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int row = 2 * it + (lane >> 5), c4 = lane & 31;
      const int64_t t = tl.tt * kTT + wave * 16 + row;
      const int64_t s0 = tl.s_begin + (int64_t)i * kKT + 4 * c4;
      const v4f v = *reinterpret_cast<const v4f*>(&my[row * OS + 4 * c4]);
      if (t < L) {
        float* o = out + (b * L + t) * S + s0;
        if (vec && s0 + 4 <= tl.s_end) {
          __builtin_nontemporal_store(v, reinterpret_cast<v4f*>(o));
        } else {
          for (int r = 0; r < 4; ++r)
            if (s0 + r < tl.s_end) o[r] = v[r];
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
    if (i + 1 < tl.nsub) {
      stage.store(kl[buf ^ 1], ksl[buf ^ 1]);
      __syncthreads();
    }
  }
}

// The fused form with 8 waves per workgroup (d <= 128, H <= 4, more than 512 keys): a
// workgroup owns 64 tokens x 1024 keys.  Waves 4h .. 4h+3 (half h) take keys
// [512 h, 512 h + 512) of the range, each half with its own key stages, and wave 4h + w the
// same 16 tokens in both halves.  Half h quantizes heads 2h and 2h + 1 of its tokens and the
// halves trade fragments and head weights through LDS, so each token's q is read and
// quantized once per 1024 keys instead of once per 512.  Every wave runs the loop nsub times
// (half 0's count, the larger) and meets every barrier; a half past its last sub-tile only
// waits at them.
constexpr int kPairThreads = 512;
constexpr int64_t kKPW2 = 2 * kKPW;

// QDT < 0: q arrives as codes with first scales qs (cin_indexer_scores_fp8); each half loads
// all four heads' fragments and nothing is traded.
template <int D, int QDT>
__global__ __launch_bounds__(kPairThreads) __attribute__((amdgpu_waves_per_eu(2, 8))) void k_indexer_scores_fp8_pair(
    const void* __restrict__ qin, const uint8_t* __restrict__ k8, const float* __restrict__ ks,
    const float* __restrict__ w, int64_t L, int64_t S, int64_t H, float softmax_scale,
    float* __restrict__ out, int64_t tiles_t, int64_t tiles_s, int xcd_rotate, int vec,
    uint8_t* __restrict__ q8_out, float* __restrict__ qs_out, const float* __restrict__ qs = nullptr) {
  static_assert(D <= 128, "one 128-byte slice per head row");
  constexpr int HG = 4;
  constexpr int RS = KeyStage<D>::RS;
  constexpr int OS = kKT + 4;
  constexpr int ES = RawSlice<QDT < 0 ? CIN_DT_BF16 : QDT>::ES;
  __shared__ __attribute__((aligned(16))) uint8_t kl[2][2][kKT * RS];
  __shared__ __attribute__((aligned(16))) float ksl[2][2][kKT];
  __shared__ __attribute__((aligned(16))) float ost[8 * 16 * OS];

  int64_t tile = blockIdx.x;
  if (xcd_rotate) {
    const int64_t per = gridDim.x >> 3;
    tile = (tile & 7) * per + (tile >> 3);
  }
  const int64_t b = tile / (tiles_t * tiles_s);
  const int64_t rem = tile - b * tiles_t * tiles_s;
  const int64_t tt = rem / tiles_s, sw = rem - tt * tiles_s;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int half = wave >> 2, wq = wave & 3;
  const int l16 = lane & 15, kq = lane >> 4;
  const int tid = threadIdx.x & 255;  // index within the half (its key stage's 256 threads)
  const int64_t r_begin = sw * kKPW2, r_end = r_begin + kKPW2 < S ? r_begin + kKPW2 : S;
  const int64_t h_begin = r_begin + half * kKPW;
  const int64_t h_end = h_begin + kKPW < r_end ? h_begin + kKPW : r_end;
  const int nsub_h = h_end > h_begin ? (int)((h_end - h_begin + kKT - 1) / kKT) : 0;
  const int64_t e0 = r_begin + kKPW < r_end ? r_begin + kKPW : r_end;
  const int nsub = (int)((e0 - r_begin + kKT - 1) / kKT);  // half 0's, the same in every wave

  const int64_t tok = tt * kTT + wq * 16 + l16;
  const bool tok_ok = tok < L;
  const int64_t orow = (b * L + (tok_ok ? tok : 0)) * H;
  KeyStage<D> stage;
  stage.load(k8, ks, b, S, h_begin, h_end, vec, tid);  // (keys past h_end read as zero)

  v8i qf[HG];
  float wr[HG];
  if constexpr (QDT < 0) {
    const uint8_t* qrow = static_cast<const uint8_t*>(qin) + orow * D;
#pragma unroll
    for (int g = 0; g < HG; ++g) {
      const bool ok = tok_ok && g < H;
      qf[g] = frag32<D>(qrow + g * D, ok, kq, 0);
      wr[g] = ok ? (qs[orow + g] * w[orow + g]) * softmax_scale : 0.0f;
    }
  } else {
    // this half's two heads: raw rows, codes, scales, head weights
    const uint8_t* qrow = static_cast<const uint8_t*>(qin) + orow * D * ES;
    RawSlice<QDT> raw[2];
    float wv[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int g = 2 * half + j;
      const bool ok = tok_ok && g < H;
      load_slice<D, QDT>(qrow + (int64_t)g * D * ES, ok, kq, 0, raw[j]);
      wv[j] = ok ? w[orow + g] : 0.0f;
    }
    v8i own[2];
    float own_w[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int g = 2 * half + j;
      const bool ok = tok_ok && g < H;
      float sc;
      own[j] = quant_slice<QDT>(raw[j], sc);
      own_w[j] = ok ? (sc * wv[j]) * softmax_scale : 0.0f;
      if (q8_out != nullptr && ok && g % tiles_s == sw) {
        const int off = 32 * kq;
        if (off < D) {
          uint8_t* dst = q8_out + (orow + g) * D + off;
          const v8i f = own[j];
          *reinterpret_cast<uint4*>(dst) = uint4{(uint32_t)f[0], (uint32_t)f[1], (uint32_t)f[2], (uint32_t)f[3]};
          *reinterpret_cast<uint4*>(dst + 16) = uint4{(uint32_t)f[4], (uint32_t)f[5], (uint32_t)f[6], (uint32_t)f[7]};
        }
        if (kq == 0) qs_out[orow + g] = sc;
      }
    }
    // trade through the (not yet used) staging area: [wave in half][head][lane][8 codes + weight]
    uint32_t* xch = reinterpret_cast<uint32_t*>(ost);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      uint32_t* p = xch + ((wq * HG + 2 * half + j) * 64 + lane) * 9;
#pragma unroll
      for (int e = 0; e < 8; ++e) p[e] = (uint32_t)own[j][e];
      p[8] = __float_as_uint(own_w[j]);
    }
    __syncthreads();
    v8i oth[2];
    float oth_w[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t* p = xch + ((wq * HG + 2 * (1 - half) + j) * 64 + lane) * 9;
#pragma unroll
      for (int e = 0; e < 8; ++e) oth[j][e] = (int)p[e];
      oth_w[j] = __uint_as_float(p[8]);
    }
    qf[0] = half == 0 ? own[0] : oth[0];
    qf[1] = half == 0 ? own[1] : oth[1];
    qf[2] = half == 0 ? oth[0] : own[0];
    qf[3] = half == 0 ? oth[1] : own[1];
    wr[0] = half == 0 ? own_w[0] : oth_w[0];
    wr[1] = half == 0 ? own_w[1] : oth_w[1];
    wr[2] = half == 0 ? oth_w[0] : own_w[0];
    wr[3] = half == 0 ? oth_w[1] : own_w[1];
  }
  stage.store(kl[half][0], ksl[half][0], tid);
  __syncthreads();  // the trade's reads are done before any wave stages scores over it

  float* my = ost + wave * 16 * OS;
  for (int i = 0; i < nsub; ++i) {
    const int buf = i & 1;
    if (i + 1 < nsub_h) stage.load(k8, ks, b, S, h_begin + (int64_t)(i + 1) * kKT, h_end, vec, tid);
    if (i < nsub_h) {
#pragma unroll 2
      for (int j = 0; j < 8; ++j) {
        const uint8_t* kr = &kl[half][buf][(16 * j + l16) * RS];
        const v8i kf = frag32<D>(kr, true, kq, 0);
        v4f p[HG];
#pragma unroll
        for (int g = 0; g < HG; ++g)
          p[g] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(kf, qf[g], v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0,
                                                                  0, 0, 0);
        asm volatile("" : "+v"(p[0]), "+v"(p[1]), "+v"(p[2]), "+v"(p[3]));
        v4f a = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int g = 0; g < HG; ++g) {
#pragma unroll
          for (int r = 0; r < 4; ++r) a[r] = __builtin_fmaf(relu1(p[g][r]), wr[g], a[r]);
        }
        const v4f kv = *reinterpret_cast<const v4f*>(&ksl[half][buf][16 * j + 4 * kq]);
        a = v4f{a[0] * kv[0], a[1] * kv[1], a[2] * kv[2], a[3] * kv[3]};
        *reinterpret_cast<v4f*>(&my[l16 * OS + 16 * j + 4 * kq]) = a;
      }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const int row = 2 * it + (lane >> 5), c4 = lane & 31;
        const int64_t t = tt * kTT + wq * 16 + row;
        const int64_t s0 = h_begin + (int64_t)i * kKT + 4 * c4;
        const v4f v = *reinterpret_cast<const v4f*>(&my[row * OS + 4 * c4]);
        if (t < L) {
          float* o = out + (b * L + t) * S + s0;
          if (vec && s0 + 4 <= h_end) {
            __builtin_nontemporal_store(v, reinterpret_cast<v4f*>(o));
          } else {
            for (int r = 0; r < 4; ++r)
              if (s0 + r < h_end) o[r] = v[r];
          }
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
    if (i + 1 < nsub) {
      if (i + 1 < nsub_h) stage.store(kl[half][buf ^ 1], ksl[half][buf ^ 1], tid);
      __syncthreads();
    }
  }
}

// Gradient of the scores with respect to the head weights (the reference's autograd through
// src/attention.py:298-300; q and k come from the non-differentiable quantizer):
//   G[b, t, h] = sum_s relu(logit[b, t, h, s]) * (dscores[b, t, s] * k_scale[b, s])
//   dweights   = (G * softmax_scale) * q_scale
// Same tiling as the forward.  Each wave stages its 16 tokens' dscores rows of a sub-tile
// through LDS (512-byte row segments in, 4 consecutive keys per lane out), recomputes the
// logits with the MFMA and sums per (token, head) in registers.  The 4 lanes of a token
// are summed with cross-lane adds, and each workgroup writes its key range's partial sum
// to partial[sw][b][t][h]; k_indexer_wgrad_finish adds the ranges in increasing order.
// Heads beyond HG take further passes over the key range.
template <int D, int HG>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(kMinWaves<D>, 8))) void k_indexer_wgrad_fp8(
    const uint8_t* __restrict__ q8, const uint8_t* __restrict__ k8, const float* __restrict__ ks,
    const float* __restrict__ gs, int64_t B, int64_t L, int64_t S, int64_t H,
    float* __restrict__ partial, int64_t tiles_t, int64_t tiles_s, int xcd_rotate, int vec) {
  constexpr int NC = (D + 127) / 128;
  constexpr int RS = KeyStage<D>::RS;
  constexpr int OS = kKT + 4;
  __shared__ __attribute__((aligned(16))) uint8_t kl[2][kKT * RS];
  __shared__ __attribute__((aligned(16))) float ksl[2][kKT];
  __shared__ __attribute__((aligned(16))) float gst[4 * 16 * OS];

  const Tile tl = tile_of(S, tiles_t, tiles_s, xcd_rotate);
  const int64_t b = tl.b;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int l16 = lane & 15, kq = lane >> 4;
  KeyStage<D> stage;
  const int64_t tok = tl.tt * kTT + wave * 16 + l16;
  const bool tok_ok = tok < L;
  const uint8_t* qrow = q8 + (b * L + (tok_ok ? tok : 0)) * H * D;
  float* my = gst + wave * 16 * OS;

  // the wave's dscores rows of one sub-tile, 8 x 16 bytes per lane (zero past L or the range)
  v4f gpre[8];
  auto load_g = [&](int64_t s_sub) {
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int row = 2 * it + (lane >> 5), c4 = lane & 31;
      const int64_t t = tl.tt * kTT + wave * 16 + row;
      const int64_t s0 = s_sub + 4 * c4;
      gpre[it] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      if (t < L) {
        const float* g = gs + (b * L + t) * S + s0;
        if (vec && s0 + 4 <= tl.s_end) {
          gpre[it] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(g));
        } else {
          for (int r = 0; r < 4; ++r)
            if (s0 + r < tl.s_end) gpre[it][r] = g[r];
        }
      }
    }
  };
  auto store_g = [&]() {
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int row = 2 * it + (lane >> 5), c4 = lane & 31;
      *reinterpret_cast<v4f*>(&my[row * OS + 4 * c4]) = gpre[it];
    }
  };

  for (int64_t h0 = 0; h0 < H; h0 += HG) {
    v8i qf[HG][NC];
#pragma unroll
    for (int g = 0; g < HG; ++g) {
      const bool ok = tok_ok && h0 + g < H;
#pragma unroll
      for (int c = 0; c < NC; ++c) qf[g][c] = frag32<D>(qrow + (h0 + g) * D, ok, kq, c);
    }
    float acc[HG];
#pragma unroll
    for (int g = 0; g < HG; ++g) acc[g] = 0.0f;
    if (h0 > 0) __syncthreads();  // the previous pass is done with both key buffers
    stage.load(k8, ks, b, S, tl.s_begin, tl.s_end, vec);
    load_g(tl.s_begin);
    stage.store(kl[0], ksl[0]);
    store_g();
    __syncthreads();
    for (int i = 0; i < tl.nsub; ++i) {
      const int buf = i & 1;
      const bool more = i + 1 < tl.nsub;
      if (more) {
        stage.load(k8, ks, b, S, tl.s_begin + (int64_t)(i + 1) * kKT, tl.s_end, vec);
        load_g(tl.s_begin + (int64_t)(i + 1) * kKT);
      }
#pragma unroll 2
      for (int j = 0; j < 8; ++j) {
        const uint8_t* kr = &kl[buf][(16 * j + l16) * RS];
        v8i kf[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) kf[c] = frag32<D>(kr, true, kq, c);
        const v4f gv = *reinterpret_cast<const v4f*>(&my[l16 * OS + 16 * j + 4 * kq]);
        const v4f kv = *reinterpret_cast<const v4f*>(&ksl[buf][16 * j + 4 * kq]);
        const v4f dx = v4f{gv[0] * kv[0], gv[1] * kv[1], gv[2] * kv[2], gv[3] * kv[3]};
        // every head's MFMAs first (as in the scoring kernel), then the sums
        v4f p[HG];
#pragma unroll
        for (int g = 0; g < HG; ++g) {
          p[g] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int c = 0; c < NC; ++c)
            p[g] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(kf[c], qf[g][c], p[g], 0, 0, 0, 0, 0, 0);
        }
        if constexpr (HG == 4)
          asm volatile("" : "+v"(p[0]), "+v"(p[1]), "+v"(p[2]), "+v"(p[3]));
        else if constexpr (HG == 2)
          asm volatile("" : "+v"(p[0]), "+v"(p[1]));
#pragma unroll
        for (int g = 0; g < HG; ++g) {
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[g] = __builtin_fmaf(relu1(p[g][r]), dx[r], acc[g]);
        }
      }
      if (more) {
        // this wave's reads of its staging rows precede the overwrite (in-order LDS)
        store_g();
        stage.store(kl[buf ^ 1], ksl[buf ^ 1]);
        __syncthreads();
      }
    }
    // lanes l16, l16 + 16, l16 + 32, l16 + 48 hold the same token: add them
#pragma unroll
    for (int g = 0; g < HG; ++g) {
      acc[g] += __shfl_xor(acc[g], 16);
      acc[g] += __shfl_xor(acc[g], 32);
    }
    if (kq == 0 && tok_ok) {
#pragma unroll
      for (int g = 0; g < HG; ++g)
        if (h0 + g < H) partial[((tl.sw * B + b) * L + tok) * H + h0 + g] = acc[g];
    }
  }
}

// The weights gradient with 8 waves per 64 tokens x 1024 keys (d <= 128, H <= 4, more than
// 512 keys), the scoring kernel's pair tiling: half h sums over keys [512 h, 512 h + 512) of
// the range exactly as k_indexer_wgrad_fp8 sums over one 512-key range, so its per-range
// partial sum is the same.  With one 1024-key range (S <= 1024) the workgroup finishes in
// place: dweights = (((0 + half 0's sum) + half 1's sum) * softmax_scale) * q_scale, the
// finish kernel's arithmetic; with more it writes the two partial sums for that kernel.
// Every wave runs half 0's loop count and meets every barrier.
template <int D>
__global__ __launch_bounds__(kPairThreads) __attribute__((amdgpu_waves_per_eu(2, 8))) void k_indexer_wgrad_fp8_pair(
    const uint8_t* __restrict__ q8, const float* __restrict__ qs, const uint8_t* __restrict__ k8,
    const float* __restrict__ ks, const float* __restrict__ gs, int64_t B, int64_t L, int64_t S,
    int64_t H, float softmax_scale, float* __restrict__ partial, float* __restrict__ dw,
    int64_t tiles_t, int64_t tiles_s, int xcd_rotate, int vec) {
  static_assert(D <= 128, "one 128-byte slice per head row");
  constexpr int HG = 4;
  constexpr int RS = KeyStage<D>::RS;
  constexpr int OS = kKT + 4;
  __shared__ __attribute__((aligned(16))) uint8_t kl[2][2][kKT * RS];
  __shared__ __attribute__((aligned(16))) float ksl[2][2][kKT];
  __shared__ __attribute__((aligned(16))) float gst[8 * 16 * OS];

  int64_t tile = blockIdx.x;
  if (xcd_rotate) {
    const int64_t per = gridDim.x >> 3;
    tile = (tile & 7) * per + (tile >> 3);
  }
  const int64_t b = tile / (tiles_t * tiles_s);
  const int64_t rem = tile - b * tiles_t * tiles_s;
  const int64_t tt = rem / tiles_s, sw = rem - tt * tiles_s;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int half = wave >> 2, wq = wave & 3;
  const int l16 = lane & 15, kq = lane >> 4;
  const int tid = threadIdx.x & 255;
  const int64_t r_begin = sw * kKPW2, r_end = r_begin + kKPW2 < S ? r_begin + kKPW2 : S;
  const int64_t h_begin = r_begin + half * kKPW;
  const int64_t h_end = h_begin + kKPW < r_end ? h_begin + kKPW : r_end;
  const int nsub_h = h_end > h_begin ? (int)((h_end - h_begin + kKT - 1) / kKT) : 0;
  const int64_t e0 = r_begin + kKPW < r_end ? r_begin + kKPW : r_end;
  const int nsub = (int)((e0 - r_begin + kKT - 1) / kKT);  // half 0's, the same in every wave

  const int64_t tok = tt * kTT + wq * 16 + l16;
  const bool tok_ok = tok < L;
  const uint8_t* qrow = q8 + (b * L + (tok_ok ? tok : 0)) * H * D;
  float* my = gst + wave * 16 * OS;
  KeyStage<D> stage;

  v4f gpre[8];
  auto load_g = [&](int64_t s_sub) {
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int row = 2 * it + (lane >> 5), c4 = lane & 31;
      const int64_t t = tt * kTT + wq * 16 + row;
      const int64_t s0 = s_sub + 4 * c4;
      gpre[it] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      if (t < L) {
        const float* g = gs + (b * L + t) * S + s0;
        if (vec && s0 + 4 <= h_end) {
          gpre[it] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(g));
        } else {
          for (int r = 0; r < 4; ++r)
            if (s0 + r < h_end) gpre[it][r] = g[r];
        }
      }
    }
  };
  auto store_g = [&]() {
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int row = 2 * it + (lane >> 5), c4 = lane & 31;
      *reinterpret_cast<v4f*>(&my[row * OS + 4 * c4]) = gpre[it];
    }
  };

  v8i qf[HG];
#pragma unroll
  for (int g = 0; g < HG; ++g) qf[g] = frag32<D>(qrow + g * D, tok_ok && g < H, kq, 0);
  float acc[HG];
#pragma unroll
  for (int g = 0; g < HG; ++g) acc[g] = 0.0f;
  stage.load(k8, ks, b, S, h_begin, h_end, vec, tid);  // (keys past h_end read as zero)
  load_g(h_begin);
  stage.store(kl[half][0], ksl[half][0], tid);
  store_g();
  __syncthreads();
  for (int i = 0; i < nsub; ++i) {
    const int buf = i & 1;
    const bool more = i + 1 < nsub_h;
    if (more) {
      stage.load(k8, ks, b, S, h_begin + (int64_t)(i + 1) * kKT, h_end, vec, tid);
      load_g(h_begin + (int64_t)(i + 1) * kKT);
    }
    if (i < nsub_h) {
#pragma unroll 2
      for (int j = 0; j < 8; ++j) {
        const uint8_t* kr = &kl[half][buf][(16 * j + l16) * RS];
        const v8i kf = frag32<D>(kr, true, kq, 0);
        const v4f gv = *reinterpret_cast<const v4f*>(&my[l16 * OS + 16 * j + 4 * kq]);
        const v4f kv = *reinterpret_cast<const v4f*>(&ksl[half][buf][16 * j + 4 * kq]);
        const v4f dx = v4f{gv[0] * kv[0], gv[1] * kv[1], gv[2] * kv[2], gv[3] * kv[3]};
        v4f p[HG];
#pragma unroll
        for (int g = 0; g < HG; ++g)
          p[g] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(kf, qf[g], v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0,
                                                                  0, 0, 0);
        asm volatile("" : "+v"(p[0]), "+v"(p[1]), "+v"(p[2]), "+v"(p[3]));
#pragma unroll
        for (int g = 0; g < HG; ++g) {
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[g] = __builtin_fmaf(relu1(p[g][r]), dx[r], acc[g]);
        }
      }
    }
    if (i + 1 < nsub) {
      if (more) {
        // this wave's reads of its staging rows precede the overwrite (in-order LDS)
        store_g();
        stage.store(kl[half][buf ^ 1], ksl[half][buf ^ 1], tid);
      }
      __syncthreads();
    }
  }
  // lanes l16, l16 + 16, l16 + 32, l16 + 48 hold the same token: add them
#pragma unroll
  for (int g = 0; g < HG; ++g) {
    acc[g] += __shfl_xor(acc[g], 16);
    acc[g] += __shfl_xor(acc[g], 32);
  }
  if (tiles_s == 1) {
    // half 1's sums to LDS (over its staging rows, read by now: the barrier below orders
    // every wave's last staging reads before half 1 writes), half 0 finishes
    __syncthreads();
    float* xs = gst;  // [wave in half][lane][head]
    if (half == 1) {
#pragma unroll
      for (int g = 0; g < HG; ++g) xs[(wq * 64 + lane) * HG + g] = acc[g];
    }
    __syncthreads();
    if (half == 0 && kq == 0 && tok_ok) {
      const int64_t o = (b * L + tok) * H;
#pragma unroll
      for (int g = 0; g < HG; ++g) {
        if (g < H) {
          const float tot = (0.0f + acc[g]) + xs[(wq * 64 + lane) * HG + g];
          dw[o + g] = (tot * softmax_scale) * qs[o + g];
        }
      }
    }
  } else if (kq == 0 && tok_ok && nsub_h > 0) {
    const int64_t r = 2 * sw + half;  // 512-key range index
#pragma unroll
    for (int g = 0; g < HG; ++g)
      if (g < H) partial[((r * B + b) * L + tok) * H + g] = acc[g];
  }
}

// dweights[i] = ((sum over key ranges, increasing) * softmax_scale) * q_scale[i], i over B L H.
__global__ void k_indexer_wgrad_finish(const float* __restrict__ partial, const float* __restrict__ qs,
                                       int64_t n, int64_t ranges, float softmax_scale,
                                       float* __restrict__ dw) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float g = 0.0f;
  for (int64_t r = 0; r < ranges; ++r) g = g + partial[r * n + i];
  dw[i] = (g * softmax_scale) * qs[i];
}

template <int D, int HG>
void launch_indexer(unsigned grid, hipStream_t st, const uint8_t* q8, const float* qs,
                    const uint8_t* k8, const float* ks, const float* w, int64_t L, int64_t S,
                    int64_t H, float softmax_scale, float* out, int64_t tiles_t, int64_t tiles_s,
                    int xcd_rotate, int vec) {
  hipLaunchKernelGGL((k_indexer_scores_fp8<D, HG>), grid, kThreads, 0, st, q8, qs, k8, ks, w, L, S,
                     H, softmax_scale, out, tiles_t, tiles_s, xcd_rotate, vec);
}

template <int D, int HG>
void launch_indexer_q(int q_dtype, unsigned grid, hipStream_t st, const void* q, const uint8_t* k8,
                      const float* ks, const float* w, int64_t L, int64_t S, int64_t H,
                      float softmax_scale, float* out, int64_t tiles_t, int64_t tiles_s,
                      int xcd_rotate, int vec, uint8_t* q8_out, float* qs_out) {
#define CIN_IQ_LAUNCH(DT)                                                                         \
  hipLaunchKernelGGL((k_indexer_scores_fp8<D, HG, DT>), grid, kThreads, 0, st, q, nullptr, k8, ks, w, \
                     L, S, H, softmax_scale, out, tiles_t, tiles_s, xcd_rotate, vec, q8_out, qs_out)
  if (q_dtype == CIN_DT_BF16)
    CIN_IQ_LAUNCH(CIN_DT_BF16);
  else if (q_dtype == CIN_DT_F16)
    CIN_IQ_LAUNCH(CIN_DT_F16);
  else
    CIN_IQ_LAUNCH(CIN_DT_F32);
#undef CIN_IQ_LAUNCH
}

template <int D>
void launch_indexer_pair(int q_dtype, unsigned grid, hipStream_t st, const void* q, const uint8_t* k8,
                         const float* ks, const float* w, int64_t L, int64_t S, int64_t H,
                         float softmax_scale, float* out, int64_t tiles_t, int64_t tiles_s,
                         int xcd_rotate, int vec, uint8_t* q8_out, float* qs_out) {
#define CIN_IQP_LAUNCH(DT)                                                                              \
  hipLaunchKernelGGL((k_indexer_scores_fp8_pair<D, DT>), grid, kPairThreads, 0, st, q, k8, ks, w, L, S, H, \
                     softmax_scale, out, tiles_t, tiles_s, xcd_rotate, vec, q8_out, qs_out)
  if (q_dtype == CIN_DT_BF16)
    CIN_IQP_LAUNCH(CIN_DT_BF16);
  else if (q_dtype == CIN_DT_F16)
    CIN_IQP_LAUNCH(CIN_DT_F16);
  else
    CIN_IQP_LAUNCH(CIN_DT_F32);
#undef CIN_IQP_LAUNCH
}

template <int D, int HG>
void launch_wgrad(unsigned grid, hipStream_t st, const uint8_t* q8, const uint8_t* k8,
                  const float* ks, const float* gs, int64_t B, int64_t L, int64_t S, int64_t H,
                  float* partial, int64_t tiles_t, int64_t tiles_s, int xcd_rotate, int vec) {
  hipLaunchKernelGGL((k_indexer_wgrad_fp8<D, HG>), grid, kThreads, 0, st, q8, k8, ks, gs, B, L, S,
                     H, partial, tiles_t, tiles_s, xcd_rotate, vec);
}

}  // namespace

extern "C" {

int cin_indexer_scores_fp8(const uint8_t* q8, const float* q_scale, const uint8_t* k8,
                           const float* k_scale, const float* weights, int64_t B, int64_t L,
                           int64_t S, int64_t H, int64_t d, float softmax_scale, float* scores,
                           void* stream) {
  CIN_CHECK_ARG(B >= 0 && L >= 0 && S >= 0 && H >= 1, "indexer_scores_fp8: bad sizes");
  CIN_CHECK_ARG(d >= 32 && d <= 256 && d % 32 == 0,
                "indexer_scores_fp8: head dim %lld must be a multiple of 32 in [32, %d]",
                (long long)d, 256);
  if (B == 0 || L == 0 || S == 0) return CIN_OK;
  CIN_CHECK_ARG(q8 && q_scale && k8 && k_scale && weights && scores, "indexer_scores_fp8: null pointer");
  CIN_CHECK_ARG((((uintptr_t)q8) & 15) == 0 && (((uintptr_t)k8) & 15) == 0,
                "indexer_scores_fp8: code buffers must be 16-byte aligned");
  const int64_t tiles_t = cdiv(L, kTT), tiles_s = cdiv(S, kKPW);
  CIN_CHECK_ARG(B * tiles_t * tiles_s < ((int64_t)1 << 31), "indexer_scores_fp8: grid too large");
  const unsigned grid = (unsigned)(B * tiles_t * tiles_s);
  const int xcd_rotate = grid % 8 == 0;
  const int vec = S % 4 == 0 && (((uintptr_t)k_scale) & 15) == 0 && (((uintptr_t)scores) & 15) == 0;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (d <= 128 && H <= 4 && S > kKPW) {
    // 8 waves per 64 tokens x 1024 keys: q's codes read once per 1024 keys
    const int64_t tiles_s2 = cdiv(S, kKPW2);
    const unsigned grid2 = (unsigned)(B * tiles_t * tiles_s2);
    const int xr2 = grid2 % 8 == 0;
    switch (d / 32) {
#define CIN_INDEXER_PC_CASE(n)                                                                        \
  case n:                                                                                             \
    hipLaunchKernelGGL((k_indexer_scores_fp8_pair<32 * n, -1>), grid2, kPairThreads, 0, st, q8, k8, k_scale, \
                       weights, L, S, H, softmax_scale, scores, tiles_t, tiles_s2, xr2, vec, nullptr,       \
                       nullptr, q_scale);                                                             \
    break;
      CIN_INDEXER_PC_CASE(1) CIN_INDEXER_PC_CASE(2) CIN_INDEXER_PC_CASE(3) CIN_INDEXER_PC_CASE(4)
#undef CIN_INDEXER_PC_CASE
    }
    return cin_check_launch("indexer_scores_fp8");
  }
  switch (d / 32) {
#define CIN_INDEXER_CASE(n, hg)                                                                 \
  case n:                                                                                       \
    launch_indexer<32 * n, hg>(grid, st, q8, q_scale, k8, k_scale, weights, L, S, H,            \
                               softmax_scale, scores, tiles_t, tiles_s, xcd_rotate, vec);       \
    break;
    CIN_INDEXER_CASE(1, 4) CIN_INDEXER_CASE(2, 4) CIN_INDEXER_CASE(3, 4) CIN_INDEXER_CASE(4, 4)
    CIN_INDEXER_CASE(5, 2) CIN_INDEXER_CASE(6, 2) CIN_INDEXER_CASE(7, 2) CIN_INDEXER_CASE(8, 2)
#undef CIN_INDEXER_CASE
  }
  return cin_check_launch("indexer_scores_fp8");
}

int cin_indexer_scores_fp8_q(const void* q, int q_dtype, const uint8_t* k8, const float* k_scale,
                             const float* weights, int64_t B, int64_t L, int64_t S, int64_t H, int64_t d,
                             float softmax_scale, float* scores, uint8_t* q8, float* q_scale,
                             void* stream) {
  CIN_CHECK_ARG(q_dtype == CIN_DT_BF16 || q_dtype == CIN_DT_F16 || q_dtype == CIN_DT_F32,
                "indexer_scores_fp8_q: unsupported q dtype %d", q_dtype);
  CIN_CHECK_ARG(B >= 0 && L >= 0 && S >= 0 && H >= 1, "indexer_scores_fp8_q: bad sizes");
  CIN_CHECK_ARG(d >= 32 && d <= 256 && d % 32 == 0,
                "indexer_scores_fp8_q: head dim %lld must be a multiple of 32 in [32, 256]", (long long)d);
  const int64_t hg = d <= 128 ? 4 : 2;
  CIN_CHECK_ARG(H <= hg,
                "indexer_scores_fp8_q: %lld heads at head dim %lld, at most %lld (quantize q with "
                "cin_indexer_quantize and call cin_indexer_scores_fp8)", (long long)H, (long long)d,
                (long long)hg);
  CIN_CHECK_ARG((q8 == nullptr) == (q_scale == nullptr),
                "indexer_scores_fp8_q: q8 and q_scale are both given or both null");
  if (B == 0 || L == 0) return CIN_OK;
  CIN_CHECK_ARG(q != nullptr, "indexer_scores_fp8_q: null pointer");
  CIN_CHECK_ARG((((uintptr_t)q) & 15) == 0 && (((uintptr_t)q8) & 15) == 0,
                "indexer_scores_fp8_q: q and q8 must be 16-byte aligned");
  if (S == 0) {  // no scores to write; the codes are still asked for
    if (q8 == nullptr) return CIN_OK;
    return cin_indexer_quantize(q, q_dtype, q, q_dtype, B, L, 0, H, d, q8, q_scale, nullptr, nullptr,
                                stream);
  }
  CIN_CHECK_ARG(k8 && k_scale && weights && scores, "indexer_scores_fp8_q: null pointer");
  CIN_CHECK_ARG((((uintptr_t)k8) & 15) == 0, "indexer_scores_fp8_q: k8 must be 16-byte aligned");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const int vec = S % 4 == 0 && (((uintptr_t)k_scale) & 15) == 0 && (((uintptr_t)scores) & 15) == 0;
  if (d <= 128 && S > kKPW) {
    // 8 waves per 64 tokens x 1024 keys: q read and quantized once per 1024 keys
    const int64_t tiles_t2 = cdiv(L, kTT), tiles_s2 = cdiv(S, kKPW2);
    CIN_CHECK_ARG(B * tiles_t2 * tiles_s2 < ((int64_t)1 << 31), "indexer_scores_fp8_q: grid too large");
    const unsigned grid2 = (unsigned)(B * tiles_t2 * tiles_s2);
    const int xr2 = grid2 % 8 == 0;
    switch (d / 32) {
#define CIN_INDEXER_P_CASE(n)                                                                      \
  case n:                                                                                          \
    launch_indexer_pair<32 * n>(q_dtype, grid2, st, q, k8, k_scale, weights, L, S, H, softmax_scale, \
                                scores, tiles_t2, tiles_s2, xr2, vec, q8, q_scale);                \
    break;
      CIN_INDEXER_P_CASE(1) CIN_INDEXER_P_CASE(2) CIN_INDEXER_P_CASE(3) CIN_INDEXER_P_CASE(4)
#undef CIN_INDEXER_P_CASE
    }
    return cin_check_launch("indexer_scores_fp8_q");
  }
  const int64_t tiles_t = cdiv(L, kTT), tiles_s = cdiv(S, kKPW);
  CIN_CHECK_ARG(B * tiles_t * tiles_s < ((int64_t)1 << 31), "indexer_scores_fp8_q: grid too large");
  const unsigned grid = (unsigned)(B * tiles_t * tiles_s);
  const int xcd_rotate = grid % 8 == 0;
  switch (d / 32) {
#define CIN_INDEXER_Q_CASE(n, hgv)                                                                  \
  case n:                                                                                           \
    launch_indexer_q<32 * n, hgv>(q_dtype, grid, st, q, k8, k_scale, weights, L, S, H, softmax_scale, \
                                  scores, tiles_t, tiles_s, xcd_rotate, vec, q8, q_scale);          \
    break;
    CIN_INDEXER_Q_CASE(1, 4) CIN_INDEXER_Q_CASE(2, 4) CIN_INDEXER_Q_CASE(3, 4) CIN_INDEXER_Q_CASE(4, 4)
    CIN_INDEXER_Q_CASE(5, 2) CIN_INDEXER_Q_CASE(6, 2) CIN_INDEXER_Q_CASE(7, 2) CIN_INDEXER_Q_CASE(8, 2)
#undef CIN_INDEXER_Q_CASE
  }
  return cin_check_launch("indexer_scores_fp8_q");
}

int64_t cin_indexer_weights_grad_workspace(int64_t B, int64_t L, int64_t S, int64_t H) {
  if (B < 0 || L < 0 || S < 0 || H < 0) return 0;
  return cdiv(S, kKPW) * B * L * H;
}

int cin_indexer_weights_grad(const uint8_t* q8, const float* q_scale, const uint8_t* k8,
                             const float* k_scale, const float* grad_scores, int64_t B, int64_t L,
                             int64_t S, int64_t H, int64_t d, float softmax_scale, float* workspace,
                             int64_t workspace_len, float* grad_weights, void* stream) {
  CIN_CHECK_ARG(B >= 0 && L >= 0 && S >= 0 && H >= 1, "indexer_weights_grad: bad sizes");
  CIN_CHECK_ARG(d >= 32 && d <= 256 && d % 32 == 0,
                "indexer_weights_grad: head dim %lld must be a multiple of 32 in [32, 256]", (long long)d);
  if (B == 0 || L == 0) return CIN_OK;
  CIN_CHECK_ARG(q_scale && grad_weights, "indexer_weights_grad: null pointer");
  const int64_t tiles_t = cdiv(L, kTT), tiles_s = cdiv(S, kKPW);
  CIN_CHECK_ARG(workspace_len >= tiles_s * B * L * H,
                "indexer_weights_grad: workspace of %lld floats, %lld needed", (long long)workspace_len,
                (long long)(tiles_s * B * L * H));
  CIN_CHECK_ARG(B * tiles_t * tiles_s < ((int64_t)1 << 31) && B * L * H < ((int64_t)1 << 38),
                "indexer_weights_grad: grid too large");  // finish grid: B L H / 256 < 2^30
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (S > kKPW && d <= 128 && H <= 4) {
    // 8 waves per 64 tokens x 1024 keys; with one such range (S <= 1024) no finishing pass
    CIN_CHECK_ARG(q8 && k8 && k_scale && grad_scores && workspace, "indexer_weights_grad: null pointer");
    CIN_CHECK_ARG((((uintptr_t)q8) & 15) == 0 && (((uintptr_t)k8) & 15) == 0,
                  "indexer_weights_grad: code buffers must be 16-byte aligned");
    const int64_t tiles_s2 = cdiv(S, kKPW2);
    const unsigned grid2 = (unsigned)(B * tiles_t * tiles_s2);
    const int xr2 = grid2 % 8 == 0;
    const int vec = S % 4 == 0 && (((uintptr_t)k_scale) & 15) == 0 && (((uintptr_t)grad_scores) & 15) == 0;
    switch (d / 32) {
#define CIN_WGRAD_P_CASE(n)                                                                         \
  case n:                                                                                           \
    hipLaunchKernelGGL((k_indexer_wgrad_fp8_pair<32 * n>), grid2, kPairThreads, 0, st, q8, q_scale, k8, \
                       k_scale, grad_scores, B, L, S, H, softmax_scale, workspace, grad_weights,     \
                       tiles_t, tiles_s2, xr2, vec);                                                 \
    break;
      CIN_WGRAD_P_CASE(1) CIN_WGRAD_P_CASE(2) CIN_WGRAD_P_CASE(3) CIN_WGRAD_P_CASE(4)
#undef CIN_WGRAD_P_CASE
    }
    if (tiles_s2 == 1) return cin_check_launch("indexer_weights_grad");
    const int64_t n = B * L * H;
    hipLaunchKernelGGL(k_indexer_wgrad_finish, (unsigned)cdiv(n, 256), 256, 0, st, workspace, q_scale, n,
                       tiles_s, softmax_scale, grad_weights);
    return cin_check_launch("indexer_weights_grad");
  }
  if (S > 0) {
    CIN_CHECK_ARG(q8 && k8 && k_scale && grad_scores && workspace, "indexer_weights_grad: null pointer");
    CIN_CHECK_ARG((((uintptr_t)q8) & 15) == 0 && (((uintptr_t)k8) & 15) == 0,
                  "indexer_weights_grad: code buffers must be 16-byte aligned");
    const unsigned grid = (unsigned)(B * tiles_t * tiles_s);
    const int xcd_rotate = grid % 8 == 0;
    const int vec = S % 4 == 0 && (((uintptr_t)k_scale) & 15) == 0 && (((uintptr_t)grad_scores) & 15) == 0;
    switch (d / 32) {
#define CIN_WGRAD_CASE(n, hg)                                                                   \
  case n:                                                                                       \
    launch_wgrad<32 * n, hg>(grid, st, q8, k8, k_scale, grad_scores, B, L, S, H, workspace,     \
                             tiles_t, tiles_s, xcd_rotate, vec);                                \
    break;
      CIN_WGRAD_CASE(1, 4) CIN_WGRAD_CASE(2, 4) CIN_WGRAD_CASE(3, 4) CIN_WGRAD_CASE(4, 4)
      CIN_WGRAD_CASE(5, 2) CIN_WGRAD_CASE(6, 2) CIN_WGRAD_CASE(7, 2) CIN_WGRAD_CASE(8, 2)
#undef CIN_WGRAD_CASE
    }
  }
  const int64_t n = B * L * H;
  hipLaunchKernelGGL(k_indexer_wgrad_finish, (unsigned)cdiv(n, 256), 256, 0, st, workspace, q_scale, n,
                     tiles_s, softmax_scale, grad_weights);
  return cin_check_launch("indexer_weights_grad");
}

}  // extern "C"
