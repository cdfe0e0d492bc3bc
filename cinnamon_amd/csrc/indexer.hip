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

// D = head dim (multiple of 32, <= 256), HG = heads whose q fragments are held at once.
// vec: k_scale and scores rows are 16-byte aligned (S % 4 == 0 and aligned bases).
template <int D, int HG>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 8))) void k_indexer_scores_fp8(
    const uint8_t* __restrict__ q8, const float* __restrict__ qs, const uint8_t* __restrict__ k8,
    const float* __restrict__ ks, const float* __restrict__ w, int64_t L, int64_t S, int64_t H,
    float softmax_scale, float* __restrict__ out, int64_t tiles_t, int64_t tiles_s, int xcd_rotate,
    int vec) {
  constexpr int NC = (D + 127) / 128;           // 128-byte slices of d
  constexpr int RS = D + 16;                    // LDS key row stride (bytes)
  constexpr int CH = D / 16;                    // 16-byte chunks per key row
  constexpr int PER = (kKT * CH + kThreads - 1) / kThreads;
  constexpr int OS = kKT + 4;                   // staging row stride (floats)
  __shared__ __attribute__((aligned(16))) uint8_t kl[2][kKT * RS];
  __shared__ __attribute__((aligned(16))) float ksl[2][kKT];
  __shared__ __attribute__((aligned(16))) float ost[4 * 16 * OS];

  int64_t tile = blockIdx.x;
  if (xcd_rotate) {  // grid is a multiple of 8: XCD x = blockIdx % 8 runs tiles [x n/8, (x+1) n/8)
    const int64_t per = gridDim.x >> 3;
    tile = (tile & 7) * per + (tile >> 3);
  }
  const int64_t b = tile / (tiles_t * tiles_s);
  const int64_t rem = tile - b * tiles_t * tiles_s;
  const int64_t tt = rem / tiles_s, sw = rem - tt * tiles_s;
  const int64_t s_begin = sw * kKPW;
  const int64_t s_end = s_begin + kKPW < S ? s_begin + kKPW : S;
  const int nsub = (int)((s_end - s_begin + kKT - 1) / kKT);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int l16 = lane & 15, kq = lane >> 4;

  // ---- key sub-tile staging: global -> registers (issued early) -> LDS
  uint4 pre[PER];
  v4f kpre = {0.0f, 0.0f, 0.0f, 0.0f};
  auto load_sub = [&](int i) {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int idx = threadIdx.x + u * kThreads;
      const int row = idx / CH, c = idx - row * CH;
      const int64_t s = s_begin + (int64_t)i * kKT + row;
      pre[u] = uint4{0u, 0u, 0u, 0u};
      if (idx < kKT * CH && s < s_end) pre[u] = *reinterpret_cast<const uint4*>(k8 + (b * S + s) * D + 16 * c);
    }
    if (threadIdx.x < kKT / 4) {
      const int64_t s0 = s_begin + (int64_t)i * kKT + 4 * threadIdx.x;
      kpre = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      if (vec && s0 + 4 <= s_end) {
        kpre = *reinterpret_cast<const v4f*>(ks + b * S + s0);
      } else {
        for (int r = 0; r < 4; ++r)
          if (s0 + r < s_end) kpre[r] = ks[b * S + s0 + r];
      }
    }
  };
  auto store_sub = [&](int buf) {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int idx = threadIdx.x + u * kThreads;
      const int row = idx / CH, c = idx - row * CH;
      if (idx < kKT * CH) *reinterpret_cast<uint4*>(&kl[buf][row * RS + 16 * c]) = pre[u];
    }
    if (threadIdx.x < kKT / 4) *reinterpret_cast<v4f*>(&ksl[buf][4 * threadIdx.x]) = kpre;
  };

  // ---- the wave's tokens: q fragments and head weights for HG heads
  const int64_t tok = tt * kTT + wave * 16 + l16;
  const bool tok_ok = tok < L;
  const uint8_t* qrow = q8 + (b * L + (tok_ok ? tok : 0)) * H * D;
  const int64_t orow = (b * L + (tok_ok ? tok : 0)) * H;
  v8i qf[HG][NC];
  float wr[HG];
  auto load_q = [&](int64_t h0) {
#pragma unroll
    for (int g = 0; g < HG; ++g) {
      const bool ok = tok_ok && h0 + g < H;
#pragma unroll
      for (int c = 0; c < NC; ++c) qf[g][c] = frag32<D>(qrow + (h0 + g) * D, ok, kq, c);
      wr[g] = ok ? (qs[orow + h0 + g] * w[orow + h0 + g]) * softmax_scale : 0.0f;
    }
  };
  const bool one_group = H <= HG;

  load_sub(0);
  load_q(0);
  store_sub(0);
  __syncthreads();
  float* my = ost + wave * 16 * OS;
  for (int i = 0; i < nsub; ++i) {
    const int buf = i & 1;
    if (i + 1 < nsub) load_sub(i + 1);
    // Each 16-key tile's head sum goes straight to the wave's staging rows; a later head
    // group continues the sum from there (same increasing head order).  The staging rows
    // belong to this wave alone and a wave's LDS accesses complete in order, so no
    // workgroup barrier is needed around them.
    for (int64_t h0 = 0; h0 < H; h0 += HG) {
      if (!one_group) load_q(h0);
      const bool first = h0 == 0, last = h0 + HG >= H;
#pragma unroll 2
      for (int j = 0; j < 8; ++j) {
        const uint8_t* kr = &kl[buf][(16 * j + l16) * RS];
        v8i kf[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) kf[c] = frag32<D>(kr, true, kq, c);
        v4f* slot = reinterpret_cast<v4f*>(&my[l16 * OS + 16 * j + 4 * kq]);
        v4f a = first ? v4f{0.0f, 0.0f, 0.0f, 0.0f} : *slot;
#pragma unroll
        for (int g = 0; g < HG; ++g) {
          v4f p = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int c = 0; c < NC; ++c)
            p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(kf[c], qf[g][c], p, 0, 0, 0, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) a[r] = a[r] + fmaxf(p[r], 0.0f) * wr[g];
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
      const int64_t t = tt * kTT + wave * 16 + row;
      const int64_t s0 = s_begin + (int64_t)i * kKT + 4 * c4;
      const v4f v = *reinterpret_cast<const v4f*>(&my[row * OS + 4 * c4]);
      if (t < L) {
        float* o = out + (b * L + t) * S + s0;
        if (vec && s0 + 4 <= s_end) {
          __builtin_nontemporal_store(v, reinterpret_cast<v4f*>(o));
        } else {
          for (int r = 0; r < 4; ++r)
            if (s0 + r < s_end) o[r] = v[r];
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
    if (i + 1 < nsub) {
      store_sub(buf ^ 1);
      __syncthreads();
    }
  }
}

template <int D, int HG>
void launch_indexer(unsigned grid, hipStream_t st, const uint8_t* q8, const float* qs,
                    const uint8_t* k8, const float* ks, const float* w, int64_t L, int64_t S,
                    int64_t H, float softmax_scale, float* out, int64_t tiles_t, int64_t tiles_s,
                    int xcd_rotate, int vec) {
  hipLaunchKernelGGL((k_indexer_scores_fp8<D, HG>), grid, kThreads, 0, st, q8, qs, k8, ks, w, L, S,
                     H, softmax_scale, out, tiles_t, tiles_s, xcd_rotate, vec);
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

}  // extern "C"
