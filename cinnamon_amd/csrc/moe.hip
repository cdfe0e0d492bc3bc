// MoE dispatch and combine on the device: the permute / unpermute around the grouped
// expert GEMMs (reference src/layers.py:126-157), with no host synchronisation.
//
//   route    : stable counting sort of the flattened top-k expert ids.  perm[r] is the
//              flattened assignment (token * k + slot) at sorted position r, inv is its
//              inverse, starts/ends/counts are the experts' row ranges (int64, on the
//              device: the reference's bincount + cumsum + `.item()`).  Ids outside [0, E)
//              are dropped: inv = -1 for them and perm = -1 at the unused tail positions.
//   gather   : the row-wise quantizer reads x rows through perm (quant.hip,
//              cin_moe_gather_quant_rowwise); its backward is gather_sum here.
//   combine  : out[t] = sum over the token's assignments of sorted_out[r] * score[t, slot],
//              added in increasing sorted position: the order of a sequential
//              scatter_add_ over sorted rows (reference :152-154).  Its backward gives the
//              sorted-row gradient and the score gradient.
//
// Every kernel checks the indices it follows against the sizes it was given, so a bad
// map costs a wrong row, never an access outside the buffers.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "cin_common.h"
#include "cin_runtime.h"

using namespace cin;

// Scratch of cin_moe_route_noalloc: the route's [nblocks, E] per-block counts and bases
// (int32), for callers that cannot allocate.  Each GPU the library runs on holds its own
// copy (4 MiB) until the process ends.  Host code never passes this name to a kernel: it
// is a host-side stand-in, and the device address comes from hipGetSymbolAddress.
constexpr int64_t kRouteScratchElems = (int64_t)1 << 20;
static __device__ __align__(256) int32_t scratch[kRouteScratchElems];

namespace {

constexpr int kRT = 256;           // threads of the route kernels
constexpr int kRounds = 4;         // assignments per thread in a route block
constexpr int kChunk = kRT * kRounds;
constexpr int kMaxExperts = 4096;  // LDS counters of the route kernels
constexpr int kMaxTopK = 16;       // positions a combine thread sorts in registers
constexpr int kRowBatch = 8;       // rows whose pieces a combine wave loads together
constexpr int kStage = 8192;       // int32 entries of the count matrix staged in LDS by the scan

inline bool valid_dtype(int dt) { return dt == CIN_DT_BF16 || dt == CIN_DT_F32 || dt == CIN_DT_F16; }


// Sum over the 64 lanes (a fixed butterfly: the same inputs give the same bits).
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// Per-block expert histogram.
__global__ __launch_bounds__(kRT) void k_route_hist(const int64_t* __restrict__ idx, int64_t A,
                                                    int32_t E, int32_t* __restrict__ blockcounts) {
  __shared__ int hist[kMaxExperts];
  for (int e = threadIdx.x; e < E; e += kRT) hist[e] = 0;
  __syncthreads();
  const int64_t b0 = (int64_t)blockIdx.x * kChunk;
  for (int r = 0; r < kRounds; ++r) {
    const int64_t i = b0 + r * kRT + threadIdx.x;
    if (i < A) {
      const int64_t e = idx[i];
      if (e >= 0 && e < E) atomicAdd(&hist[e], 1);
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += kRT) blockcounts[(int64_t)blockIdx.x * E + e] = hist[e];
}

// Exclusive prefix sum over kRT values held one per thread (Hillis-Steele in LDS); returns
// the thread's exclusive prefix and leaves the total in *total.
__device__ inline int64_t block_exclusive_scan(int64_t v, int64_t* buf, int64_t* total) {
  const int tid = threadIdx.x;
  buf[tid] = v;
  __syncthreads();
#pragma unroll
  for (int off = 1; off < kRT; off <<= 1) {
    const int64_t add = tid >= off ? buf[tid - off] : 0;
    __syncthreads();
    buf[tid] += add;
    __syncthreads();
  }
  const int64_t incl = buf[tid];
  *total = buf[kRT - 1];
  __syncthreads();  // buf is reused by the caller
  return incl - v;
}

// One workgroup: per-expert totals, expert ranges, and each (block, expert)'s first
// sorted position: base = starts[e] + the expert's assignments in earlier blocks.  The
// unused tail of perm (dropped ids) gets -1.
//   1. totals: LDS atomics over the [nblocks, E] count matrix;
//   2. starts: exclusive scan of the totals, each thread owning a run of experts;
//   3. bases: the count matrix in row chunks staged through LDS (coalesced loads and
//      stores); within a chunk, P = kRT / E threads per expert (at least 1) each sum a run
//      of blocks, a scan over each expert's P run sums gives every run its offset, and
//      each run is rewritten as exclusive prefixes; the expert's running total carries
//      across chunks.
__global__ __launch_bounds__(kRT) void k_route_scan(const int32_t* __restrict__ blockcounts,
                                                    int32_t nblocks, int32_t E, int64_t A,
                                                    int32_t* __restrict__ blockbase,
                                                    int64_t* __restrict__ counts,
                                                    int64_t* __restrict__ starts,
                                                    int64_t* __restrict__ ends,
                                                    int64_t* __restrict__ perm) {
  __shared__ int32_t stage[kStage];
  __shared__ int32_t tot32[kMaxExperts];
  __shared__ int64_t run[kMaxExperts];   // starts[e] + the expert's assignments so far
  __shared__ int64_t scan_buf[kRT];
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += kRT) tot32[e] = 0;
  __syncthreads();
  // 1. totals (each total <= A < 2^31)
  const int64_t nall = (int64_t)nblocks * E;
  for (int64_t j = tid; j < nall; j += kRT) atomicAdd(&tot32[j % E], blockcounts[j]);
  __syncthreads();
  // 2. starts: thread t owns experts [t * per, (t + 1) * per)
  const int per = (E + kRT - 1) / kRT;
  const int e0 = tid * per;
  int64_t mine = 0;
  for (int e = e0; e < e0 + per && e < E; ++e) mine += tot32[e];
  int64_t total = 0;
  int64_t acc = block_exclusive_scan(mine, scan_buf, &total);
  for (int e = e0; e < e0 + per && e < E; ++e) {
    const int64_t c = tot32[e];
    starts[e] = acc;
    ends[e] = acc + c;
    counts[e] = c;
    run[e] = acc;
    acc += c;
  }
  // 3. bases
  const int P = E <= kRT ? kRT / E : 1;             // threads per expert
  const int rows_per = kStage / E >= 1 ? kStage / E : 1;  // E <= kMaxExperts <= kStage
  for (int b0 = 0; b0 < nblocks; b0 += rows_per) {
    const int nb = nblocks - b0 < rows_per ? nblocks - b0 : rows_per;
    const int64_t n = (int64_t)nb * E;
    __syncthreads();  // stage[] and run[] are free (previous chunk stored, starts written)
    for (int64_t j = tid; j < n; j += kRT) stage[j] = blockcounts[(int64_t)b0 * E + j];
    __syncthreads();
    const int len = (nb + P - 1) / P;               // blocks per run
    int64_t rsum = 0;
    int e = -1, p = 0;
    if (E <= kRT) {
      if (tid < E * P) {
        e = tid / P;
        p = tid - e * P;
        for (int b = p * len; b < (p + 1) * len && b < nb; ++b) rsum += stage[b * E + e];
      }
      // offsets of the runs within each expert: the P runs of an expert are P
      // consecutive threads, so a segmented scan of width P over scan_buf gives them
      scan_buf[tid] = rsum;
      __syncthreads();
      int64_t off = 0;
      if (e >= 0)
        for (int q = 0; q < p; ++q) off += scan_buf[tid - p + q];
      __syncthreads();
      if (e >= 0) {
        int64_t r = run[e] + off;
        for (int b = p * len; b < (p + 1) * len && b < nb; ++b) {
          const int32_t c = stage[b * E + e];
          stage[b * E + e] = (int32_t)r;
          r += c;
        }
      }
      __syncthreads();
      if (e >= 0 && p == P - 1) run[e] += off + rsum;  // the last run ends the expert's chunk
    } else {
      // E > kRT: one thread walks each expert's blocks
      for (int ee = tid; ee < E; ee += kRT) {
        int64_t r = run[ee];
        for (int b = 0; b < nb; ++b) {
          const int32_t c = stage[b * E + ee];
          stage[b * E + ee] = (int32_t)r;
          r += c;
        }
        run[ee] = r;
      }
    }
    __syncthreads();
    for (int64_t j = tid; j < n; j += kRT) blockbase[(int64_t)b0 * E + j] = stage[j];
  }
  for (int64_t r = total + tid; r < A; r += kRT) perm[r] = -1;
}

// Stable scatter: an assignment's sorted position is its block's first position for its
// expert, plus the assignments of that expert earlier in the block.  One wave per block
// walks the block's assignments in rounds of 64 in index order.  In a round, 12 ballots
// over the bits of the id (E <= 4096) give each lane the mask of lanes holding the same
// id; its rank is the number of those below it, and the group's highest lane advances
// the expert's LDS counter (its read by the group precedes the update in program order).
constexpr int kIdBits = 12;
static_assert((1 << kIdBits) >= kMaxExperts, "ids must fit the ballot bits");
__global__ __launch_bounds__(64) void k_route_scatter(const int64_t* __restrict__ idx, int64_t A,
                                                      int32_t E,
                                                      const int32_t* __restrict__ blockbase,
                                                      int64_t* __restrict__ perm,
                                                      int32_t* __restrict__ inv) {
  __shared__ int running[kMaxExperts];
  const int lane = threadIdx.x;
  for (int e = lane; e < E; e += 64) running[e] = 0;
  __syncthreads();
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const int64_t b0 = (int64_t)blockIdx.x * kChunk;
  for (int r = 0; r < kChunk / 64; ++r) {
    const int64_t i = b0 + r * 64 + lane;
    int e = -1;
    if (i < A) {
      const int64_t v = idx[i];
      e = (v >= 0 && v < E) ? (int)v : -1;
    }
    uint64_t peers = __ballot(e >= 0);
#pragma unroll
    for (int b = 0; b < kIdBits; ++b) {
      const bool bit = (e >> b) & 1;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    if (e >= 0) {
      const int rank = __popcll(peers & below);
      const int64_t pos = (int64_t)blockbase[(int64_t)blockIdx.x * E + e] + running[e] + rank;
      if (pos >= 0 && pos < A) {
        perm[pos] = i;
        inv[i] = (int32_t)pos;
      }
      if (lane == 63 - __clzll(peers)) running[e] += __popcll(peers);
    } else if (i < A) {
      inv[i] = -1;
    }
  }
}

// Sorted positions of token t's assignments in increasing order, with their slots; the
// missing ones (dropped ids, slots past k) get INT32_MAX and sort last.  A fixed
// compare-swap network keeps every index a compile-time one (registers, no scratch).
// Returns the number of valid positions.
__device__ inline int token_positions(const int32_t* __restrict__ inv, int64_t t, int k, int64_t A,
                                      int32_t (&pos)[kMaxTopK], int32_t (&slot)[kMaxTopK]) {
  int n = 0;
#pragma unroll
  for (int j = 0; j < kMaxTopK; ++j) {
    const int32_t p = j < k ? inv[t * k + j] : -1;
    const bool ok = p >= 0 && p < A;
    pos[j] = ok ? p : INT32_MAX;
    slot[j] = j;
    n += ok;
  }
#pragma unroll
  for (int i = 0; i < kMaxTopK - 1; ++i) {
#pragma unroll
    for (int j = 0; j < kMaxTopK - 1 - i; ++j) {
      if (pos[j] > pos[j + 1]) {
        const int32_t tp = pos[j], ts = slot[j];
        pos[j] = pos[j + 1];
        slot[j] = slot[j + 1];
        pos[j + 1] = tp;
        slot[j + 1] = ts;
      }
    }
  }
  return n;
}

template <int DT>
__device__ inline void load4(const void* base, int64_t off, int64_t nv, float (&v)[4]) {
  if constexpr (DT == CIN_DT_F32) {
    const float* p = static_cast<const float*>(base) + off;
    if (nv >= 4 && (((uintptr_t)p) & 15) == 0) {
      const float4 w = *reinterpret_cast<const float4*>(p);
      v[0] = w.x; v[1] = w.y; v[2] = w.z; v[3] = w.w;
    } else {
      for (int e = 0; e < 4; ++e) v[e] = e < nv ? p[e] : 0.0f;
    }
  } else {
    const uint16_t* p = static_cast<const uint16_t*>(base) + off;
    if (nv >= 4 && (((uintptr_t)p) & 7) == 0) {
      const uint2 w = *reinterpret_cast<const uint2*>(p);
      const uint32_t h[2] = {w.x, w.y};
      for (int e = 0; e < 4; ++e) {
        v[e] = half_bits_to_f32(DT, (uint16_t)(h[e >> 1] >> (16 * (e & 1))));
      }
    } else {
      for (int e = 0; e < 4; ++e) v[e] = e < nv ? load_elem(base, DT, off + e) : 0.0f;
    }
  }
}

// 8 consecutive 16-bit values (bf16 or fp16) widened to fp32; one 16-byte load when whole
// and aligned, zeros past nv.
template <int DT>
__device__ inline void load8h(const void* base, int64_t off, int64_t nv, float (&v)[8]) {
  const uint16_t* p = static_cast<const uint16_t*>(base) + off;
  if (nv >= 8 && (((uintptr_t)p) & 15) == 0) {
    const uint4 w = *reinterpret_cast<const uint4*>(p);
    const uint32_t h[4] = {w.x, w.y, w.z, w.w};
    for (int e = 0; e < 8; ++e) v[e] = half_bits_to_f32(DT, (uint16_t)(h[e >> 1] >> (16 * (e & 1))));
  } else {
    for (int e = 0; e < 8; ++e) v[e] = e < nv ? load_elem(base, DT, off + e) : 0.0f;
  }
}

// Word i (compile-time) of a 16-byte piece.
__device__ __forceinline__ uint32_t word_of(const uint4& q, int i) {
  return i == 0 ? q.x : i == 1 ? q.y : i == 2 ? q.z : q.w;
}

// Element e (compile-time) of W consecutive 16-byte pieces holding DT values, widened to fp32.
template <int DT, int W>
__device__ __forceinline__ float piece_elem(const uint4 (&q)[W], int e) {
  if constexpr (DT == CIN_DT_F32) {
    return __uint_as_float(word_of(q[e >> 2], e & 3));
  } else {
    return half_bits_to_f32(DT, (uint16_t)(word_of(q[e >> 3], (e & 7) >> 1) >> (16 * (e & 1))));
  }
}

// W 16-byte pieces of G of a token's rows, pos[j0] .. pos[j0 + G - 1], at byte `cb` of
// each row (rows `rb` bytes apart), every load issued before any result is used: one wave
// keeps G W loads in flight instead of one.  Rows at or past n load row pos[j0] again
// (j0 < n); their pieces are never used.  Needs 16-byte aligned pieces.
template <int G, int W>
__device__ __forceinline__ void load_rows(const void* base, int64_t cb, int64_t rb,
                                          const int32_t (&pos)[kMaxTopK], int j0, int n,
                                          uint4 (&raw)[G][W]) {
#pragma unroll
  for (int jj = 0; jj < G; ++jj) {
    const int64_t r = j0 + jj < n ? pos[j0 + jj] : pos[j0];
    const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(base) + r * rb + cb);
#pragma unroll
    for (int u = 0; u < W; ++u) raw[jj][u] = p[u];
  }
}

template <int OT>
__device__ inline void store4(void* base, int64_t off, int64_t nv, const float (&v)[4]) {
  if constexpr (OT == CIN_DT_F32) {
    float* p = static_cast<float*>(base) + off;
    if (nv >= 4 && (((uintptr_t)p) & 15) == 0) {
      *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      for (int e = 0; e < 4; ++e)
        if (e < nv) p[e] = v[e];
    }
  } else {
    uint16_t* p = static_cast<uint16_t*>(base) + off;
    uint32_t b[4];
    for (int e = 0; e < 4; ++e) b[e] = f32_to_half_bits(OT, v[e]);
    if (nv >= 4 && (((uintptr_t)p) & 7) == 0) {
      *reinterpret_cast<uint2*>(p) = make_uint2(b[0] | (b[1] << 16), b[2] | (b[3] << 16));
    } else {
      for (int e = 0; e < 4; ++e)
        if (e < nv) p[e] = (uint16_t)b[e];
    }
  }
}

// dx[t] = sum of g[r] over token t's sorted positions r (increasing r), fp32 sums.
// One wave per token; lane l covers columns 8 l + 512 i of fp32 rows and 16 l + 1024 i of
// 16-bit rows (two 16-byte pieces per row and step: the rows sit at scattered sorted
// positions, and 2 KB runs per row read ~6-10% faster than 1 KB runs).
template <int GT, int OT>
__global__ __launch_bounds__(kRT) void k_moe_gather_sum(const void* __restrict__ g, int64_t sgm,
                                                        const int32_t* __restrict__ inv,
                                                        int64_t T, int k, int64_t A, int64_t N,
                                                        void* __restrict__ out, int64_t som) {
  const int lane = threadIdx.x & 63;
  const int64_t t = ((int64_t)blockIdx.x * kRT + threadIdx.x) >> 6;
  if (t >= T) return;  // uniform per wave
  int32_t pos[kMaxTopK], slot[kMaxTopK];
  const int n = token_positions(inv, t, k, A, pos, slot);
  // whole chunks of rows whose pieces are 16-byte aligned take the batched loads
  const bool vec = ((((uintptr_t)g) & 15) == 0) && ((sgm * (GT == CIN_DT_F32 ? 4 : 2)) & 15) == 0;
  if constexpr (GT == CIN_DT_F32) {
    for (int64_t c = (int64_t)lane * 8; c < N; c += 512) {
      float acc[2][4] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
      if (vec && c + 8 <= N) {
#pragma unroll
        for (int j0 = 0; j0 < kMaxTopK; j0 += kRowBatch) {
          if (j0 < n) {
            uint4 raw[kRowBatch][2];
            load_rows<kRowBatch, 2>(g, c * 4, sgm * 4, pos, j0, n, raw);
#pragma unroll
            for (int jj = 0; jj < kRowBatch; ++jj)
              if (j0 + jj < n)
                for (int e = 0; e < 8; ++e) acc[e >> 2][e & 3] = acc[e >> 2][e & 3] + piece_elem<GT, 2>(raw[jj], e);
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j) {
          if (j < n) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              float v[4];
              load4<GT>(g, (int64_t)pos[j] * sgm + c + 4 * u, N - c - 4 * u, v);
              for (int e = 0; e < 4; ++e) acc[u][e] = acc[u][e] + v[e];
            }
          }
        }
      }
      store4<OT>(out, t * som + c, N - c, acc[0]);
      store4<OT>(out, t * som + c + 4, N - c - 4, acc[1]);
    }
  } else {
    // 16-bit rows: 16 columns per lane (two 16-byte loads), 2 KB runs per row
    for (int64_t c = (int64_t)lane * 16; c < N; c += 1024) {
      float acc[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
      if (vec && c + 16 <= N) {
#pragma unroll
        for (int j0 = 0; j0 < kMaxTopK; j0 += kRowBatch) {
          if (j0 < n) {
            uint4 raw[kRowBatch][2];
            load_rows<kRowBatch, 2>(g, c * 2, sgm * 2, pos, j0, n, raw);
#pragma unroll
            for (int jj = 0; jj < kRowBatch; ++jj)
              if (j0 + jj < n)
                for (int e = 0; e < 16; ++e) acc[e] = acc[e] + piece_elem<GT, 2>(raw[jj], e);
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j) {
          if (j < n) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              float v[8];
              load8h<GT>(g, (int64_t)pos[j] * sgm + c + 8 * u, N - c - 8 * u, v);
              for (int e = 0; e < 8; ++e) acc[8 * u + e] = acc[8 * u + e] + v[e];
            }
          }
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float a4[4] = {acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
        store4<OT>(out, t * som + c + 4 * q, N - c - 4 * q, a4);
      }
    }
  }
}

template <int ST>
__device__ inline float score_at(const void* s, int64_t off) {
  return load_elem(s, ST, off);
}

// out[t] = sum over the token's positions r (increasing) of y[r] * score[t, slot(r)]:
// a product then an add, both rounded (built without contraction), fp32.  One wave per
// token; lane l covers columns 8 l + 512 i of fp32 rows (as k_moe_gather_sum) and
// 16 l + 1024 i of 16-bit rows: 2 KB runs per scattered row either way.
template <int YT, int ST>
__global__ __launch_bounds__(kRT) void k_moe_combine(const void* __restrict__ y, int64_t sym,
                                                     const void* __restrict__ scores,
                                                     int64_t ssm, const int32_t* __restrict__ inv,
                                                     int64_t T, int k, int64_t A, int64_t N,
                                                     float* __restrict__ out, int64_t som) {
  const int lane = threadIdx.x & 63;
  const int64_t t = ((int64_t)blockIdx.x * kRT + threadIdx.x) >> 6;
  if (t >= T) return;  // uniform per wave
  int32_t pos[kMaxTopK], slot[kMaxTopK];
  const int n = token_positions(inv, t, k, A, pos, slot);
  float w[kMaxTopK];
#pragma unroll
  for (int j = 0; j < kMaxTopK; ++j) w[j] = j < n ? score_at<ST>(scores, t * ssm + slot[j]) : 0.0f;
  // whole chunks of rows whose pieces are 16-byte aligned take the batched loads
  const bool vec = ((((uintptr_t)y) & 15) == 0) && ((sym * (YT == CIN_DT_F32 ? 4 : 2)) & 15) == 0;
  if constexpr (YT == CIN_DT_F32) {
    for (int64_t c = (int64_t)lane * 8; c < N; c += 512) {
      float acc[2][4] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
      if (vec && c + 8 <= N) {
#pragma unroll
        for (int j0 = 0; j0 < kMaxTopK; j0 += kRowBatch) {
          if (j0 < n) {
            uint4 raw[kRowBatch][2];
            load_rows<kRowBatch, 2>(y, c * 4, sym * 4, pos, j0, n, raw);
#pragma unroll
            for (int jj = 0; jj < kRowBatch; ++jj)
              if (j0 + jj < n)
                for (int e = 0; e < 8; ++e)
                  acc[e >> 2][e & 3] = acc[e >> 2][e & 3] + piece_elem<YT, 2>(raw[jj], e) * w[j0 + jj];
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j) {
          if (j < n) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              float v[4];
              load4<YT>(y, (int64_t)pos[j] * sym + c + 4 * u, N - c - 4 * u, v);
              for (int e = 0; e < 4; ++e) acc[u][e] = acc[u][e] + v[e] * w[j];
            }
          }
        }
      }
      store4<CIN_DT_F32>(out, t * som + c, N - c, acc[0]);
      store4<CIN_DT_F32>(out, t * som + c + 4, N - c - 4, acc[1]);
    }
  } else {
    // 16-bit rows: 16 columns per lane (two 16-byte loads), the same 2 KB runs per row
    for (int64_t c = (int64_t)lane * 16; c < N; c += 1024) {
      float acc[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
      if (vec && c + 16 <= N) {
#pragma unroll
        for (int j0 = 0; j0 < kMaxTopK; j0 += kRowBatch) {
          if (j0 < n) {
            uint4 raw[kRowBatch][2];
            load_rows<kRowBatch, 2>(y, c * 2, sym * 2, pos, j0, n, raw);
#pragma unroll
            for (int jj = 0; jj < kRowBatch; ++jj)
              if (j0 + jj < n)
                for (int e = 0; e < 16; ++e) acc[e] = acc[e] + piece_elem<YT, 2>(raw[jj], e) * w[j0 + jj];
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j) {
          if (j < n) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              float v[8];
              load8h<YT>(y, (int64_t)pos[j] * sym + c + 8 * u, N - c - 8 * u, v);
              for (int e = 0; e < 8; ++e) acc[8 * u + e] = acc[8 * u + e] + v[e] * w[j];
            }
          }
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float a4[4] = {acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
        store4<CIN_DT_F32>(out, t * som + c + 4 * q, N - c - 4 * q, a4);
      }
    }
  }
}

// Combine backward, both gradients in one pass per token (one wave): the token's dout row
// is read once; for each of its sorted positions r (increasing), y[r] is read for the score
// gradient dscore[t, j] = sum_c dout[t, c] * y[r, c] (lane l over columns 8 l + 512 i, then
// a wave sum) and dy[r] = dout[t] * score[t, j] is written in dy's dtype DT (RNE of the
// fp32 product).  Slots whose assignment was dropped get dscore 0; the dy rows no
// assignment maps to are zeroed by k_moe_zero_unmapped_rows.
template <int YT, int DT>
__global__ __launch_bounds__(kRT) void k_moe_combine_bwd_tokens(
    const float* __restrict__ dout, int64_t sdm, const void* __restrict__ y, int64_t sym,
    const void* __restrict__ scores, int st, int64_t ssm, const int32_t* __restrict__ inv, int64_t T,
    int k, int64_t A, int64_t N, void* __restrict__ dy, int64_t sdym, float* __restrict__ dscores) {
  const int lane = threadIdx.x & 63;
  const int64_t t = ((int64_t)blockIdx.x * kRT + threadIdx.x) >> 6;
  if (t >= T) return;  // uniform per wave
  int32_t pos[kMaxTopK], slot[kMaxTopK];
  const int n = token_positions(inv, t, k, A, pos, slot);
  float w[kMaxTopK], acc[kMaxTopK];
#pragma unroll
  for (int j = 0; j < kMaxTopK; ++j) {
    w[j] = j < n ? load_elem(scores, st, t * ssm + slot[j]) : 0.0f;
    acc[j] = 0.0f;
  }
  const int64_t db = t * sdm;
  // 16-bit rows whose 16-byte pieces are aligned: up to kRowBatch rows' pieces are loaded
  // together before any is used (the per-row form has one row's load in flight per wave);
  // the same products and sums in the same order either way
  const bool vec = YT != CIN_DT_F32 && ((((uintptr_t)y) & 15) == 0) && (((sym * 2) & 15) == 0);
  for (int64_t c = (int64_t)lane * 8; c < N; c += 512) {
    float a[2][4];
    load4<CIN_DT_F32>(dout, db + c, N - c, a[0]);
    load4<CIN_DT_F32>(dout, db + c + 4, N - c - 4, a[1]);
    if constexpr (YT != CIN_DT_F32) {
      if (vec && c + 8 <= N) {
#pragma unroll
        for (int j0 = 0; j0 < kMaxTopK; j0 += kRowBatch) {
          if (j0 < n) {
            uint4 raw[kRowBatch][1];
            load_rows<kRowBatch, 1>(y, c * 2, sym * 2, pos, j0, n, raw);
#pragma unroll
            for (int jj = 0; jj < kRowBatch; ++jj) {
              const int j = j0 + jj;
              if (j < n) {
                for (int e = 0; e < 8; ++e) acc[j] += a[e >> 2][e & 3] * piece_elem<YT, 1>(raw[jj], e);
                float d0[4], d1[4];
                for (int e = 0; e < 4; ++e) {
                  d0[e] = a[0][e] * w[j];
                  d1[e] = a[1][e] * w[j];
                }
                const int64_t ob = (int64_t)pos[j] * sdym;
                store4<DT>(dy, ob + c, N - c, d0);
                store4<DT>(dy, ob + c + 4, N - c - 4, d1);
              }
            }
          }
        }
        continue;
      }
    }
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) {
      if (j < n) {
        const int64_t yb = (int64_t)pos[j] * sym;
        float b[8];
        if constexpr (YT == CIN_DT_F32) {
          float b0[4], b1[4];
          load4<CIN_DT_F32>(y, yb + c, N - c, b0);
          load4<CIN_DT_F32>(y, yb + c + 4, N - c - 4, b1);
          for (int e = 0; e < 4; ++e) {
            b[e] = b0[e];
            b[4 + e] = b1[e];
          }
        } else {
          load8h<YT>(y, yb + c, N - c, b);
        }
        for (int e = 0; e < 8; ++e) acc[j] += a[e >> 2][e & 3] * b[e];
        float d0[4], d1[4];
        for (int e = 0; e < 4; ++e) {
          d0[e] = a[0][e] * w[j];
          d1[e] = a[1][e] * w[j];
        }
        const int64_t ob = (int64_t)pos[j] * sdym;
        store4<DT>(dy, ob + c, N - c, d0);
        store4<DT>(dy, ob + c + 4, N - c - 4, d1);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < kMaxTopK; ++j) {
    if (j < n) {
      const float sum = wave_sum(acc[j]);
      if (lane == 0) dscores[t * k + slot[j]] = sum;
    }
  }
  for (int j = lane; j < k; j += 64) {
    const int32_t p = inv[t * k + j];
    if (p < 0 || p >= A) dscores[t * k + j] = 0.0f;
  }
}

// dy rows that no assignment maps to (perm[r] < 0) are zero.  One wave per row; the rows
// an assignment maps to exit at once.
template <int DT>
__global__ __launch_bounds__(kRT) void k_moe_zero_unmapped_rows(const int64_t* __restrict__ perm,
                                                                int64_t T, int k, int64_t A,
                                                                int64_t N, void* __restrict__ dy,
                                                                int64_t sdym) {
  const int lane = threadIdx.x & 63;
  const int64_t r = ((int64_t)blockIdx.x * kRT + threadIdx.x) >> 6;
  if (r >= A) return;
  const int64_t i = perm[r];
  if (i >= 0 && i < T * k) return;  // uniform per wave
  const float z[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int64_t c = (int64_t)lane * 4; c < N; c += 256) store4<DT>(dy, r * sdym + c, N - c, z);
}

// The route's three launches over a caller's int32 workspace of ws_elems entries.
int route_launch(const char* name, const int64_t* idx, int64_t T, int64_t k, int64_t E, int64_t* perm,
                 int32_t* inv, int64_t* counts, int64_t* starts, int64_t* ends, int32_t* workspace,
                 int64_t workspace_elems, void* stream) {
  CIN_CHECK_ARG(T >= 0 && k >= 1 && E >= 1, "%s: need T >= 0, k >= 1, E >= 1", name);
  CIN_CHECK_ARG(E <= kMaxExperts, "%s: at most %d experts", name, kMaxExperts);
  const int64_t A = T * k;
  CIN_CHECK_ARG(A < ((int64_t)1 << 31), "%s: T*k must fit in 31 bits", name);
  CIN_CHECK_ARG(idx && perm && inv && counts && starts && ends && (A == 0 || workspace),
                "%s: null pointer", name);
  const int64_t nblocks = cdiv(A, kChunk);
  CIN_CHECK_ARG(workspace_elems >= 2 * nblocks * E, "%s: workspace needs %lld int32", name,
                (long long)(2 * nblocks * E));
  CIN_CHECK_ARG(nblocks < ((int64_t)1 << 20), "%s: too many assignments", name);
  hipStream_t s = static_cast<hipStream_t>(stream);
  int32_t* blockbase = workspace + nblocks * E;
  if (nblocks > 0) hipLaunchKernelGGL(k_route_hist, (unsigned)nblocks, kRT, 0, s, idx, A, (int32_t)E, workspace);
  hipLaunchKernelGGL(k_route_scan, 1, kRT, 0, s, workspace, (int32_t)nblocks, (int32_t)E, A, blockbase,
                     counts, starts, ends, perm);
  if (nblocks > 0)
    hipLaunchKernelGGL(k_route_scatter, (unsigned)nblocks, 64, 0, s, idx, A, (int32_t)E, blockbase,
                       perm, inv);
  return cin_check_launch(name);
}

// Device address of `scratch` on the current device, looked up once per device (with that
// device current) and kept.  Every call on one GPU shares that GPU's array: the route
// overwrites all of the entries it reads, so nothing needs clearing between calls, and
// calls that overlap on one GPU (two streams, or two host threads) race on it.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
int32_t* g_scratch_ptr[kMaxDevices] = {};

int route_scratch(int32_t** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return cin_set_error(CIN_ERR_HIP, "moe_route_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return cin_set_error(CIN_ERR_UNSUPPORTED, "moe_route_noalloc: device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return cin_set_error(CIN_ERR_HIP, "moe_route_noalloc: hipGetSymbolAddress(scratch): %s",
                           hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<int32_t*>(p);
  }
  *out = g_scratch_ptr[dev];
  return CIN_OK;
}

}  // namespace

extern "C" {

int cin_moe_route(const int64_t* idx, int64_t T, int64_t k, int64_t E, int64_t* perm, int32_t* inv,
                  int64_t* counts, int64_t* starts, int64_t* ends, int32_t* workspace,
                  int64_t workspace_elems, void* stream) {
  return route_launch("moe_route", idx, T, k, E, perm, inv, counts, starts, ends, workspace,
                      workspace_elems, stream);
}

int cin_moe_route_noalloc(const int64_t* idx, int64_t T, int64_t k, int64_t E, int64_t* perm,
                          int32_t* inv, int64_t* counts, int64_t* starts, int64_t* ends,
                          void* stream) {
  CIN_CHECK_ARG(T >= 0 && k >= 1 && E >= 1, "moe_route_noalloc: need T >= 0, k >= 1, E >= 1");
  // bound E and T*k before forming the scratch size, so its product cannot overflow
  CIN_CHECK_ARG(E <= kMaxExperts, "moe_route_noalloc: at most %d experts", kMaxExperts);
  CIN_CHECK_ARG(T <= (((int64_t)1 << 31) - 1) / k, "moe_route_noalloc: T*k must fit in 31 bits");
  const int64_t need = 2 * cdiv(T * k, kChunk) * E;
  CIN_CHECK_ARG(need <= kRouteScratchElems,
                "moe_route_noalloc: needs %lld int32 of scratch (2 * ceil(T*k / %d) * E), the "
                "library holds %lld; use cin_moe_route with a workspace",
                (long long)need, kChunk, (long long)kRouteScratchElems);
  int32_t* ws = nullptr;
  const int rc = route_scratch(&ws);
  if (rc != CIN_OK) return rc;
  return route_launch("moe_route_noalloc", idx, T, k, E, perm, inv, counts, starts, ends, ws,
                      kRouteScratchElems, stream);
}

int cin_moe_route_workspace(int64_t T, int64_t k, int64_t E) {
  if (T < 0 || k < 1 || E < 1) return 0;
  if (E > kMaxExperts || T > (((int64_t)1 << 31) - 1) / k) return INT32_MAX;  // the route rejects these
  const int64_t n = 2 * cdiv(T * k, kChunk) * E;
  return n > INT32_MAX ? INT32_MAX : (int)n;
}

int cin_moe_gather_sum(const void* g, int g_dtype, int64_t sgm, const int32_t* inv, int64_t T,
                       int64_t k, int64_t A, int64_t N, void* out, int out_dtype, int64_t som,
                       void* stream) {
  CIN_CHECK_ARG(valid_dtype(g_dtype) && valid_dtype(out_dtype), "moe_gather_sum: unsupported dtype");
  CIN_CHECK_ARG(T >= 0 && k >= 1 && k <= kMaxTopK && A >= 0 && N >= 0,
                "moe_gather_sum: need k in [1, %d] and non-negative sizes", kMaxTopK);
  if (T == 0 || N == 0) return CIN_OK;
  CIN_CHECK_ARG(g && inv && out && sgm >= N && som >= N, "moe_gather_sum: bad pointers or strides");
  CIN_CHECK_ARG(cdiv(T * 64, kRT) < ((int64_t)1 << 31), "moe_gather_sum: grid too large");
  const unsigned grid = (unsigned)cdiv(T * 64, kRT);  // one wave per token
  hipStream_t s = static_cast<hipStream_t>(stream);
#define CIN_GS(GT, OT) \
  hipLaunchKernelGGL((k_moe_gather_sum<GT, OT>), grid, kRT, 0, s, g, sgm, inv, T, (int)k, A, N, out, som)
  if (g_dtype == CIN_DT_F32) {
    if (out_dtype == CIN_DT_F32) CIN_GS(CIN_DT_F32, CIN_DT_F32);
    else if (out_dtype == CIN_DT_BF16) CIN_GS(CIN_DT_F32, CIN_DT_BF16);
    else CIN_GS(CIN_DT_F32, CIN_DT_F16);
  } else if (g_dtype == CIN_DT_BF16) {
    if (out_dtype == CIN_DT_F32) CIN_GS(CIN_DT_BF16, CIN_DT_F32);
    else if (out_dtype == CIN_DT_BF16) CIN_GS(CIN_DT_BF16, CIN_DT_BF16);
    else CIN_GS(CIN_DT_BF16, CIN_DT_F16);
  } else {
    if (out_dtype == CIN_DT_F32) CIN_GS(CIN_DT_F16, CIN_DT_F32);
    else if (out_dtype == CIN_DT_BF16) CIN_GS(CIN_DT_F16, CIN_DT_BF16);
    else CIN_GS(CIN_DT_F16, CIN_DT_F16);
  }
#undef CIN_GS
  return cin_check_launch("moe_gather_sum");
}

int cin_moe_combine(const void* y, int y_dtype, int64_t sym, const void* scores, int s_dtype,
                    int64_t ssm, const int32_t* inv, int64_t T, int64_t k, int64_t A, int64_t N,
                    float* out, int64_t som, void* stream) {
  CIN_CHECK_ARG(valid_dtype(s_dtype) && valid_dtype(y_dtype), "moe_combine: unsupported dtype (y %d, scores %d)",
                y_dtype, s_dtype);
  CIN_CHECK_ARG(T >= 0 && k >= 1 && k <= kMaxTopK && A >= 0 && N >= 0,
                "moe_combine: need k in [1, %d] and non-negative sizes", kMaxTopK);
  if (T == 0 || N == 0) return CIN_OK;
  CIN_CHECK_ARG(y && scores && inv && out && sym >= N && som >= N && ssm >= k,
                "moe_combine: bad pointers or strides");
  CIN_CHECK_ARG(cdiv(T * 64, kRT) < ((int64_t)1 << 31), "moe_combine: grid too large");
  const unsigned grid = (unsigned)cdiv(T * 64, kRT);  // one wave per token
  hipStream_t s = static_cast<hipStream_t>(stream);
#define CIN_COMB(YT, ST) \
  hipLaunchKernelGGL((k_moe_combine<YT, ST>), grid, kRT, 0, s, y, sym, scores, ssm, inv, T, (int)k, A, N, out, som)
#define CIN_COMB_S(YT)                          \
  if (s_dtype == CIN_DT_F32) CIN_COMB(YT, CIN_DT_F32);       \
  else if (s_dtype == CIN_DT_BF16) CIN_COMB(YT, CIN_DT_BF16); \
  else CIN_COMB(YT, CIN_DT_F16);
  if (y_dtype == CIN_DT_F32) {
    CIN_COMB_S(CIN_DT_F32)
  } else if (y_dtype == CIN_DT_F16) {
    CIN_COMB_S(CIN_DT_F16)
  } else {
    CIN_COMB_S(CIN_DT_BF16)
  }
#undef CIN_COMB_S
#undef CIN_COMB
  return cin_check_launch("moe_combine");
}

int cin_moe_combine_backward(const float* dout, int64_t sdm, const void* y, int y_dtype, int64_t sym,
                             const void* scores, int s_dtype, int64_t ssm, const int64_t* perm,
                             const int32_t* inv, int64_t T, int64_t k, int64_t A, int64_t N,
                             void* dy, int dy_dtype, int64_t sdym, float* dscores, void* stream) {
  CIN_CHECK_ARG(valid_dtype(s_dtype) && valid_dtype(y_dtype) && valid_dtype(dy_dtype),
                "moe_combine_backward: unsupported dtype (y %d, scores %d, dy %d)", y_dtype, s_dtype,
                dy_dtype);
  CIN_CHECK_ARG(T >= 0 && k >= 1 && A >= 0 && N >= 0, "moe_combine_backward: bad sizes");
  CIN_CHECK_ARG(A <= T * k, "moe_combine_backward: more sorted rows than assignments");
  CIN_CHECK_ARG(dout && y && scores && perm && inv && dy && dscores, "moe_combine_backward: null pointer");
  CIN_CHECK_ARG(sdm >= N && sym >= N && sdym >= N && ssm >= k, "moe_combine_backward: bad strides");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (A > 0 && N > 0) {
    CIN_CHECK_ARG(cdiv(A * 64, kRT) < ((int64_t)1 << 31), "moe_combine_backward: grid too large");
    const unsigned grid = (unsigned)cdiv(A * 64, kRT);  // one wave per sorted row
    if (dy_dtype == CIN_DT_F32)
      hipLaunchKernelGGL(k_moe_zero_unmapped_rows<CIN_DT_F32>, grid, kRT, 0, s, perm, T, (int)k, A, N, dy, sdym);
    else if (dy_dtype == CIN_DT_F16)
      hipLaunchKernelGGL(k_moe_zero_unmapped_rows<CIN_DT_F16>, grid, kRT, 0, s, perm, T, (int)k, A, N, dy, sdym);
    else
      hipLaunchKernelGGL(k_moe_zero_unmapped_rows<CIN_DT_BF16>, grid, kRT, 0, s, perm, T, (int)k, A, N, dy, sdym);
  }
  if (T > 0) {
    CIN_CHECK_ARG(k <= kMaxTopK, "moe_combine_backward: k must be at most %d", kMaxTopK);
    CIN_CHECK_ARG(cdiv(T * 64, kRT) < ((int64_t)1 << 31), "moe_combine_backward: grid too large");
    const unsigned grid = (unsigned)cdiv(T * 64, kRT);  // one wave per token
#define CIN_TOK(YT, DT)                                                                          \
  hipLaunchKernelGGL((k_moe_combine_bwd_tokens<YT, DT>), grid, kRT, 0, s, dout, sdm, y, sym, scores, \
                     s_dtype, ssm, inv, T, (int)k, A, N, dy, sdym, dscores)
#define CIN_TOK_D(YT)                                        \
  if (dy_dtype == CIN_DT_F32) CIN_TOK(YT, CIN_DT_F32);       \
  else if (dy_dtype == CIN_DT_BF16) CIN_TOK(YT, CIN_DT_BF16); \
  else CIN_TOK(YT, CIN_DT_F16);
    if (y_dtype == CIN_DT_F32) {
      CIN_TOK_D(CIN_DT_F32)
    } else if (y_dtype == CIN_DT_F16) {
      CIN_TOK_D(CIN_DT_F16)
    } else {
      CIN_TOK_D(CIN_DT_BF16)
    }
#undef CIN_TOK_D
#undef CIN_TOK
  }
  return cin_check_launch("moe_combine_backward");
}

}  // extern "C"
