// Shared device helpers for the cinnamon FP8 path on gfx950 (CDNA4).
//
// Arithmetic restated from the reference quantizers
// (reference src/kernels.py:50-62 row-wise, :111-123 block-wise):
//   amax  = maxnum-reduction of |x| over the tile (NaN elements ignored, as
//           Triton's tl.max / tl.maximum lower to maxnum)
//   amax  = maxnum(amax, fp32(1e-4)) for every input dtype: Triton's tl.max widens
//           bf16/fp16 to fp32 before it reduces (triton/language/standard.py, max),
//           so tl.maximum(abs_max, 1e-4) compares two fp32 values
//   scale = fp32(amax) / 448      (IEEE fp32 division), or with round_scale
//           exp2(ceil(log2(amax / 448)))
//   code  = e4m3fn_rne(minnum(maxnum(x / scale, -448), 448))
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/cinnamon_fp8.h"

namespace cin {

constexpr float kFp8Max = 448.0f;
// Floor of the tile amax: fp32(1e-4) whatever the input dtype.
constexpr float kFloorF32 = 9.99999974737875163555e-05f;   // fp32(1e-4)

__host__ __device__ inline float amax_floor(int /*dtype*/) { return kFloorF32; }

// Scale from a floored amax.  round_scale follows torch.exp2(torch.ceil(torch.log2(v)))
// in fp32, where torch's log2 is correctly rounded over the reachable range: for
// v = 2^k * (1 + m * 2^-23), m > 0, fl32(log2 v) stays equal to k (so the ceiling is
// k, not k + 1) while m is below a threshold fixed by the fp32 spacing just above
// (k >= 0) or just below (k < 0) the integer k.
__device__ inline float compute_scale(float amax, bool round_scale) {
  float v = amax / kFp8Max;
  if (!round_scale) return v;
  uint32_t b = __float_as_uint(v);
  if (!(v > 0.0f) || b >= 0x7f800000u) return v;   // inf/NaN pass through (exp2(inf) = inf)
  int k = (int)(b >> 23) - 127;
  uint32_t m = b & 0x7fffffu;
  if (k < -126 + 1) {
    // Not reachable: amax >= 1e-4 keeps v above 2^-22.
    return v;
  }
  int e = k;
  if (m != 0) {
    int a = k > 0 ? k : (k < 0 ? -k - 1 : 0);
    int j = a ? 31 - __builtin_clz((unsigned)a) : -1;
    uint32_t t = j <= 1 ? 1u : (j == 2 ? 2u : (j == 3 ? 3u : (j == 4 ? 6u : (j == 5 ? 12u : 23u))));
    e = (m >= t) ? k + 1 : k;
  }
  if (e > 127) return __uint_as_float(0x7f800000u);
  return __uint_as_float((uint32_t)(e + 127) << 23);
}

// RN(x / s) for a finite scale s > 0 from r = RN(1 / s), without a division:
//   q0 = RN(x * r)                (within 1.5 fp32 ulp of x / s)
//   q  = RN(q - RN(q * s - x) * r)  (one fma pair per step; the residual is exact)
// This is Markstein's final step: once q is within 1 ulp of x / s and r within 1/2 ulp
// of 1 / s, one more step returns the correctly rounded quotient, so two steps are
// exact for any fp32 x.  For x and amax that are bf16 or fp16 values (s = RN(amax/448),
// |x| <= amax) one step already is: checked against the IEEE division for every pair of
// mantissas over every exponent gap down to 2^-30, and for every bf16 and fp16 x below
// the floor with s = RN(fp32(1e-4) / 448) (a floored tile).  STEPS is therefore 1 for 16-bit
// inputs and 2 for fp32.  The residual is formed as q * s - x, not x - q * s, so that
// x = -0 keeps its sign (-0 - (+0) * r = -0; the other order would add +0 to -0).  An
// infinite scale (infinite amax) is left to the caller.
template <int STEPS>
__device__ inline float div_by_scale(float x, float s, float r) {
  float q = x * r;
#pragma unroll
  for (int i = 0; i < STEPS; ++i) q = __builtin_fmaf(-__builtin_fmaf(q, s, -x), r, q);
  return q;
}

template <int DT>
constexpr int kDivSteps = DT == CIN_DT_F32 ? 2 : 1;

// Clamp with maxnum/minnum semantics: NaN maps to -448 like the reference's
// tl.minimum(tl.maximum(x, -448), 448).
__device__ inline float clamp448(float y) {
  return fminf(fmaxf(y, -kFp8Max), kFp8Max);
}

// Two fp32 (already clamped to [-448, 448]) -> two OCP e4m3fn codes in the low
// 16 bits, round-to-nearest-even.  gfx950's conversion was checked bit-exact
// against a software RNE over every finite magnitude <= 448.
__device__ inline uint32_t cvt2_e4m3(float a, float b) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu;
}
// Four clamped fp32 -> packed 4 codes (byte i = value i).
__device__ inline uint32_t cvt4_e4m3(float a, float b, float c, float d) {
  int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
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

// 1 / d for d >= 1 (the sigmoid's 1 / (1 + e^-x)), equal to the IEEE division 1.0f / d:
// v_rcp_f32 followed by one Newton step r + r (1 - d r) in FMAs returns the correctly rounded
// reciprocal for every fp32 d in [1, 2^126).  Above 2^126 the reciprocal is a denormal, which
// v_rcp_f32 flushes: those d, infinity and NaN take the division (a branch that sigmoid inputs
// above -87 never enter).  tests/test_gpu_recip.py compares recip_ge1 with the division on
// the device for every fp32 d >= 1.
// recip_ge1_fast is the first form alone: callers that take it for d outside [1, 2^126)
// must redo those values with the division (d >= 1 has bits >= 0x3f800000, and every d at or
// above 2^126, infinity and NaN have bits >= kRecipFastLimitBits, so an unsigned max of the
// bits tells whether any value needs it).
constexpr uint32_t kRecipFastLimitBits = 0x7e800000u;  // 2^126
__device__ inline float recip_ge1_fast(float d) {
  const float r = __builtin_amdgcn_rcpf(d);
  return __builtin_fmaf(__builtin_fmaf(-d, r, 1.0f), r, r);
}
__device__ inline float recip_ge1(float d) {
  if (__builtin_expect(__float_as_uint(d) < kRecipFastLimitBits, 1)) return recip_ge1_fast(d);
  return 1.0f / d;
}

// e4m3fn code -> fp32 (exact).
__device__ inline float e4m3_to_f32(uint32_t c) {
  uint32_t s = (c & 0x80u) << 24;
  uint32_t e = (c >> 3) & 0xfu;
  uint32_t m = c & 0x7u;
  if (e == 0xfu && m == 0x7u) return __uint_as_float(s | 0x7fc00000u);
  if (e == 0) {
    const float v = (float)m * 0.001953125f;  // m * 2^-9, exact
    return s ? -v : v;
  }
  return __uint_as_float(s | ((e + 120u) << 23) | (m << 20));
}

__device__ inline float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ inline float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Two fp32 values -> packed bf16 bits (lo in bits 0-15), by gfx950's v_cvt_pk_bf16_f32:
// round to nearest even, a NaN kept quiet with its sign and upper payload (bits 16-31 of
// the input, quiet bit set), denormals kept.  That is, per value: u = bits of f; NaN ->
// (u >> 16) | 0x40, else (u + 0x7fff + ((u >> 16) & 1)) >> 16 -- the instruction gives
// exactly this on every one of the 2^32 inputs (checked exhaustively on an MI355X against
// the integer formula, which is what this file computed before).  gfx950 has no
// instruction that fuses a multiply-add with a bf16 rounding, so unlike the fp16 case
// below the inputs need no pinning as fp32 values.
typedef __bf16 cin_bf16x2 __attribute__((ext_vector_type(2)));
__device__ inline uint32_t f32x2_to_bf16x2_bits(float lo, float hi) {
  const cin_bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// fp32 -> bf16 bits with round-to-nearest-even (NaN kept quiet), as above.
__device__ inline uint32_t f32_to_bf16_bits(float f) {
  return f32x2_to_bf16x2_bits(f, 0.0f) & 0xffffu;
}

// fp32 -> fp16 bits, round to nearest even (overflow to inf, as a torch .half()).  The
// empty asm pins f as an fp32 value: otherwise the compiler may fuse the multiply or FMA
// that produced it with this conversion into one mixed-precision instruction (one rounding
// of the exact result to fp16), which differs from fp32-then-fp16 at fp32 ties.
__device__ inline uint16_t f32_to_f16_bits(float f) {
  asm volatile("" : "+v"(f));
  const _Float16 h = (_Float16)f;
  uint16_t b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}

// fp32 -> the bits of a 16-bit output dtype (CIN_DT_F16 or CIN_DT_BF16), RNE.
__device__ inline uint32_t f32_to_half_bits(int dt, float f) {
  return dt == CIN_DT_F16 ? (uint32_t)f32_to_f16_bits(f) : f32_to_bf16_bits(f);
}

// Two fp32 values -> packed bits (lo in bits 0-15) of the 16-bit dtype OUT, RNE.  OUT is
// a template argument so that loops over many values carry no per-value dtype test.
template <int OUT>
__device__ inline uint32_t f32x2_to_half2_bits(float lo, float hi) {
  static_assert(OUT == CIN_DT_BF16 || OUT == CIN_DT_F16, "16-bit output dtype");
  if constexpr (OUT == CIN_DT_BF16)
    return f32x2_to_bf16x2_bits(lo, hi);
  else
    return (uint32_t)f32_to_f16_bits(lo) | ((uint32_t)f32_to_f16_bits(hi) << 16);
}

// The bits of a 16-bit dtype (CIN_DT_F16 or CIN_DT_BF16) widened to fp32 (exact).
__device__ inline float half_bits_to_f32(int dt, uint16_t bits) {
  if (dt == CIN_DT_BF16) return __uint_as_float((uint32_t)bits << 16);
  _Float16 h;
  __builtin_memcpy(&h, &bits, 2);
  return (float)h;
}

// Load one element of dtype `dt` at element index i and widen to fp32 (exact).
__device__ inline float load_elem(const void* p, int dt, int64_t i) {
  if (dt == CIN_DT_BF16) return __uint_as_float(((uint32_t)((const uint16_t*)p)[i]) << 16);
  if (dt == CIN_DT_F16) return (float)((const _Float16*)p)[i];
  return ((const float*)p)[i];
}

// Max over the 16 lanes of a DPP row for values that are >= 0 and not NaN (maxima of
// |x| started from 0 under maxnum): their bit patterns order as unsigned integers, so each
// step is one v_max_u32 with a DPP operand and needs no NaN quieting.
__device__ inline float row16_max_pos(float a) {
  uint32_t u = __float_as_uint(a);
  u = max(u, (uint32_t)__builtin_amdgcn_mov_dpp((int)u, 0xB1, 0xF, 0xF, true));   // quad [1,0,3,2]
  u = max(u, (uint32_t)__builtin_amdgcn_mov_dpp((int)u, 0x4E, 0xF, 0xF, true));   // quad [2,3,0,1]
  u = max(u, (uint32_t)__builtin_amdgcn_mov_dpp((int)u, 0x141, 0xF, 0xF, true));  // row_half_mirror
  u = max(u, (uint32_t)__builtin_amdgcn_mov_dpp((int)u, 0x140, 0xF, 0xF, true));  // row_mirror
  return __uint_as_float(u);
}

// The same over the 8 lanes of a DPP half-row.
__device__ inline float row8_max_pos(float a) {
  uint32_t u = __float_as_uint(a);
  u = max(u, (uint32_t)__builtin_amdgcn_mov_dpp((int)u, 0xB1, 0xF, 0xF, true));   // quad [1,0,3,2]
  u = max(u, (uint32_t)__builtin_amdgcn_mov_dpp((int)u, 0x4E, 0xF, 0xF, true));   // quad [2,3,0,1]
  u = max(u, (uint32_t)__builtin_amdgcn_mov_dpp((int)u, 0x141, 0xF, 0xF, true));  // row_half_mirror
  return __uint_as_float(u);
}

// The same over a whole wave64.
__device__ inline float wave_max_pos(float a) {
  uint32_t u = __float_as_uint(row16_max_pos(a));
  u = max(u, (uint32_t)__shfl_xor((int)u, 16));
  u = max(u, (uint32_t)__shfl_xor((int)u, 32));
  return __uint_as_float(u);
}

// Max over the 16 lanes of a DPP row (lanes 16r..16r+15), maxnum semantics.
__device__ inline float row16_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));  // quad [1,0,3,2]
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));  // quad [2,3,0,1]
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false))); // row_half_mirror
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false))); // row_mirror
  return v;
}

// Max over a whole wave64.
__device__ inline float wave_max(float v) {
  v = row16_max(v);
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

// Raw buffer resource over [p, p + bytes): accesses are an SGPR base plus a 32-bit lane
// offset, and anything past `bytes` reads as zero and is not written.
// The operands are wave-uniform by construction; readfirstlane says so to the compiler,
// so the descriptor lives in SGPRs even when it was computed from loaded values.
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* p, int64_t bytes) {
  const int64_t cap = 0xffffffffLL;
  // (readfirstlane returns int: go through uint32_t, or a low word with bit 31 set
  // would sign-extend into the high word of the address)
  const uint32_t n = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(bytes < cap ? bytes : cap));
  const uint64_t a = (uint64_t)(uintptr_t)p;
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
  void* pu = (void*)(uintptr_t)((hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(pu, (short)0, (int)n, 0x00020000);
}

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace cin
