/*
 * cinnamon_fp8.h — C ABI of the MI355X (gfx950) FP8 hot path.
 *
 * Every entry point below replaces one operator of the reference's FP8 path
 * (shyampathak22/cinnamon, src/kernels.py) and is cited at its declaration.
 * The reference binds its kernels from Python; the binding a maintainer adds
 * is a ctypes stub (see cinnamon_amd/_lib.py), so these signatures use only
 * plain pointers, 64-bit sizes/strides and small integer enums.
 *
 * Conventions shared by all entry points:
 *   - Pointers are device pointers on the caller's current HIP device.
 *   - Strides are in ELEMENTS, row-major unless a stride argument says
 *     otherwise.  FP8 codes are OCP e4m3fn bytes (torch.float8_e4m3fn).
 *   - Outputs are caller-allocated; the library allocates nothing.
 *   - `stream` is a hipStream_t passed as void* (NULL = default stream).
 *     Calls are asynchronous and never synchronize the device.
 *   - Return value: CIN_OK (0) or a negative error code; cin_last_error()
 *     returns a message for the calling thread's last failure.
 */
#ifndef CINNAMON_FP8_H
#define CINNAMON_FP8_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type of a floating-point tensor argument. */
enum cin_dtype { CIN_DT_BF16 = 0, CIN_DT_F32 = 1, CIN_DT_F16 = 2 };

/* Return codes. */
enum cin_status {
  CIN_OK = 0,
  CIN_ERR_ARG = -1,          /* invalid shape/stride/pointer/enum argument   */
  CIN_ERR_UNSUPPORTED = -2,  /* valid but unsupported combination            */
  CIN_ERR_HIP = -3           /* the HIP runtime reported an error            */
};

/* Library ABI version (bumped on any signature change). */
int cin_abi_version(void);

/*
 * Scale matrices.  Every matrix of per-row (1 x 128) scales below is addressed with two
 * strides, scale[r, c] = base[r * row stride + c * column stride], and may be row-major
 * (column stride 1, row stride >= its columns: the reference's layout) or column-major
 * (row stride 1, column stride >= its rows).  Column-major puts the scales of one
 * 128-column block of consecutive rows next to each other: the GEMMs read the A scales of
 * a K block as one contiguous run, and the 128 x 128 tile quantizers write and read a
 * tile's 128 row scales as one run.  The reference's Python API keeps row-major; the FP8
 * linear and the experts layer use column-major internally.
 */

/* Message for the last failing call on this thread ("" if none). */
const char* cin_last_error(void);

/*
 * Row-wise (1 x block) quantization.
 * Replaces quantize_fp8_rowwise / quantize_fp8_rowwise_kernel
 * (reference src/kernels.py:178-216 and :19-71).
 *   x      [M, N] of dtype x_dtype, strides (sxm, sxn)
 *   q      [M, N] e4m3 codes, row stride sqm, column stride 1
 *   scales [M, ceil(N/block)] fp32, strides (ssm, ssk)
 * block in [1, 1024]; round_scale != 0 selects power-of-two scales.
 */
int cin_quant_rowwise(const void* x, int x_dtype, int64_t M, int64_t N, int64_t sxm, int64_t sxn,
                      int64_t block, int round_scale, uint8_t* q, int64_t sqm, float* scales,
                      int64_t ssm, int64_t ssk, void* stream);

/*
 * Block-wise (bm x bn) quantization.
 * Replaces quantize_fp8_blockwise / quantize_fp8_blockwise_kernel
 * (reference src/kernels.py:219-259 and :74-132).
 *   x      [M, N] of dtype x_dtype, strides (sxm, sxn)
 *   q      [M, N] codes, row stride sqm (may be NULL if qt is given)
 *   qt     optional [N, M] codes of the transpose (row stride sqtm), or NULL;
 *          the same codes as q, laid out K-contiguous for the dgrad GEMM
 *   scales [ceil(M/bm), ceil(N/bn)] fp32, row stride ssm
 * bm, bn in [1, 1024] with bm * bn <= 65536.
 */
int cin_quant_blockwise(const void* x, int x_dtype, int64_t M, int64_t N, int64_t sxm, int64_t sxn,
                        int64_t bm, int64_t bn, int round_scale, uint8_t* q, int64_t sqm,
                        uint8_t* qt, int64_t sqtm, float* scales, int64_t ssm, void* stream);

/*
 * The two quantizations of the FP8 linear forward in one call: X [M, K] in 1 x 128 row
 * tiles (as cin_quant_rowwise, block 128) and the weight W [N, K] in 128 x 128 blocks
 * with round_scale off (as cin_quant_blockwise, 128 x 128).
 * Replaces the pair quantize_fp8_rowwise(x_flat, 128, round_scale) and
 * quantize_fp8_blockwise(weight.float(), 128, 128) in FP8MatmulFunction.forward
 * (reference src/kernels.py:746-747).  Codes and scales are bit-identical to those two
 * calls; with K % 128 == 0, a 16-bit W and 16-byte aligned rows both run in one launch.
 *   x  [M, K] of dtype x_dtype, row stride sxm (unit column stride)
 *   xq [M, K] codes (row stride sxqm) and xs [M, ceil(K/128)] (strides (sxsm, sxsk))
 *   w  [N, K] of dtype w_dtype, row stride swm (unit column stride)
 *   wq [N, K] codes (row stride swqm), or NULL; wqt [K, N] transposed codes (row stride
 *   swqtm), or NULL; at least one of the two.  ws [ceil(N/128), ceil(K/128)] (row stride swsm)
 */
int cin_quant_fwd(const void* x, int x_dtype, int64_t M, int64_t K, int64_t sxm, int round_scale,
                  uint8_t* xq, int64_t sxqm, float* xs, int64_t sxsm, int64_t sxsk, const void* w,
                  int w_dtype, int64_t N, int64_t swm, uint8_t* wq, int64_t swqm, uint8_t* wqt,
                  int64_t swqtm, float* ws, int64_t swsm, void* stream);

/*
 * Dequantization with (bm x bn) block scales; bm = 1 gives row-wise scales.
 * Replaces dequantize_fp8 / dequantize_fp8_kernel (reference src/kernels.py:284-314,
 * :135-173; bf16 output) and dequantize_fp8_rowwise (:262-281; fp32 output).
 *   q      [M, N] codes, strides (sqm, sqn)
 *   scales indexed [m / bm, n / bn] with strides (ssm, ssn)
 *   out    [M, N] of dtype out_dtype (CIN_DT_BF16 or CIN_DT_F32), row stride som
 */
int cin_dequant(const uint8_t* q, int64_t M, int64_t N, int64_t sqm, int64_t sqn,
                const float* scales, int64_t ssm, int64_t ssn, int64_t bm, int64_t bn,
                void* out, int out_dtype, int64_t som, void* stream);

/*
 * Dual 1x128 quantization of a gradient in one read: row tiles of dy and row
 * tiles of dy^T (= 128 x 1 column tiles of dy).
 * Replaces the pair quantize_fp8_rowwise(grad_flat) and
 * quantize_fp8_rowwise(grad_flat.t().contiguous()) in FP8MatmulFunction.backward
 * (reference src/kernels.py:771 and :781-783).
 *   dy [M, N] of dtype dy_dtype, strides (sdm, sdn)
 *   q  [M, N] codes (row stride sqm) and s  [M, ceil(N/128)] (strides (ssm, ssk))
 *   qt [N, M] codes (row stride sqtm) and st [N, ceil(M/128)] (strides (sstm, sstk))
 */
int cin_quant_dual(const void* dy, int dy_dtype, int64_t M, int64_t N, int64_t sdm, int64_t sdn,
                   int round_scale, uint8_t* q, int64_t sqm, float* s, int64_t ssm, int64_t ssk,
                   uint8_t* qt, int64_t sqtm, float* st, int64_t sstm, int64_t sstk, void* stream);

/*
 * Re-quantize 1x128 row-quantized codes into 128x128 blocks, bit-identical to
 * quantize_fp8_blockwise(dequantize_fp8_rowwise(q, s), round_scale=False)
 * (reference src/kernels.py:784-787), without the fp32 temporary.
 *   q    [M, K] codes (row stride sqm), srow [M, ceil(K/128)] (strides (ssm, ssk))
 *   qb   optional [M, K] block codes (row stride sqbm) or NULL
 *   qbt  optional [K, M] block codes of the transpose (row stride sqbtm) or NULL
 *   sblk [ceil(M/128), ceil(K/128)] block scales (row stride ssbm)
 */
int cin_requant_row_to_block(const uint8_t* q, int64_t M, int64_t K, int64_t sqm,
                             const float* srow, int64_t ssm, int64_t ssk, uint8_t* qb, int64_t sqbm,
                             uint8_t* qbt, int64_t sqbtm, float* sblk, int64_t ssbm, void* stream);

/*
 * The backward's three quantizations in one launch: cin_quant_dual of dy [M, N] (unit
 * column stride) and cin_requant_row_to_block of the saved X codes [M, K] into transposed
 * block codes only (qb = NULL), with the same outputs, bit for bit, as those two calls.
 * Replaces, in FP8MatmulFunction.backward, quantize_fp8_rowwise(grad_flat) (reference
 * src/kernels.py:771), quantize_fp8_rowwise(grad_flat.t().contiguous()) (:781-783) and
 * quantize_fp8_blockwise(dequantize_fp8_rowwise(x_fp8, x_scale)) (:784-787).
 *   dy, q, s, qt, st           as cin_quant_dual (sdn = 1)
 *   xq [M, K], xs [M, ceil(K/128)]   the forward's row-wise X codes and scales (xs strides
 *                                    (sxsm, sxsk))
 *   xbt [K, M] block codes of X^T (row stride sxbtm), sblk [ceil(M/128), ceil(K/128)]
 * One launch for 16-bit dy with N and K multiples of 128; otherwise the two calls in turn.
 */
int cin_quant_backward(const void* dy, int dy_dtype, int64_t M, int64_t N, int64_t sdm,
                       int round_scale, uint8_t* q, int64_t sqm, float* s, int64_t ssm, int64_t ssk,
                       uint8_t* qt, int64_t sqtm, float* st, int64_t sstm, int64_t sstk,
                       const uint8_t* xq, int64_t K, int64_t sxqm, const float* xs, int64_t sxsm,
                       int64_t sxsk, uint8_t* xbt, int64_t sxbtm, float* sblk, int64_t ssbm,
                       void* stream);

/*
 * Byte transpose: dst[c, r] = src[r, c] for an [R, C] matrix of codes.
 * Replaces the code-layout copies w_fp8.t().contiguous() (reference src/kernels.py:748).
 */
int cin_transpose_u8(const uint8_t* src, int64_t R, int64_t C, int64_t lds, uint8_t* dst,
                     int64_t ldd, void* stream);

/*
 * Block-scaled FP8 GEMM, both operands K-contiguous:
 *   C[m, n] = sum_kb  sa[m, kb] * sb[n / 128, kb] * sum_{k in kb} A[m, k] * B[n, k]
 * which is fp8_gemm_kernel / fp8_matmul_dsv3 (reference src/kernels.py:588-702)
 * with its B operand given as B^T.  fp32 accumulation, fp32 epilogue.
 *   A  [M, K] codes, row stride lda;  sa indexed [m, kb] with strides (ssam, ssak)
 *   B  [N, K] codes, row stride ldb;  sb indexed [nb, kb] with strides (ssbn, ssbk)
 *   C  [M, N] of c_dtype (CIN_DT_BF16 or CIN_DT_F16: round-to-nearest-even of the fp32 value;
 *      CIN_DT_F32: the fp32 value), row stride ldc
 * Requires K % 16 == 0, lda % 16 == 0, ldb % 16 == 0 and 16-byte aligned A, B.
 */
int cin_gemm_fp8_bs(const uint8_t* A, int64_t lda, const float* sa, int64_t ssam, int64_t ssak,
                    const uint8_t* B, int64_t ldb, const float* sb, int64_t ssbn, int64_t ssbk,
                    int64_t M, int64_t N, int64_t K, void* C, int c_dtype, int64_t ldc,
                    void* stream);

/*
 * Grouped (MoE) block-scaled FP8 GEMM over routed experts in ONE launch with a
 * device-side expert tile table (no host sync, no host loop):
 *   for each expert e with rows [starts[e], ends[e]):
 *     C[r, n] = sum_kb sa[r, kb] * sb_e[n / 128, kb] * sum_k A[r, k] * B_e[n, k]
 * FP8 counterpart of moe_grouped_gemm / grouped_gemm_kernel (reference
 * src/kernels.py:526-581, :440-523), with the reference's per-expert loop
 * semantics of GroupedExperts (src/layers.py:79-86).
 *   A  [T, K] codes (row stride lda), sa [T, ceil(K/128)] (strides ssam, ssak)
 *   B  expert e at B + e * sbe: [N, K] codes, row stride ldb
 *   sb expert e at sb + e * ssbe, indexed [nb, kb] with strides (ssbn, ssbk)
 *   starts, ends  int64 device arrays of length E (rows outside every
 *                 [starts[e], ends[e]) are not written)
 *   C  [T, N] of c_dtype, row stride ldc
 */
int cin_grouped_gemm_fp8(const uint8_t* A, int64_t lda, const float* sa, int64_t ssam,
                         int64_t ssak, const uint8_t* B, int64_t sbe, int64_t ldb, const float* sb,
                         int64_t ssbe, int64_t ssbn, int64_t ssbk, const int64_t* starts,
                         const int64_t* ends, int64_t E, int64_t T, int64_t N, int64_t K, void* C,
                         int c_dtype, int64_t ldc, void* stream);

/*
 * MoE backward (grouped dgrad / wgrad).  The reference's grouped GEMM has no backward
 * (src/kernels.py:440-581, src/layers.py:69-75 run it without autograd); these entry
 * points apply the FP8MatmulFunction.backward recipe (src/kernels.py:763-794) to each
 * expert's row slice [starts[e], ends[e]).
 *
 * Padded token axis: expert e's tokens are split into 128-token chunks aligned at its
 * first row; chunk c sits at columns [p_e + 128 c, p_e + 128 c + 128) of the transposed
 * outputs, p_e = sum_{e' < e} 128 * ceil(m_e' / 128), and the columns past the expert's
 * last token hold code 0.  The padded length never exceeds 128 * (ceil(T / 128) + E);
 * outputs sized with that many columns always suffice.
 */

/*
 * Grouped dual quantization of the output gradient dC [T, N] (contiguous rows):
 *   q  [T, N] 1x128 row tiles (row stride sqm), s [T, ceil(N/128)] (strides (ssm, ssk))
 *      -- the dgrad operand, as quantize_fp8_rowwise(dC) for every row inside a range;
 *   qt [N, Tpad] per-expert 128x1 column tiles on the padded axis (row stride sqtm =
 *      the padded capacity), st [N, sqtm / 128] (strides (sstm, sstk))
 *      -- the wgrad operand, as quantize_fp8_rowwise(dC[s_e:e_e].t()) for each expert.
 */
int cin_quant_dual_grouped(const void* dy, int dy_dtype, int64_t T, int64_t N, int64_t sdm,
                           const int64_t* starts, const int64_t* ends, int64_t E, int round_scale,
                           uint8_t* q, int64_t sqm, float* s, int64_t ssm, int64_t ssk, uint8_t* qt,
                           int64_t sqtm, float* st, int64_t sstm, int64_t sstk, void* stream);

/*
 * Grouped re-quantization of the expert inputs for wgrad: for each expert, 128x128 blocks
 * of quantize_fp8_blockwise(dequantize_fp8_rowwise(q, srow)[s_e:e_e]) (reference
 * src/kernels.py:784-787 per slice), written transposed on the padded axis:
 *   q    [T, K] row-wise codes (row stride sqm), srow [T, ceil(K/128)] (strides (ssm, ssk))
 *   qbt  [K, Tpad] block codes (row stride sqbtm = padded capacity)
 *   sblk [sqbtm / 128, ceil(K/128)] block scales, row = padded chunk (row stride ssbm)
 */
int cin_requant_row_to_block_grouped(const uint8_t* q, int64_t T, int64_t K, int64_t sqm,
                                     const float* srow, int64_t ssm, int64_t ssk,
                                     const int64_t* starts, const int64_t* ends, int64_t E,
                                     uint8_t* qbt, int64_t sqbtm, float* sblk, int64_t ssbm,
                                     void* stream);

/*
 * Grouped weight gradient, one launch over all experts:
 *   C_e[n, k] = sum over expert e's padded chunks j of
 *               sa[n, j] * sb[j, k / 128] * sum_{t in chunk j} A[n, t] * B[k, t]
 * i.e. dW_e = dC_e^T X_e with A = qt/st of cin_quant_dual_grouped (A[N, Tpad], lda; st
 * strides (ssam, ssak), row- or column-major) and
 * B = qbt/sblk of cin_requant_row_to_block_grouped (B[K, Tpad], ldb; sb row stride ssbm).
 * T is the token count the ranges refer to; tcap the padded columns A and B hold (an
 * expert whose padded range would pass tcap gets zeros).  C is [E, N, K] (row stride
 * ldc, expert stride sce); experts without tokens get zeros.
 * Needs N >= 256, K >= 256, K % 128 == 0.
 */
int cin_grouped_gemm_fp8_wgrad(const uint8_t* A, int64_t lda, const float* sa, int64_t ssam,
                               int64_t ssak, const uint8_t* B, int64_t ldb, const float* sb, int64_t ssbm,
                               const int64_t* starts, const int64_t* ends, int64_t E, int64_t T,
                               int64_t tcap, int64_t N, int64_t K, void* C, int c_dtype,
                               int64_t ldc, int64_t sce, void* stream);

/*
 * Unquantized grouped GEMM, replacing the reference's moe_grouped_gemm /
 * grouped_gemm_kernel (src/kernels.py:526-581, :440-523) as GroupedExperts calls it
 * (src/layers.py:71, :74): for each expert e with rows [starts[e], ends[e]),
 *   C[r, n] = fp16( sum_k fp16(A[r, k]) * fp16(B_e[n, k]) )   (fp32 sums)
 *   A [T, K] of a_dtype (row stride lda, K contiguous)
 *   B expert e at B + e * sbe: [N, K] of b_dtype (row stride ldb, K contiguous)
 *   C [T, N] fp16 (row stride ldc); rows outside every range are not written.
 * One launch, device-side ranges (no max_expert_tokens host value needed).
 */
int cin_grouped_gemm_f16(const void* A, int a_dtype, int64_t lda, const void* B, int b_dtype,
                         int64_t sbe, int64_t ldb, const int64_t* starts, const int64_t* ends,
                         int64_t E, int64_t T, int64_t N, int64_t K, void* C, int64_t ldc,
                         void* stream);

/*
 * SwiGLU activation fused into the row-wise quantizer.  Replaces, in the experts' forward
 * (reference GroupedExperts.forward, src/layers.py:72-74), the chain
 *   h1, h2 = h12.float().chunk(2, -1);  h = (silu(h1) * h2).to(dtype)
 * followed by quantize_fp8_rowwise(h) (src/kernels.py:178-216) before the down GEMM:
 *   h12    [M, 2H] of in_dtype (row stride s12; both halves 16-byte aligned)
 *   q      [M, H] codes (row stride sqm), scales [M, ceil(H/128)] (strides (ssm, ssk))
 *   out_dtype is the dtype h is rounded to before quantization (the activation dtype).
 * silu(a) = a / (1 + exp(-a)) with an IEEE division, torch's GPU formula.
 */
int cin_silu_mul_quant_rowwise(const void* h12, int in_dtype, int64_t M, int64_t H, int64_t s12,
                               int out_dtype, int round_scale, uint8_t* q, int64_t sqm,
                               float* scales, int64_t ssm, int64_t ssk, void* stream);

/*
 * SwiGLU backward in one pass, replacing the elementwise chain of the experts' backward
 * (the derivative of src/layers.py:72-73, h = silu(h1) * h2 with [h1 h2] = h12):
 *   dh12[:, :H] = dh * h2 * (sig * (1 + h1 * (1 - sig))),  dh12[:, H:] = dh * (h1 * sig)
 * with sig = 1 / (1 + exp(-h1)), in fp32 with one rounding per operation in that order.
 *   dh   [M, H] fp32 (row stride sdm), h12 [M, 2H] of h12_dtype (row stride s12)
 *   dh12 [M, 2H] fp32 (row stride som).  H % 4 == 0; fp32 rows 16-byte aligned.
 * No counterpart in the reference (its grouped GEMM has no backward); the FP8 experts'
 * backward (layers.FP8GroupedExpertsFunction) calls it.
 */
int cin_swiglu_backward(const float* dh, int64_t sdm, const void* h12, int h12_dtype, int64_t s12,
                        int64_t M, int64_t H, float* dh12, int64_t som, void* stream);

/*
 * cin_swiglu_backward followed by cin_quant_dual_grouped of its output, in one pass: the
 * fp32 dh12 [T, 2H] is formed tile by tile in registers and never stored.  Arguments as the
 * two calls' (dh, h12 as cin_swiglu_backward's with M = T; the outputs and ranges as
 * cin_quant_dual_grouped's with N = 2H); the codes and scales are bit for bit those of the
 * two calls.  H % 128 == 0; dh and h12 rows 16-byte aligned.  No counterpart in the
 * reference (its grouped GEMM has no backward); the FP8 experts' backward calls it.
 */
int cin_swiglu_dual_grouped(const float* dh, int64_t sdm, const void* h12, int h12_dtype, int64_t s12,
                            int64_t T, int64_t H, const int64_t* starts, const int64_t* ends, int64_t E,
                            int round_scale, uint8_t* q, int64_t sqm, float* s, int64_t ssm, int64_t ssk,
                            uint8_t* qt, int64_t sqtm, float* st, int64_t sstm, int64_t sstk, void* stream);

/*
 * Zero the rows r of a [T, *] matrix (rows ldc_bytes apart, row_bytes written) with r outside
 * every range [starts[e], ends[e]).  The grouped GEMMs leave such rows untouched (as the
 * reference's moe_grouped_gemm leaves them unset, src/kernels.py:550); callers that need
 * them zero call this instead of zero-filling the whole output.  No counterpart in the
 * reference.
 */
int cin_zero_rows_outside_ranges(void* C, int64_t ldc_bytes, int64_t row_bytes, int64_t T,
                                 const int64_t* starts, const int64_t* ends, int64_t E,
                                 void* stream);

/*
 * DSA indexer scoring on FP8 codes, fused (no [B, L, H, S] logits):
 *   scores[b,t,s] = k_scale[b,s] * sum_h relu(sum_d q8[b,t,h,d] k8[b,s,d])
 *                                 * ((q_scale[b,t,h] * weights[b,t,h]) * softmax_scale)
 * Replaces the FP8 branch of DSAIndexer.forward (reference src/attention.py:288-300) after
 * its two row-wise quantizations: q_scale / k_scale are the first 1x128 scale of each row
 * (:296-297).  All arrays contiguous: q8 [B, L, H, d] and k8 [B, S, d] e4m3 codes (8-byte
 * aligned), q_scale and weights [B, L, H] fp32, k_scale [B, S] fp32, scores [B, L, S] fp32.
 * d a multiple of 32 in [32, 256].
 */
/*
 * The two row-wise quantizations of DSAIndexer.forward's FP8 branch (reference
 * src/attention.py:292-297) in one call: q [B*L*H, d] and k [B*S, d] (contiguous, 16-byte
 * aligned, bf16/fp16/fp32) -> e4m3 codes (same layout, 8-byte aligned) and the FIRST 1x128
 * scale of each row only, q_scale [B*L*H] and k_scale [B*S] fp32, the `[..., 0]` the
 * reference keeps.  Codes and scales are bit-identical to cin_quant_rowwise(block 128).
 */
int cin_indexer_quantize(const void* q, int q_dtype, const void* k, int k_dtype, int64_t B,
                         int64_t L, int64_t S, int64_t H, int64_t d, uint8_t* q8, float* q_scale,
                         uint8_t* k8, float* k_scale, void* stream);

int cin_indexer_scores_fp8(const uint8_t* q8, const float* q_scale, const uint8_t* k8,
                           const float* k_scale, const float* weights, int64_t B, int64_t L,
                           int64_t S, int64_t H, int64_t d, float softmax_scale, float* scores,
                           void* stream);

/*
 * cin_indexer_quantize's q side and cin_indexer_scores_fp8 in one launch (no counterpart in
 * the reference, whose FP8 branch quantizes q as a separate step, src/attention.py:292-297):
 * q [B, L, H, d] arrives unquantized (bf16, fp16 or fp32, contiguous, 16-byte aligned) and
 * each workgroup quantizes its own tokens' rows with cin_indexer_quantize's arithmetic, so
 * the scores are bit-identical to the two calls.  k8 / k_scale as for cin_indexer_scores_fp8
 * (cin_indexer_quantize with L = 0 makes them).  When q8 and q_scale are not null the codes
 * [B, L, H, d] and first scales [B, L, H] are written as well (what
 * cin_indexer_weights_grad takes); both null skips them.  H <= 4 for d <= 128 and H <= 2
 * above; more heads are rejected (use the two calls).
 */
int cin_indexer_scores_fp8_q(const void* q, int q_dtype, const uint8_t* k8, const float* k_scale,
                             const float* weights, int64_t B, int64_t L, int64_t S, int64_t H, int64_t d,
                             float softmax_scale, float* scores, uint8_t* q8, float* q_scale,
                             void* stream);

/*
 * Gradient of cin_indexer_scores_fp8's scores with respect to `weights`, the reference's
 * autograd through its FP8 branch (src/attention.py:298-300; the codes come from the
 * quantizer and carry no gradient, so q and k get none):
 *   grad_weights[b,t,h] = ((sum_s relu(logit[b,t,h,s]) * (grad_scores[b,t,s] * k_scale[b,s]))
 *                          * softmax_scale) * q_scale[b,t,h]
 * with logit as in cin_indexer_scores_fp8.  grad_scores [B, L, S] and grad_weights [B, L, H]
 * fp32, contiguous.  workspace: fp32, at least cin_indexer_weights_grad_workspace(B, L, S, H)
 * elements (one partial sum per 512-key range, added in increasing range order, so the
 * result is deterministic).  Same layouts and limits as cin_indexer_scores_fp8.
 */
int cin_indexer_weights_grad(const uint8_t* q8, const float* q_scale, const uint8_t* k8,
                             const float* k_scale, const float* grad_scores, int64_t B, int64_t L,
                             int64_t S, int64_t H, int64_t d, float softmax_scale, float* workspace,
                             int64_t workspace_len, float* grad_weights, void* stream);
int64_t cin_indexer_weights_grad_workspace(int64_t B, int64_t L, int64_t S, int64_t H);

/* ---------------------------- MoE dispatch / combine ---------------------------- */

/*
 * Device-side routing: a stable counting sort of the flattened top-k expert ids.
 * Replaces the sort / bincount / cumsum / .item() of MoE.forward (reference
 * src/layers.py:133-148).
 *   idx       [T, k] int64 expert ids (contiguous); ids outside [0, E) are dropped
 *   perm      [T*k] int64: perm[r] = t*k + j of the assignment at sorted position r
 *             (the reference's sort_order, in stable order); -1 past the last kept one
 *   inv       [T*k] int32: sorted position of assignment t*k + j, -1 if dropped
 *   counts, starts, ends  [E] int64 expert row ranges (bincount, cumsum)
 *   workspace int32, at least cin_moe_route_workspace(T, k, E) elements
 * E <= 4096, T*k < 2^31.
 */
int cin_moe_route(const int64_t* idx, int64_t T, int64_t k, int64_t E, int64_t* perm, int32_t* inv,
                  int64_t* counts, int64_t* starts, int64_t* ends, int32_t* workspace,
                  int64_t workspace_elems, void* stream);
int cin_moe_route_workspace(int64_t T, int64_t k, int64_t E);

/*
 * cin_moe_route without a workspace argument: it allocates nothing (no hipMalloc, no
 * allocating library call) and keeps its [nblocks, E] counts and bases in a scratch array
 * the library holds on each GPU: 1,048,576 int32 (4 MiB), so it needs
 * 2 * ceil(T*k / 1024) * E <= 1,048,576 (= cin_moe_route_workspace(T, k, E)), and rejects
 * larger routes with CIN_ERR_ARG.  Same outputs as cin_moe_route.  Calls that overlap on
 * one GPU (two streams or two host threads) share the array and race; the array needs no
 * clearing between calls.  The first call on each device looks up the array's device
 * address (hipGetSymbolAddress, no stream work): a caller that captures the route in a HIP
 * graph makes one call outside the capture first (tests/test_zz_no_alloc.py replays such a
 * graph).
 * No counterpart in the reference: it is for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 */
int cin_moe_route_noalloc(const int64_t* idx, int64_t T, int64_t k, int64_t E, int64_t* perm,
                          int32_t* inv, int64_t* counts, int64_t* starts, int64_t* ends,
                          void* stream);

/*
 * Dispatch gather fused into the 1x128 row-wise quantizer: row r of q / scales is
 * quantize_fp8_rowwise(x[rowmap[r] / rowdiv]) bit for bit; a negative or out-of-range map
 * entry gives a zero row.  Replaces sorted_x = flat_x[token_indices] (reference
 * src/layers.py:139-141) followed by the activation quantization of the grouped GEMM
 * (src/kernels.py:178-216): the gathered bf16 rows are never written.
 *   x [src_rows, N], rows 16-byte aligned (sxm elements apart); rowmap [rows] int64
 *   (perm from cin_moe_route, rowdiv = k); q [rows, N] (8-byte aligned rows),
 *   scales [rows, ceil(N/128)] fp32 (strides (ssm, ssk)).
 */
int cin_moe_gather_quant_rowwise(const void* x, int x_dtype, int64_t src_rows, int64_t N,
                                 int64_t sxm, const int64_t* rowmap, int64_t rows, int64_t rowdiv,
                                 int round_scale, uint8_t* q, int64_t sqm, float* scales,
                                 int64_t ssm, int64_t ssk, void* stream);

/*
 * The same codes and scales as cin_moe_gather_quant_rowwise(x, perm, k), computed from the
 * token side: token row t is quantized once and written to its sorted rows inv[t*k + j]
 * (one read of x instead of k); rows r with perm[r] < 0 get the zero-row quantization.
 *   x [T, N] (16-byte aligned rows), inv [T*k] int32 and perm [rows] int64 from
 *   cin_moe_route, q [rows, N] (8-byte aligned rows), scales [rows, ceil(N/128)] (strides
 *   (ssm, ssk)).
 */
int cin_moe_scatter_quant_rowwise(const void* x, int x_dtype, int64_t T, int64_t N, int64_t sxm,
                                  const int32_t* inv, int64_t k, const int64_t* perm, int64_t rows,
                                  int round_scale, uint8_t* q, int64_t sqm, float* scales,
                                  int64_t ssm, int64_t ssk, void* stream);

/*
 * cin_moe_scatter_quant_rowwise with a workspace ws [T, ceil(N/128)] fp32 (T * ceil(N/128)
 * floats, 16-byte aligned, contents on entry ignored): each token's scales are written once into ws, and a
 * second pass over the sorted rows copies them into scales (threads of consecutive rows store
 * consecutive addresses), instead of k scattered 4-byte stores per token scale.  Same codes
 * and scales.  No counterpart in the reference; the MoE dispatch (moe.py) calls it.
 */
int cin_moe_scatter_quant_rowwise_ws(const void* x, int x_dtype, int64_t T, int64_t N, int64_t sxm,
                                     const int32_t* inv, int64_t k, const int64_t* perm, int64_t rows,
                                     int round_scale, uint8_t* q, int64_t sqm, float* scales,
                                     int64_t ssm, int64_t ssk, float* ws, void* stream);

/*
 * Backward of the dispatch gather: out[t] = sum over token t's sorted positions r
 * (increasing r, fp32 sums) of g[r]; the gradient of flat_x[token_indices] (reference
 * src/layers.py:140).  g [A, N] (g_dtype, row stride sgm), inv [T*k] from cin_moe_route,
 * out [T, N] (out_dtype, row stride som).  k <= 16.
 */
int cin_moe_gather_sum(const void* g, int g_dtype, int64_t sgm, const int32_t* inv, int64_t T,
                       int64_t k, int64_t A, int64_t N, void* out, int out_dtype, int64_t som,
                       void* stream);

/*
 * Weighted combine: out[t] = sum over token t's sorted positions r, in increasing r, of
 * y[r] * score[t, slot(r)], fp32 (product and sum each rounded), i.e. the reference's
 * weighted_out = sorted_out * sorted_scores[:, None] followed by a sequential
 * routed_out.scatter_add_ (src/layers.py:151-154).  y [A, N] of y_dtype (fp32, or fp16 as
 * the reference's expert outputs, src/layers.py:69-75, widened exactly), scores [T, k]
 * (s_dtype, row stride ssm), out [T, N] fp32.  k <= 16.
 */
int cin_moe_combine(const void* y, int y_dtype, int64_t sym, const void* scores, int s_dtype,
                    int64_t ssm, const int32_t* inv, int64_t T, int64_t k, int64_t A, int64_t N,
                    float* out, int64_t som, void* stream);

/*
 * Backward of cin_moe_combine: dy[r] = dout[t] * score[t, j] for the assignment t*k + j at
 * sorted position r (zero rows where perm is -1), and dscores[t, j] = sum_c dout[t, c] *
 * y[inv[t*k + j], c] (fp32, 0 for dropped assignments); the autograd of reference
 * src/layers.py:151-154.  dout [T, N] fp32, y [A, N] of y_dtype, dy [A, N] of dy_dtype (the
 * fp32 product rounded to it, RNE; bf16 keeps fp32's range for small gradients where fp16
 * would flush them), k <= 16, dscores [T, k] fp32 contiguous.
 */
int cin_moe_combine_backward(const float* dout, int64_t sdm, const void* y, int y_dtype, int64_t sym,
                             const void* scores, int s_dtype, int64_t ssm, const int64_t* perm,
                             const int32_t* inv, int64_t T, int64_t k, int64_t A, int64_t N,
                             void* dy, int dy_dtype, int64_t sdym, float* dscores, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CINNAMON_FP8_H */
