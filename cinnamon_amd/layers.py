"""FP8 routed-expert layer for MI355X: grouped GEMM over experts in one launch.

Counterpart of the reference's moe_grouped_gemm (src/kernels.py:526-581) and
GroupedExperts (src/layers.py:34-87).  The reference grouped GEMM computes in fp16;
this module runs it in FP8 with the reference's quantization recipe (1x128
activation tiles, 128x128 weight blocks per expert) and the reference's per-expert
loop semantics (src/layers.py:79-86).
"""
from __future__ import annotations

import torch

from ._lib import call, dtype_code, ptr, stream_of
from .kernels import (WeightCache, _cdiv, _codes_u8, _rows8, _kcontig, _require, _scale_buf, _scales_2d,
                      _weight_cache_active, custom_op, quantize_fp8_blockwise_t,
                      quantize_fp8_rowwise)


def fp8_grouped_gemm(a_codes: torch.Tensor, a_scales: torch.Tensor, w_codes: torch.Tensor,
                     w_scales: torch.Tensor, expert_starts: torch.Tensor,
                     expert_ends: torch.Tensor, out_dtype: torch.dtype = torch.bfloat16,
                     out: torch.Tensor | None = None,
                     zero_uncovered: bool = False) -> torch.Tensor:
    """out[r] = A[r] x W_e^T for every row r in [starts[e], ends[e]), all experts in one launch.

    a_codes [T, K] e4m3 (1x128 scales a_scales [T, ceil(K/128)]), w_codes [E, N, K] e4m3
    (per-expert 128x128 block scales w_scales [E, ceil(N/128), ceil(K/128)]), expert
    ranges as int64 device tensors (no host sync).  Rows outside every range are left
    untouched (as in the reference, whose output is torch.empty), or zeroed with
    ``zero_uncovered`` when the output is allocated here.
    """
    _require(a_codes.is_cuda and w_codes.is_cuda, "Input must be on CUDA")
    T, K = a_codes.shape
    E, N, K2 = w_codes.shape
    _require(K == K2, f"Dimension mismatch: {K} vs {K2}")
    _require(K % 16 == 0, "grouped GEMM needs K % 16 == 0")
    _require(w_scales.shape[0] == E and w_scales.shape[1] >= _cdiv(N, 128)
             and w_scales.shape[2] >= _cdiv(K, 128), "w_scales must be [E, ceil(N/128), ceil(K/128)]")
    starts = expert_starts.to(torch.int64)
    ends = expert_ends.to(torch.int64)
    _require(starts.numel() == E and ends.numel() == E, "expert ranges must have E entries")
    if out is None:
        return _grouped_gemm_op(a_codes, a_scales, w_codes, w_scales, starts, ends, out_dtype,
                                bool(zero_uncovered))
    _require(out.stride(1) == 1, "out must have unit column stride")
    return _grouped_gemm_into(a_codes, a_scales, w_codes, w_scales, starts, ends, out)


def _grouped_gemm_into(a_codes, a_scales, w_codes, w_scales, starts, ends, out):
    T, K = a_codes.shape
    E, N, _ = w_codes.shape
    aq, _ = _kcontig(a_codes, K)
    wq = w_codes.view(torch.uint8) if w_codes.dtype == torch.float8_e4m3fn else w_codes
    if wq.stride(2) != 1 or wq.stride(1) % 16 or wq.stride(0) % 16 or wq.data_ptr() % 16:
        wq = wq.contiguous()
    call("cin_grouped_gemm_fp8", ptr(aq), aq.stride(0), ptr(a_scales), a_scales.stride(0),
         a_scales.stride(1), ptr(wq), wq.stride(0), wq.stride(1), ptr(w_scales),
         w_scales.stride(0), w_scales.stride(1), w_scales.stride(2), ptr(starts), ptr(ends), E, T,
         N, K, ptr(out), dtype_code(out), out.stride(0), stream_of(aq))
    return out


@custom_op("grouped_gemm_fp8", "(Tensor a_codes, Tensor a_scales, Tensor w_codes, Tensor w_scales, "
           "Tensor starts, Tensor ends, ScalarType out_dtype, bool zero_uncovered) -> Tensor")
def _grouped_gemm_op(a_codes, a_scales, w_codes, w_scales, starts, ends, out_dtype, zero_uncovered):
    T = a_codes.shape[0]
    N = w_codes.shape[1]
    out = (_empty_rows_zeroed(T, N, out_dtype, a_codes.device, starts, ends) if zero_uncovered
           else torch.empty((T, N), dtype=out_dtype, device=a_codes.device))
    return _grouped_gemm_into(a_codes, a_scales, w_codes, w_scales, starts, ends, out)


@_grouped_gemm_op.register_fake
def _(a_codes, a_scales, w_codes, w_scales, starts, ends, out_dtype, zero_uncovered):
    return a_codes.new_empty((a_codes.shape[0], w_codes.shape[1]), dtype=out_dtype)


# ---------------------------------------------------------------------------
# MoE backward.  The reference grouped GEMM has no backward (src/layers.py:69-75 runs
# it without autograd); these apply the FP8MatmulFunction.backward recipe
# (src/kernels.py:763-794) to each expert's row slice [starts[e], ends[e]).
# ---------------------------------------------------------------------------
def padded_capacity(T: int, E: int) -> int:
    """Columns that always hold the padded token axis (cin_grouped.h): 128 (ceil(T/128) + E)."""
    return 128 * (_cdiv(T, 128) + E)


def _ranges(expert_starts: torch.Tensor, expert_ends: torch.Tensor):
    starts = expert_starts.to(torch.int64).contiguous()
    ends = expert_ends.to(torch.int64).contiguous()
    _require(starts.numel() == ends.numel(), "expert_starts and expert_ends differ in length")
    return starts, ends


def quantize_fp8_dual_grouped(grad: torch.Tensor, expert_starts: torch.Tensor,
                              expert_ends: torch.Tensor, round_scale: bool = False,
                              col_scales: bool = False):
    """Grouped dual quantization of an output gradient dC [T, N].

    Returns (q [T, N], s [T, ceil(N/128)], qt [N, Tcap], st [N, Tcap/128]):
      q, s   -- quantize_fp8_rowwise(dC) for every row inside an expert range (the
                dgrad operand);
      qt, st -- for each expert, quantize_fp8_rowwise(dC[s_e:e_e].t().contiguous())
                stored at the expert's padded columns (the wgrad operand).
    """
    _require(grad.is_cuda, "Input must be on CUDA")
    _require(grad.ndim == 2, "Input must be 2D")
    starts, ends = _ranges(expert_starts, expert_ends)
    return _dual_grouped_op(grad, starts, ends, bool(round_scale), bool(col_scales))


@custom_op("quant_dual_grouped",
           "(Tensor grad, Tensor starts, Tensor ends, bool round_scale, bool col_scales) -> "
           "(Tensor, Tensor, Tensor, Tensor)")
def _dual_grouped_op(grad, starts, ends, round_scale, col_scales):
    if grad.stride(1) != 1 or (grad.stride(0) * grad.element_size()) % 16 or grad.data_ptr() % 16:
        grad = grad.contiguous()
    T, N = grad.shape
    E = starts.numel()
    cap = padded_capacity(T, E)
    dev = grad.device
    q = torch.empty((T, N), dtype=torch.float8_e4m3fn, device=dev)
    s = _scale_buf(grad, T, _cdiv(N, 128), col_scales)
    qt = torch.empty((N, cap), dtype=torch.float8_e4m3fn, device=dev)
    st = _scale_buf(grad, N, cap // 128, col_scales)
    call("cin_quant_dual_grouped", ptr(grad), dtype_code(grad), T, N, grad.stride(0), ptr(starts),
         ptr(ends), E, int(round_scale), ptr(q), q.stride(0), ptr(s), s.stride(0), s.stride(1), ptr(qt),
         qt.stride(0), ptr(st), st.stride(0), st.stride(1), stream_of(grad))
    return q, s, qt, st


@_dual_grouped_op.register_fake
def _(grad, starts, ends, round_scale, col_scales):
    T, N = grad.shape
    cap = padded_capacity(T, starts.numel())
    return (grad.new_empty((T, N), dtype=torch.float8_e4m3fn),
            _scale_buf(grad, T, _cdiv(N, 128), col_scales),
            grad.new_empty((N, cap), dtype=torch.float8_e4m3fn),
            _scale_buf(grad, N, cap // 128, col_scales))


def requantize_grouped_t(x_fp8: torch.Tensor, x_scale: torch.Tensor, expert_starts: torch.Tensor,
                         expert_ends: torch.Tensor):
    """Per-expert 128x128 block re-quantization of row-wise codes, transposed on the padded
    token axis: (codes [K, Tcap], block scales [Tcap/128, ceil(K/128)]).  For each expert it
    equals quantize_fp8_blockwise(dequantize_fp8_rowwise(x_fp8, x_scale)[s_e:e_e]) (reference
    src/kernels.py:784-787 per slice)."""
    _require(x_fp8.is_cuda, "Input must be on CUDA")
    _codes_u8(x_fp8)
    starts, ends = _ranges(expert_starts, expert_ends)
    return _requant_grouped_op(x_fp8, x_scale, starts, ends)


@custom_op("requant_row_to_block_grouped",
           "(Tensor x_fp8, Tensor x_scale, Tensor starts, Tensor ends) -> (Tensor, Tensor)")
def _requant_grouped_op(x_fp8, x_scale, starts, ends):
    q = _rows8(_codes_u8(x_fp8))
    T, K = q.shape
    E = starts.numel()
    cap = padded_capacity(T, E)
    qbt = torch.empty((K, cap), dtype=torch.float8_e4m3fn, device=q.device)
    sblk = torch.empty((cap // 128, _cdiv(K, 128)), dtype=torch.float32, device=q.device)
    xs = _scales_2d(x_scale)
    call("cin_requant_row_to_block_grouped", ptr(q), T, K, q.stride(0), ptr(xs), xs.stride(0),
         xs.stride(1), ptr(starts), ptr(ends), E, ptr(qbt), qbt.stride(0), ptr(sblk),
         sblk.stride(0), stream_of(q))
    return qbt, sblk


@_requant_grouped_op.register_fake
def _(x_fp8, x_scale, starts, ends):
    T, K = x_fp8.shape
    cap = padded_capacity(T, starts.numel())
    return (x_fp8.new_empty((K, cap), dtype=torch.float8_e4m3fn),
            x_fp8.new_empty((cap // 128, _cdiv(K, 128)), dtype=torch.float32))


def fp8_grouped_wgrad(g_t: torch.Tensor, g_st: torch.Tensor, x_bt: torch.Tensor,
                      x_blk: torch.Tensor, expert_starts: torch.Tensor, expert_ends: torch.Tensor,
                      num_tokens: int, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """dW_e = dC_e^T . X_e for every expert in one launch -> [E, N, K].

    g_t/g_st from quantize_fp8_dual_grouped, x_bt/x_blk from requantize_grouped_t (same
    expert ranges over num_tokens rows).  Experts without tokens get zeros."""
    _require(g_t.is_cuda and x_bt.is_cuda, "Input must be on CUDA")
    starts, ends = _ranges(expert_starts, expert_ends)
    _require(x_bt.shape[1] == g_t.shape[1], "operands must share the padded token axis")
    return _grouped_wgrad_op(g_t, g_st, x_bt, x_blk, starts, ends, int(num_tokens), out_dtype)


@custom_op("grouped_wgrad_fp8", "(Tensor g_t, Tensor g_st, Tensor x_bt, Tensor x_blk, Tensor starts, "
           "Tensor ends, int num_tokens, ScalarType out_dtype) -> Tensor")
def _grouped_wgrad_op(g_t, g_st, x_bt, x_blk, starts, ends, num_tokens, out_dtype):
    E = starts.numel()
    N, cap = g_t.shape
    K = x_bt.shape[0]
    a = g_t.view(torch.uint8)
    b = x_bt.view(torch.uint8)
    out = torch.empty((E, N, K), dtype=out_dtype, device=g_t.device)
    st = _scales_2d(g_st)
    call("cin_grouped_gemm_fp8_wgrad", ptr(a), a.stride(0), ptr(st), st.stride(0), st.stride(1), ptr(b),
         b.stride(0), ptr(x_blk), x_blk.stride(0), ptr(starts), ptr(ends), E, int(num_tokens), cap,
         N, K, ptr(out), dtype_code(out), out.stride(1), out.stride(0), stream_of(a))
    return out


@_grouped_wgrad_op.register_fake
def _(g_t, g_st, x_bt, x_blk, starts, ends, num_tokens, out_dtype):
    return g_t.new_empty((starts.numel(), g_t.shape[0], x_bt.shape[0]), dtype=out_dtype)


def fp8_grouped_dgrad(g_fp8: torch.Tensor, g_scale: torch.Tensor, w_codes_t: torch.Tensor,
                      w_scales: torch.Tensor, expert_starts: torch.Tensor,
                      expert_ends: torch.Tensor, n_out_per_expert: int,
                      out_dtype: torch.dtype = torch.float32,
                      out: torch.Tensor | None = None,
                      zero_uncovered: bool = False) -> torch.Tensor:
    """dA[r] = dC[r] . W_e for rows r of expert e -> [T, K].

    w_codes_t [K, E*N] and w_scales [E*N/128, ceil(K/128)] are quantize_fp8_blockwise_t of
    the stacked weights W.reshape(E*N, K); n_out_per_expert = N (multiple of 128)."""
    _require(g_fp8.is_cuda and w_codes_t.is_cuda, "Input must be on CUDA")
    starts, ends = _ranges(expert_starts, expert_ends)
    E = starts.numel()
    T, N = g_fp8.shape
    K, EN = w_codes_t.shape
    _require(N == n_out_per_expert and EN == E * N and N % 128 == 0,
             "w_codes_t must be [K, E*N] with N a multiple of 128")
    if out is None:
        return _grouped_dgrad_op(g_fp8, g_scale, w_codes_t, w_scales, starts, ends, out_dtype,
                                 bool(zero_uncovered))
    return _grouped_dgrad_into(g_fp8, g_scale, w_codes_t, w_scales, starts, ends, out)


def _grouped_dgrad_into(g_fp8, g_scale, w_codes_t, w_scales, starts, ends, out):
    E = starts.numel()
    T, N = g_fp8.shape
    K = w_codes_t.shape[0]
    aq, _ = _kcontig(g_fp8, N)
    b = w_codes_t.view(torch.uint8)
    nbk = w_scales.stride(0)  # scale columns per row block
    # B_e[k, n] = W_e[n, k]: codes at w_codes_t + e*N (row stride E*N); its block scales
    # [kb_out, nb_red] are w_scales[e*N/128 + nb_red, kb_out]
    call("cin_grouped_gemm_fp8", ptr(aq), aq.stride(0), ptr(g_scale), g_scale.stride(0),
         g_scale.stride(1), ptr(b), N, b.stride(0), ptr(w_scales), (N // 128) * nbk, 1, nbk,
         ptr(starts), ptr(ends), E, T, K, N, ptr(out), dtype_code(out), out.stride(0),
         stream_of(aq))
    return out


@custom_op("grouped_dgrad_fp8", "(Tensor g_fp8, Tensor g_scale, Tensor w_codes_t, Tensor w_scales, "
           "Tensor starts, Tensor ends, ScalarType out_dtype, bool zero_uncovered) -> Tensor")
def _grouped_dgrad_op(g_fp8, g_scale, w_codes_t, w_scales, starts, ends, out_dtype, zero_uncovered):
    T, K = g_fp8.shape[0], w_codes_t.shape[0]
    out = (_empty_rows_zeroed(T, K, out_dtype, g_fp8.device, starts, ends) if zero_uncovered
           else torch.empty((T, K), dtype=out_dtype, device=g_fp8.device))
    return _grouped_dgrad_into(g_fp8, g_scale, w_codes_t, w_scales, starts, ends, out)


@_grouped_dgrad_op.register_fake
def _(g_fp8, g_scale, w_codes_t, w_scales, starts, ends, out_dtype, zero_uncovered):
    return g_fp8.new_empty((g_fp8.shape[0], w_codes_t.shape[0]), dtype=out_dtype)


def _empty_rows_zeroed(T: int, ncols: int, dtype: torch.dtype, device, starts, ends) -> torch.Tensor:
    """torch.empty((T, ncols)) whose rows outside every expert range are zero (the grouped
    kernels write exactly the rows inside the ranges)."""
    out = torch.empty((T, ncols), dtype=dtype, device=device)
    call("cin_zero_rows_outside_ranges", ptr(out), out.stride(0) * out.element_size(),
         ncols * out.element_size(), T, ptr(starts), ptr(ends), starts.numel(), stream_of(out))
    return out


def silu_mul_quantize_fp8(h12: torch.Tensor, out_dtype: torch.dtype | None = None,
                          round_scale: bool = False, col_scales: bool = False):
    """quantize_fp8_rowwise((silu(h1) * h2).to(out_dtype)) with [h1 h2] = h12.float().chunk(2, -1),
    in one pass over h12 (reference src/layers.py:72-74 feeding src/kernels.py:178-216).
    h12 [M, 2H] (bf16, fp16 or fp32, H a multiple of 8); out_dtype defaults to h12's dtype.
    Returns (codes float8_e4m3fn [M, H], scales fp32 [M, ceil(H/128)])."""
    _require(h12.is_cuda, "Input must be on CUDA")
    _require(h12.ndim == 2 and h12.shape[1] % 2 == 0, "h12 must be [M, 2H]")
    return _silu_mul_quant_op(h12, out_dtype or h12.dtype, bool(round_scale), bool(col_scales))


@custom_op("silu_mul_quant_rowwise",
           "(Tensor h12, ScalarType out_dtype, bool round_scale, bool col_scales) -> (Tensor, Tensor)")
def _silu_mul_quant_op(h12, out_dtype, round_scale, col_scales):
    M, H = h12.shape[0], h12.shape[1] // 2
    x = h12 if (h12.stride(1) == 1 and h12.data_ptr() % 16 == 0
                and (h12.stride(0) * h12.element_size()) % 16 == 0) else h12.contiguous()
    q = torch.empty((M, H), dtype=torch.float8_e4m3fn, device=h12.device)
    s = _scale_buf(h12, M, _cdiv(H, 128), col_scales)
    call("cin_silu_mul_quant_rowwise", ptr(x), dtype_code(x), M, H, x.stride(0), dtype_code(out_dtype),
         int(round_scale), ptr(q), q.stride(0), ptr(s), s.stride(0), s.stride(1), stream_of(x))
    return q, s


@_silu_mul_quant_op.register_fake
def _(h12, out_dtype, round_scale, col_scales):
    M, H = h12.shape[0], h12.shape[1] // 2
    return (h12.new_empty((M, H), dtype=torch.float8_e4m3fn),
            _scale_buf(h12, M, _cdiv(H, 128), col_scales))


def swiglu_backward(dh: torch.Tensor, h12: torch.Tensor) -> torch.Tensor:
    """Gradient of h = silu(h1) * h2 ([h1 h2] = h12.float().chunk(2, -1)) with respect to
    h12, from dh [M, H] fp32, in one pass: [dh * h2 * silu'(h1), dh * silu(h1)] fp32 [M, 2H]."""
    _require(dh.is_cuda and h12.is_cuda, "Input must be on CUDA")
    M, H = dh.shape
    _require(h12.shape == (M, 2 * H), "h12 must be [M, 2H]")
    return _swiglu_backward_op(dh, h12)


@custom_op("swiglu_backward", "(Tensor dh, Tensor h12) -> Tensor")
def _swiglu_backward_op(dh, h12):
    M, H = dh.shape
    g = dh if (dh.dtype == torch.float32 and dh.stride(1) == 1 and dh.stride(0) % 4 == 0
               and dh.data_ptr() % 16 == 0) else dh.float().contiguous()
    x = h12 if h12.stride(1) == 1 else h12.contiguous()
    out = torch.empty((M, 2 * H), dtype=torch.float32, device=dh.device)
    call("cin_swiglu_backward", ptr(g), g.stride(0), ptr(x), dtype_code(x), x.stride(0), M, H,
         ptr(out), out.stride(0), stream_of(g))
    return out


@_swiglu_backward_op.register_fake
def _(dh, h12):
    return dh.new_empty((dh.shape[0], 2 * dh.shape[1]), dtype=torch.float32)


def swiglu_backward_dual_grouped(dh: torch.Tensor, h12: torch.Tensor, expert_starts: torch.Tensor,
                                  expert_ends: torch.Tensor, round_scale: bool = False,
                                  col_scales: bool = False):
    """quantize_fp8_dual_grouped(swiglu_backward(dh, h12), ...) in one pass, with the same
    outputs bit for bit: the fp32 gradient [T, 2H] is formed tile by tile and never stored.
    H % 128 == 0; other widths take the two calls."""
    _require(dh.is_cuda and h12.is_cuda, "Input must be on CUDA")
    T, H = dh.shape
    _require(h12.shape == (T, 2 * H), "h12 must be [T, 2H]")
    starts, ends = _ranges(expert_starts, expert_ends)
    if H % 128 != 0:
        return _dual_grouped_op(_swiglu_backward_op(dh, h12), starts, ends, bool(round_scale),
                                bool(col_scales))
    return _swiglu_dual_grouped_op(dh, h12, starts, ends, bool(round_scale), bool(col_scales))


@custom_op("swiglu_dual_grouped",
           "(Tensor dh, Tensor h12, Tensor starts, Tensor ends, bool round_scale, bool col_scales) -> "
           "(Tensor, Tensor, Tensor, Tensor)")
def _swiglu_dual_grouped_op(dh, h12, starts, ends, round_scale, col_scales):
    T, H = dh.shape
    g = dh if (dh.dtype == torch.float32 and dh.stride(1) == 1 and dh.stride(0) % 4 == 0
               and dh.data_ptr() % 16 == 0) else dh.float().contiguous()
    x = h12 if (h12.stride(1) == 1 and (h12.stride(0) * h12.element_size()) % 16 == 0
                and h12.data_ptr() % 16 == 0) else h12.contiguous()
    E = starts.numel()
    cap = padded_capacity(T, E)
    dev = dh.device
    q = torch.empty((T, 2 * H), dtype=torch.float8_e4m3fn, device=dev)
    s = _scale_buf(g, T, 2 * H // 128, col_scales)
    qt = torch.empty((2 * H, cap), dtype=torch.float8_e4m3fn, device=dev)
    st = _scale_buf(g, 2 * H, cap // 128, col_scales)
    call("cin_swiglu_dual_grouped", ptr(g), g.stride(0), ptr(x), dtype_code(x), x.stride(0), T, H,
         ptr(starts), ptr(ends), E, int(round_scale), ptr(q), q.stride(0), ptr(s), s.stride(0),
         s.stride(1), ptr(qt), qt.stride(0), ptr(st), st.stride(0), st.stride(1), stream_of(g))
    return q, s, qt, st


@_swiglu_dual_grouped_op.register_fake
def _(dh, h12, starts, ends, round_scale, col_scales):
    T, H = dh.shape
    cap = padded_capacity(T, starts.numel())
    return (dh.new_empty((T, 2 * H), dtype=torch.float8_e4m3fn),
            _scale_buf(dh, T, 2 * H // 128, col_scales),
            dh.new_empty((2 * H, cap), dtype=torch.float8_e4m3fn),
            _scale_buf(dh, 2 * H, cap // 128, col_scales))


def quantize_expert_weights(w12: torch.Tensor, w3: torch.Tensor):
    """Per-expert 128x128 quantization of the stacked SwiGLU weights, with the transposed
    codes the backward needs: ((w12q, w12qt, w12s), (w3q, w3qt, w3s)) from
    quantize_fp8_blockwise_t of w12 [E*2H, D] and w3 [E*D, H] (blocks never straddle two
    experts: 2H and D are multiples of 128)."""
    E, H2, D = w12.shape
    H = H2 // 2
    w12f = w12 if w12.dtype == torch.float32 else w12.float()
    w3f = w3 if w3.dtype == torch.float32 else w3.float()
    return (quantize_fp8_blockwise_t(w12f.reshape(E * H2, D)),
            quantize_fp8_blockwise_t(w3f.reshape(E * D, H)))


def experts_forward(xq: torch.Tensor, xs: torch.Tensor, w12: torch.Tensor, w3: torch.Tensor,
                    starts: torch.Tensor, ends: torch.Tensor, h_dtype: torch.dtype,
                    weights_fp8=None, out_dtype: torch.dtype = torch.float32):
    """FP8 SwiGLU experts on 1x128-quantized sorted rows (xq, xs): GEMM(w12), silu(h1) * h2
    in fp32 cast to h_dtype and quantized in the same pass, GEMM(w3), out_dtype out
    (reference GroupedExperts.forward, src/layers.py:71-75: fp32 values of an fp16 GEMM;
    out_dtype fp16 stores them at that precision).  weights_fp8: optional
    quantize_expert_weights(w12, w3) (a weight cache).  Returns (out [T, D], saved tensors
    for experts_backward).  Rows outside every expert range are zero."""
    E, H2, D = w12.shape
    H = H2 // 2
    if weights_fp8 is None:
        weights_fp8 = quantize_expert_weights(w12, w3)
    (w12q, w12qt, w12s), (w3q, w3qt, w3s) = weights_fp8
    h12 = fp8_grouped_gemm(xq, xs, w12q.view(E, H2, D), w12s.view(E, H2 // 128, -1),
                           starts, ends, out_dtype=torch.bfloat16, zero_uncovered=True)
    hq, hs = silu_mul_quantize_fp8(h12, out_dtype=h_dtype, col_scales=True)
    out = fp8_grouped_gemm(hq, hs, w3q.view(E, D, H), w3s.view(E, D // 128, -1), starts, ends,
                           out_dtype=out_dtype, zero_uncovered=True)
    return out, (xq, xs, w12qt, w12s, h12, hq, hs, w3qt, w3s, starts, ends)


def experts_backward(saved, grad_out: torch.Tensor, dx_dtype: torch.dtype):
    """Backward of experts_forward: the FP8MatmulFunction.backward recipe (reference
    src/kernels.py:763-794) applied per expert to both GEMMs.  Returns (dx [T, D] in dx_dtype
    (bf16 or fp32; its bf16 store is the RNE of the fp32 value), dw12 fp32, dw3 fp32)."""
    xq, xs, w12qt, w12s, h12, hq, hs, w3qt, w3s, starts, ends = saved
    D = xq.shape[1]
    H = hq.shape[1]
    g = grad_out.contiguous()
    gq, gs, gqt, gst = quantize_fp8_dual_grouped(g, starts, ends, col_scales=True)
    dh = fp8_grouped_dgrad(gq, gs, w3qt, w3s, starts, ends, D, out_dtype=torch.float32,
                           zero_uncovered=True)
    hbt, hblk = requantize_grouped_t(hq, hs, starts, ends)
    dw3 = fp8_grouped_wgrad(gqt, gst, hbt, hblk, starts, ends, g.shape[0])
    # silu(h1) * h2 in fp32 (the forward's cast to the input dtype passes the gradient),
    # its gradient quantized both ways in the same pass
    dq, ds, dqt, dst = swiglu_backward_dual_grouped(dh, h12, starts, ends, col_scales=True)
    dx = fp8_grouped_dgrad(dq, ds, w12qt, w12s, starts, ends, 2 * H, out_dtype=dx_dtype,
                           zero_uncovered=True)
    xbt, xblk = requantize_grouped_t(xq, xs, starts, ends)
    dw12 = fp8_grouped_wgrad(dqt, dst, xbt, xblk, starts, ends, g.shape[0])
    return dx, dw12, dw3


class FP8GroupedExpertsFunction(torch.autograd.Function):
    """SwiGLU experts in FP8: out = W3_e (silu(h1) * h2), [h1 h2] = W12_e x for each expert's
    rows (reference GroupedExperts.forward, src/layers.py:56-87: GEMM(w12), silu * mul in
    fp32, cast to the input dtype, GEMM(w3), fp32 out).  Both GEMMs use 1x128 activation
    tiles and 128x128 per-expert weight blocks; the backward applies the
    FP8MatmulFunction.backward recipe per expert (grouped dual quantization of the
    gradient, grouped dgrad with the transposed weight codes, grouped re-quantization of
    the saved inputs and grouped wgrad)."""

    @staticmethod
    def forward(ctx, sorted_x, w12, w3, expert_starts, expert_ends, weights_fp8=None):
        starts, ends = _ranges(expert_starts, expert_ends)
        xq, xs = quantize_fp8_rowwise(sorted_x, col_scales=True)
        out, saved = experts_forward(xq, xs, w12, w3, starts, ends, sorted_x.dtype, weights_fp8)
        ctx.save_for_backward(*saved)
        ctx.x_dtype = sorted_x.dtype
        ctx.w_dtypes = (w12.dtype, w3.dtype)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        # dx straight in the input dtype: the GEMM's bf16 store is the RNE of its fp32 value
        dx_dtype = ctx.x_dtype if ctx.x_dtype in (torch.bfloat16, torch.float32) else torch.float32
        dx, dw12, dw3 = experts_backward(ctx.saved_tensors, grad_out, dx_dtype)
        return (dx.to(ctx.x_dtype), dw12.to(ctx.w_dtypes[0]), dw3.to(ctx.w_dtypes[1]), None, None,
                None)


class GroupedExperts(torch.nn.Module):
    """Drop-in for the reference GroupedExperts (src/layers.py:34-87): stacked SwiGLU expert
    weights w12 [E, 2H, D] (w1 and w2 fused) and w3 [E, D, H], N(0, 0.02) init, forward on
    tokens sorted by expert.  On the GPU it runs FP8 (FP8GroupedExpertsFunction, with
    autograd); on the CPU it keeps the reference's per-expert loop (src/layers.py:78-87)."""

    def __init__(self, n_experts: int, d_model: int, hidden_dim: int):
        super().__init__()
        self.n_experts = n_experts
        self.d_model = d_model
        self.hidden_dim = hidden_dim
        self.w12 = torch.nn.Parameter(torch.empty(n_experts, 2 * hidden_dim, d_model))
        self.w3 = torch.nn.Parameter(torch.empty(n_experts, d_model, hidden_dim))
        self.cache_weights = False  # kernels.set_weight_cache
        self._wcache = WeightCache()
        torch.nn.init.normal_(self.w12, mean=0.0, std=0.02)
        torch.nn.init.normal_(self.w3, mean=0.0, std=0.02)

    def quantized_weights(self):
        """The experts' FP8 weights for this forward: from the weight cache when it is on,
        else freshly quantized (the reference re-quantizes on every forward)."""
        if not _weight_cache_active(self):
            return None
        w12, w3 = self.w12.detach(), self.w3.detach()
        return self._wcache.get([self.w12, self.w3], lambda: quantize_expert_weights(w12, w3))

    def forward(self, sorted_x, expert_starts, expert_ends, max_expert_tokens=None):
        if sorted_x.is_cuda:
            return FP8GroupedExpertsFunction.apply(sorted_x, self.w12, self.w3, expert_starts,
                                                   expert_ends, self.quantized_weights())
        out = torch.zeros(sorted_x.size(0), self.d_model, device=sorted_x.device,
                          dtype=sorted_x.dtype)
        for i in range(self.n_experts):
            start, end = int(expert_starts[i]), int(expert_ends[i])
            if end > start:
                h12 = torch.nn.functional.linear(sorted_x[start:end], self.w12[i])
                h1, h2 = h12.chunk(2, dim=-1)
                out[start:end] = torch.nn.functional.linear(torch.nn.functional.silu(h1) * h2,
                                                            self.w3[i])
        return out
