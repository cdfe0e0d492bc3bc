"""Device-side MoE dispatch and combine around the FP8 grouped experts.

Counterpart of the permute -> grouped experts -> unpermute block of the reference's
MoE.forward (src/layers.py:126-157):

  reference                                      here
  expanded_idx.sort(), token_indices, bincount,  moe_route: stable counting sort on the
  cumsum, max_expert_tokens = .item()            device, int64 expert ranges, no host sync
  sorted_x = flat_x[token_indices] (bf16),       moe_gather_quantize: the 1x128 quantizer
  then the experts quantize it                   reads x rows through the permutation
  sorted_out * sorted_scores, scatter_add_       moe_combine: per-token sum in sorted order

``routed_experts`` chains them with layers.experts_forward/backward; its gradients reach
x, the expert weights and the routing scores.  Every launch is a cinnamon_amd:: torch
operator (torch.compile traces through it).  The sort is stable, so within an expert the
rows keep token order (the reference's unstable sort may order them differently; each
row's result does not depend on its position, and the combine adds a token's terms in
sorted position order, the order of a sequential scatter_add_).
"""
from __future__ import annotations

import torch

from . import layers
from ._lib import call, dtype_code, ptr, stream_of
from .kernels import _cdiv, _require, _scale_buf, custom_op

_ROUTE_CHUNK = 1024  # assignments per route workgroup (csrc/moe.hip kChunk)
MAX_EXPERTS = 4096
MAX_TOP_K = 16

__all__ = ["moe_route", "moe_gather_quantize", "moe_gather_sum", "moe_combine",
           "moe_combine_backward", "RoutedExpertsFunction", "routed_experts"]


# ---------------------------------------------------------------------------
# Routing (reference src/layers.py:133-148)
# ---------------------------------------------------------------------------
def moe_route(top_idx: torch.Tensor, n_experts: int):
    """Stable sort of the flattened top-k ids on the device.

    top_idx [T, k] integer expert ids -> (perm int64 [T*k], inv int32 [T*k], counts,
    starts, ends int64 [E]).  perm[r] = t*k + j of the assignment at sorted position r
    (the reference's sort_order; token_indices = perm // k), inv its inverse.  Ids
    outside [0, E) are dropped: inv -1, and perm -1 at the positions past the kept ones.
    """
    _require(top_idx.is_cuda, "Input must be on CUDA")
    _require(top_idx.ndim == 2, "top_idx must be [n_tokens, top_k]")
    _require(1 <= n_experts <= MAX_EXPERTS, f"n_experts must be in [1, {MAX_EXPERTS}]")
    return _route_op(top_idx.to(torch.int64).contiguous(), int(n_experts))


@custom_op("moe_route", "(Tensor idx, int n_experts) -> (Tensor, Tensor, Tensor, Tensor, Tensor)")
def _route_op(idx, n_experts):
    T, k = idx.shape
    A = T * k
    dev = idx.device
    perm = torch.empty(A, dtype=torch.int64, device=dev)
    inv = torch.empty(A, dtype=torch.int32, device=dev)
    counts = torch.empty(n_experts, dtype=torch.int64, device=dev)
    starts = torch.empty(n_experts, dtype=torch.int64, device=dev)
    ends = torch.empty(n_experts, dtype=torch.int64, device=dev)
    nws = max(1, 2 * _cdiv(A, _ROUTE_CHUNK) * n_experts)
    ws = torch.empty(nws, dtype=torch.int32, device=dev)
    call("cin_moe_route", ptr(idx), T, k, n_experts, ptr(perm), ptr(inv), ptr(counts), ptr(starts),
         ptr(ends), ptr(ws), nws, stream_of(idx))
    return perm, inv, counts, starts, ends


@_route_op.register_fake
def _(idx, n_experts):
    A = idx.shape[0] * idx.shape[1]
    i64 = torch.int64
    return (idx.new_empty((A,), dtype=i64), idx.new_empty((A,), dtype=torch.int32),
            idx.new_empty((n_experts,), dtype=i64), idx.new_empty((n_experts,), dtype=i64),
            idx.new_empty((n_experts,), dtype=i64))


# ---------------------------------------------------------------------------
# Gather fused into the 1x128 quantization, and its backward (reference :139-141)
# ---------------------------------------------------------------------------
def moe_gather_quantize(x: torch.Tensor, perm: torch.Tensor, top_k: int, round_scale: bool = False,
                        inv: torch.Tensor | None = None, col_scales: bool = False):
    """quantize_fp8_rowwise(x[perm // top_k]) bit for bit, without the gathered rows:
    (codes float8_e4m3fn [A, D], scales fp32 [A, ceil(D/128)]); rows where perm is -1 get the
    quantization of a zero row.  With ``inv`` (moe_route's inverse map) each token row is
    quantized once and written to its top_k sorted rows (one read of x instead of top_k);
    without it each sorted row reads its token row."""
    _require(x.is_cuda and perm.is_cuda, "Input must be on CUDA")
    _require(x.ndim == 2 and perm.ndim == 1, "x must be [n_tokens, d] and perm 1-D")
    _require(top_k >= 1, "top_k must be >= 1")
    if inv is not None:
        _require(inv.numel() == x.shape[0] * top_k, "inv must hold n_tokens * top_k entries")
        return _scatter_quant_op(x, perm.to(torch.int64), inv.to(torch.int32), int(top_k),
                                 bool(round_scale), bool(col_scales))
    return _gather_quant_op(x, perm.to(torch.int64), int(top_k), bool(round_scale), bool(col_scales))


def _codes_rows8(A, D, like):
    """[A, D] e4m3 codes whose rows start 8 bytes apart at least (the quantizer stores 8 codes
    at a time): a view of a buffer with rows padded to a multiple of 8 when D is not."""
    Dp = _cdiv(D, 8) * 8
    buf = like.new_empty((A, Dp), dtype=torch.float8_e4m3fn)
    return buf if Dp == D else buf[:, :D]


@custom_op("moe_gather_quant_rowwise",
           "(Tensor x, Tensor perm, int top_k, bool round_scale, bool col_scales) -> (Tensor, Tensor)")
def _gather_quant_op(x, perm, top_k, round_scale, col_scales):
    x = _x_rows16(x)
    A = perm.numel()
    T, D = x.shape
    pm = perm.contiguous()
    q = _codes_rows8(A, D, x)
    s = _scale_buf(x, A, _cdiv(D, 128), col_scales)
    call("cin_moe_gather_quant_rowwise", ptr(x), dtype_code(x), T, D, x.stride(0), ptr(pm), A, top_k,
         int(round_scale), ptr(q), q.stride(0), ptr(s), s.stride(0), s.stride(1), stream_of(x))
    return q, s


@_gather_quant_op.register_fake
def _(x, perm, top_k, round_scale, col_scales):
    A, D = perm.shape[0], x.shape[1]
    return _codes_rows8(A, D, x), _scale_buf(x, A, _cdiv(D, 128), col_scales)


def _x_rows16(x):
    """x with unit column stride and 16-byte aligned rows (the quantizer loads 16 bytes at a
    time): x itself when it qualifies, else a copy whose rows are padded to 16 bytes (the
    padding is never read: the kernel loads the last chunk of a row element by element)."""
    es = x.element_size()
    if x.stride(1) == 1 and x.data_ptr() % 16 == 0 and (x.stride(0) * es) % 16 == 0:
        return x
    T, D = x.shape
    per = 16 // es
    buf = x.new_empty((T, _cdiv(max(D, 1), per) * per))
    buf[:, :D].copy_(x)
    return buf[:, :D]


@custom_op("moe_scatter_quant_rowwise",
           "(Tensor x, Tensor perm, Tensor inv, int top_k, bool round_scale, bool col_scales) -> "
           "(Tensor, Tensor)")
def _scatter_quant_op(x, perm, inv, top_k, round_scale, col_scales):
    x = _x_rows16(x)
    A = perm.numel()
    T, D = x.shape
    pm, iv = perm.contiguous(), inv.contiguous()
    q = _codes_rows8(A, D, x)
    s = _scale_buf(x, A, _cdiv(D, 128), col_scales)
    if col_scales:
        # a token's scales go once into a token-major table, then to its sorted rows with
        # stores that run along the rows (308 -> 252 us at config 3; with row-major scales
        # the stores the kernel makes itself are faster, 263 against 326 us)
        ws = torch.empty(T * _cdiv(D, 128), dtype=torch.float32, device=x.device)
        call("cin_moe_scatter_quant_rowwise_ws", ptr(x), dtype_code(x), T, D, x.stride(0), ptr(iv),
             top_k, ptr(pm), A, int(round_scale), ptr(q), q.stride(0), ptr(s), s.stride(0), s.stride(1),
             ptr(ws), stream_of(x))
    else:
        call("cin_moe_scatter_quant_rowwise", ptr(x), dtype_code(x), T, D, x.stride(0), ptr(iv), top_k,
             ptr(pm), A, int(round_scale), ptr(q), q.stride(0), ptr(s), s.stride(0), s.stride(1),
             stream_of(x))
    return q, s


@_scatter_quant_op.register_fake
def _(x, perm, inv, top_k, round_scale, col_scales):
    A, D = perm.shape[0], x.shape[1]
    return _codes_rows8(A, D, x), _scale_buf(x, A, _cdiv(D, 128), col_scales)


def moe_gather_sum(g: torch.Tensor, inv: torch.Tensor, top_k: int,
                   out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Gradient of x[perm // top_k]: out[t] = sum of g[r] over token t's sorted positions r,
    in increasing r, fp32 sums -> [T, D] in out_dtype (T = inv.numel() // top_k)."""
    _require(g.is_cuda and inv.is_cuda, "Input must be on CUDA")
    _require(1 <= top_k <= MAX_TOP_K, f"top_k must be in [1, {MAX_TOP_K}]")
    _require(inv.numel() % top_k == 0, "inv must hold n_tokens * top_k entries")
    return _gather_sum_op(g, inv.to(torch.int32), int(top_k), out_dtype)


@custom_op("moe_gather_sum", "(Tensor g, Tensor inv, int top_k, ScalarType out_dtype) -> Tensor")
def _gather_sum_op(g, inv, top_k, out_dtype):
    gc = g if g.stride(1) == 1 else g.contiguous()
    iv = inv.contiguous()
    T = iv.numel() // top_k
    A, D = gc.shape
    out = torch.empty((T, D), dtype=out_dtype, device=g.device)
    call("cin_moe_gather_sum", ptr(gc), dtype_code(gc), gc.stride(0), ptr(iv), T, top_k, A, D,
         ptr(out), dtype_code(out), out.stride(0), stream_of(gc))
    return out


@_gather_sum_op.register_fake
def _(g, inv, top_k, out_dtype):
    return g.new_empty((inv.shape[0] // top_k, g.shape[1]), dtype=out_dtype)


# ---------------------------------------------------------------------------
# Weighted combine and its backward (reference :151-154)
# ---------------------------------------------------------------------------
def moe_combine(sorted_out: torch.Tensor, top_scores: torch.Tensor, inv: torch.Tensor) -> torch.Tensor:
    """routed_out [T, D] fp32 = sum over token t's assignments of sorted_out[r] *
    top_scores[t, j], added in increasing sorted position r (sorted_out fp32, fp16 or bf16,
    widened exactly)."""
    _require(sorted_out.is_cuda and top_scores.is_cuda and inv.is_cuda, "Input must be on CUDA")
    _require(top_scores.ndim == 2 and 1 <= top_scores.shape[1] <= MAX_TOP_K,
             f"top_scores must be [n_tokens, top_k] with top_k <= {MAX_TOP_K}")
    _require(inv.numel() == top_scores.numel(), "inv must hold n_tokens * top_k entries")
    _require(sorted_out.dtype in (torch.float32, torch.float16, torch.bfloat16),
             "sorted_out must be fp32, fp16 or bf16 (the experts' output)")
    return _combine_op(sorted_out, top_scores, inv.to(torch.int32))


@custom_op("moe_combine", "(Tensor y, Tensor scores, Tensor inv) -> Tensor")
def _combine_op(y, scores, inv):
    yc = y if y.stride(1) == 1 else y.contiguous()
    sc = scores if scores.stride(1) == 1 else scores.contiguous()
    iv = inv.contiguous()
    T, k = sc.shape
    A, D = yc.shape
    out = torch.empty((T, D), dtype=torch.float32, device=y.device)
    call("cin_moe_combine", ptr(yc), dtype_code(yc), yc.stride(0), ptr(sc), dtype_code(sc), sc.stride(0),
         ptr(iv), T, k, A, D, ptr(out), out.stride(0), stream_of(yc))
    return out


@_combine_op.register_fake
def _(y, scores, inv):
    return y.new_empty((scores.shape[0], y.shape[1]), dtype=torch.float32)


def moe_combine_backward(dout: torch.Tensor, sorted_out: torch.Tensor, top_scores: torch.Tensor,
                         perm: torch.Tensor, inv: torch.Tensor, dy_dtype: torch.dtype | None = None):
    """Gradients of moe_combine: (d sorted_out [A, D], d top_scores [T, k] fp32).

    d sorted_out is the fp32 product dout * score rounded (RNE) to dy_dtype, by default
    sorted_out's dtype (the dtype autograd gives the gradient of a tensor).  For fp16 sorted
    outputs, dy_dtype=torch.bfloat16 keeps tiny gradients: a loss averaged over many tokens
    gives row gradients of 1e-6 and below, which fp16 holds only as subnormals (and flushes
    below 6e-8), while bf16 keeps fp32's range at the same traffic; RoutedExpertsFunction
    asks for it."""
    _require(dout.is_cuda and sorted_out.is_cuda, "Input must be on CUDA")
    if dy_dtype is None:
        dy_dtype = sorted_out.dtype
    _require(dy_dtype in (torch.float32, torch.bfloat16, torch.float16), "dy_dtype must be fp32, bf16 or fp16")
    return _combine_bwd_op(dout.float(), sorted_out, top_scores, perm.to(torch.int64),
                           inv.to(torch.int32), dy_dtype)


@custom_op("moe_combine_backward",
           "(Tensor dout, Tensor y, Tensor scores, Tensor perm, Tensor inv, ScalarType dy_dtype)"
           " -> (Tensor, Tensor)")
def _combine_bwd_op(dout, y, scores, perm, inv, dy_dtype):
    dc = dout if dout.stride(1) == 1 else dout.contiguous()
    yc = y if y.stride(1) == 1 else y.contiguous()
    sc = scores if scores.stride(1) == 1 else scores.contiguous()
    pm, iv = perm.contiguous(), inv.contiguous()
    T, k = sc.shape
    A, D = yc.shape
    dy = torch.empty((A, D), dtype=dy_dtype, device=y.device)
    ds = torch.empty((T, k), dtype=torch.float32, device=y.device)
    call("cin_moe_combine_backward", ptr(dc), dc.stride(0), ptr(yc), dtype_code(yc), yc.stride(0),
         ptr(sc), dtype_code(sc), sc.stride(0), ptr(pm), ptr(iv), T, k, A, D, ptr(dy), dtype_code(dy),
         dy.stride(0), ptr(ds), stream_of(yc))
    return dy, ds


@_combine_bwd_op.register_fake
def _(dout, y, scores, perm, inv, dy_dtype):
    return (y.new_empty(y.shape, dtype=dy_dtype),
            y.new_empty(scores.shape, dtype=torch.float32))


# ---------------------------------------------------------------------------
# Autograd and the routed-experts block
# ---------------------------------------------------------------------------
class RoutedExpertsFunction(torch.autograd.Function):
    """The routed block as one autograd node: gather-quantize -> FP8 SwiGLU experts ->
    weighted combine, with gradients for x, the expert weights and the routing scores.

    The sorted expert outputs [A, D] are stored in fp16: the reference's routed experts
    return fp16 GEMM results (src/layers.py:69-75), and fp16 halves the traffic of the down
    GEMM's output, the combine and its backward.  They stay inside this node, so their
    gradient is not cast back to fp16 by autograd: the combine backward writes it in bf16
    (fp32's range) for the experts' backward, and the sorted-row input gradients come back
    in bf16 too, each token's sum added in fp32 and rounded once to x's dtype."""

    @staticmethod
    def forward(ctx, x, w12, w3, top_scores, perm, inv, starts, ends, top_k, weights_fp8=None):
        ys, saved = RoutedExpertsFunction.experts(x, w12, w3, perm, inv, starts, ends, top_k, weights_fp8)
        ctx.save_for_backward(*saved, ys, top_scores, perm, inv)
        ctx.top_k = top_k
        ctx.x_dtype = x.dtype
        ctx.w_dtypes = (w12.dtype, w3.dtype)
        return moe_combine(ys, top_scores, inv)

    @staticmethod
    def backward(ctx, dout):
        *saved, ys, top_scores, perm, inv = ctx.saved_tensors
        dy, ds = moe_combine_backward(dout, ys, top_scores, perm, inv,
                                      dy_dtype=torch.float32 if ys.dtype == torch.float32 else torch.bfloat16)
        dx, dw12, dw3 = RoutedExpertsFunction.experts_backward(tuple(saved), dy, inv, ctx.top_k, ctx.x_dtype)
        return (dx, dw12.to(ctx.w_dtypes[0]), dw3.to(ctx.w_dtypes[1]), ds.to(top_scores.dtype),
                None, None, None, None, None, None)

    @staticmethod
    def experts(x, w12, w3, perm, inv, starts, ends, top_k, weights_fp8=None):
        """Sorted expert outputs (fp16 [A, D]) and the tensors their backward needs."""
        xq, xs = moe_gather_quantize(x, perm, top_k, inv=inv, col_scales=True)
        return layers.experts_forward(xq, xs, w12, w3, starts, ends, x.dtype, weights_fp8,
                                      out_dtype=torch.float16)

    @staticmethod
    def experts_backward(saved, dy, inv, top_k, x_dtype):
        """(dx, dw12, dw3) from the sorted outputs' gradient dy [A, D] (bf16 or fp32)."""
        dxs, dw12, dw3 = layers.experts_backward(saved, dy, torch.bfloat16)
        return moe_gather_sum(dxs, inv, top_k, x_dtype), dw12, dw3


def routed_experts(experts: layers.GroupedExperts, x: torch.Tensor, top_idx: torch.Tensor,
                   top_scores: torch.Tensor):
    """The routed part of MoE.forward (reference src/layers.py:126-157) on the device.

    x [n_tokens, d_model] (bf16/fp16/fp32), top_idx [n_tokens, k] expert ids, top_scores
    [n_tokens, k] gate weights.  Returns (routed_out [n_tokens, d_model] fp32, expert_counts
    int64 [E]) -- the reference's routed_out (before the view) and the bincount it feeds to
    the expert-bias update.  Autograd reaches x, experts.w12 / w3 and top_scores.
    """
    _require(x.is_cuda, "Input must be on CUDA")
    _require(top_idx.shape == top_scores.shape and top_idx.shape[0] == x.shape[0],
             "top_idx and top_scores must be [n_tokens, top_k]")
    k = top_idx.shape[1]
    _require(1 <= k <= MAX_TOP_K, f"top_k must be in [1, {MAX_TOP_K}]")
    perm, inv, counts, starts, ends = moe_route(top_idx, experts.n_experts)
    out = RoutedExpertsFunction.apply(x, experts.w12, experts.w3, top_scores, perm, inv, starts, ends, k,
                                      experts.quantized_weights())
    return out, counts
