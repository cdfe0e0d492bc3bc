"""The torch operators behind the drop-in functions (CPU, no GPU needed).

Every launch is registered as a cinnamon_amd:: operator with a shape function, so
torch.compile traces through FP8Linear and the FP8 experts instead of breaking the graph
at a native call (the reference compiles its model, src/train.py:703).  Here the shape
functions run on fake CUDA tensors: the public functions must return the shapes, dtypes
and device the real kernels produce (tests/test_gpu_*.py check the real ones against the
oracle), and a fake-mode trace of FP8Linear and GroupedExperts forward + backward must
consist of these operators and plain torch ops only.
"""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx

from cinnamon_amd import kernels, layers, moe

OPS = ["quant_rowwise", "quant_blockwise", "quant_blockwise_t", "quant_fwd", "quant_dual", "quant_bwd",
       "requant_row_to_block",
       "dequant_rowwise", "dequant", "gemm_fp8_bs", "transpose_u8", "grouped_gemm_f16",
       "grouped_gemm_fp8", "quant_dual_grouped", "requant_row_to_block_grouped",
       "grouped_wgrad_fp8", "grouped_dgrad_fp8", "silu_mul_quant_rowwise", "swiglu_backward",
       "swiglu_dual_grouped", "moe_route", "moe_gather_quant_rowwise", "moe_scatter_quant_rowwise", "moe_gather_sum",
       "moe_combine", "moe_combine_backward", "indexer_scores_fp8", "indexer_weights_grad_fp8", "indexer_quantize",
       "indexer_quantize_k", "indexer_scores_fp8_q"]
F8, F32, BF16 = torch.float8_e4m3fn, torch.float32, torch.bfloat16


def _meta(t):
    return tuple(t.shape), t.dtype, t.device.type


def test_every_operator_is_registered():
    for name in OPS:
        assert hasattr(torch.ops.cinnamon_amd, name), name


def test_shape_functions_match_the_kernels_outputs():
    with FakeTensorMode():
        dev = "cuda"
        x = torch.empty(300, 1100, dtype=BF16, device=dev)
        q, s = kernels.quantize_fp8_rowwise(x)
        assert _meta(q) == ((300, 1100), F8, "cuda") and _meta(s) == ((300, 9), F32, "cuda")
        q, s = kernels.quantize_fp8_rowwise(x, block_size=64)
        assert s.shape == (300, 18)
        q, s = kernels.quantize_fp8_blockwise(x)
        assert _meta(q) == ((300, 1100), F8, "cuda") and _meta(s) == ((3, 9), F32, "cuda")
        q, qt, s = kernels.quantize_fp8_blockwise_t(x)
        assert q.shape == (300, 1100) and qt.shape == (1100, 300) and s.shape == (3, 9)
        q, qt, s = kernels.quantize_fp8_blockwise_t(x, with_rowmajor=False)
        assert q is None and qt.shape == (1100, 300)
        w = torch.empty(260, 1100, dtype=BF16, device=dev)
        xq, xs, wq, wqt, ws = kernels.quantize_fp8_forward(x, w, with_transposed=True)
        assert [t.shape for t in (xq, xs, wq, wqt, ws)] == [(300, 1100), (300, 9), (260, 1100),
                                                            (1100, 260), (3, 9)]
        assert [t.dtype for t in (xq, xs, wq, wqt, ws)] == [F8, F32, F8, F8, F32]
        _, _, wq, wqt, _ = kernels.quantize_fp8_forward(x, w)
        assert wq.shape == (260, 1100) and wqt is None
        q, s, qt, st = kernels.quantize_fp8_dual(x)
        assert [t.shape for t in (q, s, qt, st)] == [(300, 1100), (300, 9), (1100, 300), (1100, 3)]
        assert [t.dtype for t in (q, s, qt, st)] == [F8, F32, F8, F32]
        xq, xs = kernels.quantize_fp8_rowwise(x)
        gy = torch.empty(300, 260, dtype=BF16, device=dev)
        outs = kernels.quantize_fp8_backward(gy, xq, xs)
        assert [t.shape for t in outs] == [(300, 260), (300, 3), (260, 300), (260, 3), (1100, 300), (3, 9)]
        assert [t.dtype for t in outs] == [F8, F32, F8, F32, F8, F32]
        b, bs = kernels.requantize_rowwise_to_blockwise(xq, xs)
        assert _meta(b) == ((300, 1100), F8, "cuda") and bs.shape == (3, 9)
        b, bs = kernels.requantize_rowwise_to_blockwise(xq, xs, transposed=True)
        assert b.shape == (1100, 300)
        assert _meta(kernels.dequantize_fp8_rowwise(xq, xs)) == ((300, 1100), F32, "cuda")
        wq, ws = kernels.quantize_fp8_blockwise(x)
        assert _meta(kernels.dequantize_fp8(wq, ws)) == ((300, 1100), BF16, "cuda")
        a = torch.empty(256, 512, dtype=F8, device=dev)
        sa = torch.empty(256, 4, dtype=F32, device=dev)
        bt = torch.empty(384, 512, dtype=F8, device=dev)
        sbt = torch.empty(3, 4, dtype=F32, device=dev)
        assert _meta(kernels.fp8_gemm_bs(a, sa, bt, sbt)) == ((256, 384), BF16, "cuda")
        assert kernels.fp8_gemm_bs(a, sa, bt, sbt, F32).dtype == F32
        bkn = torch.empty(512, 384, dtype=F8, device=dev)   # B [K, N], row-major: transposed on device
        assert _meta(kernels.fp8_matmul_dsv3(a, bkn, sa, sbt.t())) == ((256, 384), BF16, "cuda")
        # grouped
        T, E, D, H = 1000, 4, 256, 384
        starts = torch.tensor([0, 100, 100, 600], device=dev)
        ends = torch.tensor([100, 100, 600, 1000], device=dev)
        xg = torch.empty(T, D, dtype=BF16, device=dev)
        w = torch.empty(E, H, D, dtype=F32, device=dev)
        assert _meta(kernels.moe_grouped_gemm(xg, w, starts, ends)) == ((T, H), torch.float16, "cuda")
        aq, asc = kernels.quantize_fp8_rowwise(xg)
        wq, wqt, wsc = kernels.quantize_fp8_blockwise_t(w.reshape(E * H, D))
        out = layers.fp8_grouped_gemm(aq, asc, wq.view(E, H, D), wsc.view(E, H // 128, -1), starts, ends)
        assert _meta(out) == ((T, H), BF16, "cuda")
        g = torch.empty(T, H, dtype=BF16, device=dev)
        cap = layers.padded_capacity(T, E)
        gq, gs, gqt, gst = layers.quantize_fp8_dual_grouped(g, starts, ends)
        assert [t.shape for t in (gq, gs, gqt, gst)] == [(T, H), (T, 3), (H, cap), (H, cap // 128)]
        xbt, xblk = layers.requantize_grouped_t(aq, asc, starts, ends)
        assert xbt.shape == (D, cap) and xblk.shape == (cap // 128, 2) and xbt.dtype == F8
        dw = layers.fp8_grouped_wgrad(gqt, gst, xbt, xblk, starts, ends, T)
        assert _meta(dw) == ((E, H, D), F32, "cuda")
        dx = layers.fp8_grouped_dgrad(gq, gs, wqt, wsc, starts, ends, H, zero_uncovered=True)
        assert _meta(dx) == ((T, D), F32, "cuda")
        h12 = torch.empty(T, 2 * H, dtype=BF16, device=dev)
        hq, hs = layers.silu_mul_quantize_fp8(h12)
        assert _meta(hq) == ((T, H), F8, "cuda") and hs.shape == (T, 3)
        dh = torch.empty(T, H, dtype=F32, device=dev)
        assert _meta(layers.swiglu_backward(dh, h12)) == ((T, 2 * H), F32, "cuda")
        dq, ds, dqt, dst = layers.swiglu_backward_dual_grouped(dh, h12, starts, ends)
        assert [t.shape for t in (dq, ds, dqt, dst)] == [(T, 2 * H), (T, 6), (2 * H, cap),
                                                         (2 * H, cap // 128)]
        # indexer scores
        qi = torch.empty(2, 100, 4, 128, dtype=BF16, device=dev)
        ki = torch.empty(2, 90, 128, dtype=BF16, device=dev)
        wi = torch.empty(2, 100, 4, dtype=F32, device=dev)
        assert _meta(kernels.indexer_scores_fp8(qi, ki, wi, 0.125)) == ((2, 100, 90), F32, "cuda")
        q8i = torch.empty(2, 100, 4, 128, dtype=F8, device=dev)
        k8i = torch.empty(2, 90, 128, dtype=F8, device=dev)
        dwi = torch.ops.cinnamon_amd.indexer_weights_grad_fp8(
            q8i, torch.empty(2, 100, 4, device=dev), k8i, torch.empty(2, 90, device=dev),
            torch.empty(2, 100, 90, device=dev), 0.125)
        assert _meta(dwi) == ((2, 100, 4), F32, "cuda")


def _op_targets(gm):
    names = set()
    for n in gm.graph.nodes:
        if n.op == "call_function":
            names.add(str(n.target))
    return names


class _Ctx:
    """Stands in for autograd's ctx: without a GPU the autograd engine cannot run a
    backward pass on fake CUDA tensors, so the trace calls forward and backward directly."""

    def save_for_backward(self, *tensors):
        self.saved_tensors = tensors


@pytest.mark.parametrize("round_scale", [False, True])
def test_fp8_linear_forward_backward_traces_to_operators(round_scale):
    fn = kernels.FP8MatmulFunction

    def step(x, w, gy):
        ctx = _Ctx()
        y = fn.forward(ctx, x, w, round_scale)
        dx, dw, *_ = fn.backward(ctx, gy)
        return y, dx, dw

    with FakeTensorMode(allow_non_fake_inputs=True):
        w = torch.empty(384, 512, dtype=F32, device="cuda")
        x = torch.empty(4, 64, 512, dtype=BF16, device="cuda")
        gy = torch.empty(4, 64, 384, dtype=BF16, device="cuda")
        gm = make_fx(step, tracing_mode="fake")(x, w, gy)
        y, dx, dw = step(x, w, gy)
        assert _meta(y) == ((4, 64, 384), BF16, "cuda")
        assert _meta(dx) == ((4, 64, 512), BF16, "cuda") and _meta(dw) == ((384, 512), BF16, "cuda")
    ops = _op_targets(gm)
    for name in ["quant_fwd", "gemm_fp8_bs", "quant_bwd"]:
        assert any(f"cinnamon_amd.{name}" in o for o in ops), (name, ops)


def test_grouped_experts_forward_backward_traces_to_operators():
    fn = layers.FP8GroupedExpertsFunction
    T, E, D, H = 700, 4, 256, 256

    def step(x, w12, w3, starts, ends, gy):
        ctx = _Ctx()
        y = fn.forward(ctx, x, w12, w3, starts, ends)
        dx, dw12, dw3, *_ = fn.backward(ctx, gy)
        return y, dx, dw12, dw3

    with FakeTensorMode(allow_non_fake_inputs=True):
        w12 = torch.empty(E, 2 * H, D, dtype=F32, device="cuda")
        w3 = torch.empty(E, D, H, dtype=F32, device="cuda")
        starts = torch.empty(E, dtype=torch.int64, device="cuda")
        ends = torch.empty(E, dtype=torch.int64, device="cuda")
        x = torch.empty(T, D, dtype=BF16, device="cuda")
        gy = torch.empty(T, D, dtype=F32, device="cuda")
        gm = make_fx(step, tracing_mode="fake")(x, w12, w3, starts, ends, gy)
        y, dx, dw12, dw3 = step(x, w12, w3, starts, ends, gy)
        assert _meta(y) == ((T, D), F32, "cuda") and _meta(dx) == ((T, D), BF16, "cuda")
        assert _meta(dw12) == ((E, 2 * H, D), F32, "cuda") and _meta(dw3) == ((E, D, H), F32, "cuda")
    ops = _op_targets(gm)
    for name in ["grouped_gemm_fp8", "silu_mul_quant_rowwise", "quant_dual_grouped",
                 "grouped_dgrad_fp8", "requant_row_to_block_grouped", "grouped_wgrad_fp8",
                 "swiglu_dual_grouped"]:
        assert any(f"cinnamon_amd.{name}" in o for o in ops), (name, ops)


def test_moe_dispatch_shape_functions_and_trace():
    T, k, E, D, H = 600, 4, 8, 256, 256

    def step(x, w12, w3, top_idx, scores, dout):
        perm, inv, counts, starts, ends = moe.moe_route(top_idx, E)
        ys, saved = moe.RoutedExpertsFunction.experts(x, w12, w3, perm, inv, starts, ends, k)
        out = moe.moe_combine(ys, scores, inv)
        dys, dsc = moe.moe_combine_backward(dout, ys, scores, perm, inv, dy_dtype=BF16)
        dx, dw12, dw3 = moe.RoutedExpertsFunction.experts_backward(saved, dys, inv, k, x.dtype)
        return perm, inv, counts, ys, out, dys, dsc, dx, dw12, dw3

    with FakeTensorMode(allow_non_fake_inputs=True):
        x = torch.empty(T, D, dtype=BF16, device="cuda")
        w12 = torch.empty(E, 2 * H, D, dtype=F32, device="cuda")
        w3 = torch.empty(E, D, H, dtype=F32, device="cuda")
        top_idx = torch.empty(T, k, dtype=torch.int64, device="cuda")
        scores = torch.empty(T, k, dtype=BF16, device="cuda")
        dout = torch.empty(T, D, dtype=F32, device="cuda")
        gm = make_fx(step, tracing_mode="fake")(x, w12, w3, top_idx, scores, dout)
        perm, inv, counts, ys, out, dys, dsc, dx, dw12, dw3 = step(x, w12, w3, top_idx, scores, dout)
        assert _meta(perm) == ((T * k,), torch.int64, "cuda") and _meta(inv) == ((T * k,), torch.int32, "cuda")
        assert _meta(counts) == ((E,), torch.int64, "cuda")
        # sorted expert outputs in fp16 (the reference's expert GEMMs are fp16), their gradient
        # in bf16 (fp32's range for small gradients)
        assert _meta(ys) == ((T * k, D), torch.float16, "cuda") and _meta(out) == ((T, D), F32, "cuda")
        assert _meta(dys) == ((T * k, D), BF16, "cuda") and _meta(dsc) == ((T, k), F32, "cuda")
        assert _meta(dx) == ((T, D), BF16, "cuda") and dw12.shape == (E, 2 * H, D) and dw3.shape == (E, D, H)
        q, s = moe.moe_gather_quantize(x, perm, k)
        assert _meta(q) == ((T * k, D), F8, "cuda") and _meta(s) == ((T * k, 2), F32, "cuda")
        q, s = moe.moe_gather_quantize(x, perm, k, inv=inv)
        assert _meta(q) == ((T * k, D), F8, "cuda") and _meta(s) == ((T * k, 2), F32, "cuda")
        assert _meta(moe.moe_gather_sum(dys, inv, k, BF16)) == ((T, D), BF16, "cuda")
    ops = _op_targets(gm)
    for name in ["moe_route", "moe_scatter_quant_rowwise", "moe_combine", "moe_combine_backward",
                 "moe_gather_sum", "grouped_gemm_fp8", "grouped_wgrad_fp8"]:
        assert any(f"cinnamon_amd.{name}" in o for o in ops), (name, ops)


def test_eager_calls_bypass_the_dispatcher_only_outside_tracing():
    """kernels._run calls an operator's launch function directly only for plain tensors
    outside tracing; FakeTensorMode, make_fx and torch.compile keep the operators (their shape
    functions and schemas are what tracing needs)."""
    from torch.fx.experimental.proxy_tensor import make_fx

    t = torch.zeros(4)
    assert kernels._plain_eager(t, t)
    with FakeTensorMode():
        assert not kernels._plain_eager(torch.empty(4))
    seen = []
    make_fx(lambda x: seen.append(kernels._plain_eager(x)) or x + 1)(t)
    assert seen == [False]
    assert all(op in kernels._LAUNCH for op in (kernels._quant_fwd_op, kernels._gemm_bs_op,
                                                 kernels._quant_bwd_op, kernels._quant_rowwise_op))
