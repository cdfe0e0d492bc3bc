"""torch.compile through the FP8 layers (GPU).

The reference compiles its training model (src/train.py:703).  Every native launch here
is a cinnamon_amd:: torch operator with a shape function, so dynamo captures FP8Linear
and the FP8 experts forward + backward in one graph (fullgraph=True fails on any graph
break) and the compiled step runs the same kernels as eager: losses and gradients must be
bit-identical.  The aot_eager backend keeps the surrounding torch ops unfused, so no code
generator is involved.  opcheck checks each operator's schema and shape function against
its real outputs.
"""
import pytest
import torch

from cinnamon_amd import kernels, layers

pytestmark = pytest.mark.gpu


def _grads(step, params, *inputs):
    for p in params:
        p.grad = None
    loss = step(*inputs)
    loss.backward()
    return loss.detach().clone(), [p.grad.clone() for p in params]


@pytest.mark.parametrize("round_scale", [False, True])
def test_compiled_fp8_linear_matches_eager(dev, round_scale):
    torch.manual_seed(0)
    lin = kernels.FP8Linear(512, 384, round_scale=round_scale).to(dev)
    x = torch.randn(2, 300, 512, device=dev).to(torch.bfloat16).requires_grad_(True)

    def step(x):
        return lin(x).float().square().mean()

    params = [x, lin.weight]
    l0, g0 = _grads(step, params, x)
    compiled = torch.compile(step, backend="aot_eager", fullgraph=True)
    l1, g1 = _grads(compiled, params, x)
    l2, g2 = _grads(compiled, params, x)
    assert torch.allclose(l0, l1, rtol=1e-6, atol=0) and torch.equal(l1, l2)
    for a, b, c in zip(g0, g1, g2):
        assert torch.equal(a, b) and torch.equal(b, c)


def test_compiled_fp8_experts_match_eager(dev):
    torch.manual_seed(1)
    E, D, H = 4, 256, 256
    mod = layers.GroupedExperts(E, D, H).to(dev)
    counts = torch.tensor([300, 0, 170, 530])
    ends = counts.cumsum(0)
    starts = (ends - counts).to(dev)
    ends = ends.to(dev)
    x = torch.randn(int(counts.sum()), D, device=dev).to(torch.bfloat16).requires_grad_(True)

    def step(x):
        return mod(x, starts, ends).square().mean()

    params = [x, mod.w12, mod.w3]
    l0, g0 = _grads(step, params, x)
    compiled = torch.compile(step, backend="aot_eager", fullgraph=True)
    l1, g1 = _grads(compiled, params, x)
    assert torch.allclose(l0, l1, rtol=1e-6, atol=0)
    for a, b in zip(g0, g1):
        assert torch.equal(a, b)


def test_compiled_indexer_scores_match_eager(dev):
    """The FP8 indexer scoring (src/attention.py:288-300) and its weights gradient in one
    compiled graph: same kernels, bit-identical scores and gradients."""
    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 200, 4, 128, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(2, 200, 128, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(2, 200, 4, generator=g) * 0.5).to(dev).requires_grad_(True)
    gs = torch.randn(2, 200, 200, generator=g).to(dev)

    def step(w):
        return (kernels.indexer_scores_fp8(q, k, w, 0.125) * gs).sum()

    l0, g0 = _grads(step, [w], w)
    compiled = torch.compile(step, backend="aot_eager", fullgraph=True)
    l1, g1 = _grads(compiled, [w], w)
    assert torch.equal(l0, l1) and torch.equal(g0[0], g1[0])


def test_opcheck_operators(dev):
    g = torch.Generator(device=dev).manual_seed(2)
    x = torch.randn(256, 384, device=dev, generator=g).to(torch.bfloat16)
    # opcheck's schema test does arithmetic on inputs and outputs, which torch does not
    # implement for float8_e4m3fn: operators with fp8 outputs get the shape-function test
    # only, and fp8 inputs go in as their uint8 views (the operators take either)
    full, f8 = ("test_schema", "test_faketensor"), ("test_faketensor",)
    ops = torch.ops.cinnamon_amd
    for col in (False, True):  # row-major and column-major scale outputs (same strides in the fake)
        torch.library.opcheck(ops.quant_rowwise.default, (x, 128, False, col), test_utils=f8)
        torch.library.opcheck(ops.quant_dual.default, (x, False, col), test_utils=f8)
    torch.library.opcheck(ops.quant_blockwise.default, (x, 128, 128, True), test_utils=f8)
    torch.library.opcheck(ops.quant_blockwise_t.default, (x.float(), False, False), test_utils=f8)
    q, s = kernels.quantize_fp8_rowwise(x)
    torch.library.opcheck(ops.requant_row_to_block.default, (q, s, True), test_utils=f8)
    q8 = q.view(torch.uint8)
    torch.library.opcheck(ops.dequant_rowwise.default, (q8, s, 128), test_utils=full)
    wq, ws = kernels.quantize_fp8_blockwise(x)
    wq8 = wq.view(torch.uint8)
    torch.library.opcheck(ops.dequant.default, (wq8, ws, 128, 128), test_utils=full)
    torch.library.opcheck(ops.gemm_fp8_bs.default, (q8, s, wq8, ws, torch.float32), test_utils=full)
    torch.library.opcheck(ops.transpose_u8.default, (q8,), test_utils=full)
    h12 = torch.randn(256, 512, device=dev, generator=g).to(torch.bfloat16)
    for col in (False, True):
        torch.library.opcheck(ops.silu_mul_quant_rowwise.default, (h12, torch.bfloat16, False, col),
                              test_utils=f8)
    dh = torch.randn(256, 256, device=dev, generator=g)
    torch.library.opcheck(ops.swiglu_backward.default, (dh, h12), test_utils=full)
    se = (torch.tensor([0, 100], device=dev), torch.tensor([100, 256], device=dev))
    for col in (False, True):
        torch.library.opcheck(ops.swiglu_dual_grouped.default, (dh, h12, *se, False, col), test_utils=f8)
    # indexer: quantization (fp8 outputs), scores and weights gradient (uint8 code inputs)
    qi = torch.randn(2, 70, 4, 128, device=dev, generator=g).to(torch.bfloat16)
    ki = torch.randn(2, 90, 128, device=dev, generator=g).to(torch.bfloat16)
    torch.library.opcheck(ops.indexer_quantize.default, (qi, ki), test_utils=f8)
    q8i, qsi, k8i, ksi = ops.indexer_quantize(qi, ki)
    wi = torch.randn(2, 70, 4, device=dev, generator=g)
    args = (q8i.view(torch.uint8), qsi, k8i.view(torch.uint8), ksi)
    torch.library.opcheck(ops.indexer_scores_fp8.default, (*args, wi, 0.125), test_utils=full)
    gsi = torch.randn(2, 70, 90, device=dev, generator=g)
    torch.library.opcheck(ops.indexer_weights_grad_fp8.default, (*args, gsi, 0.125), test_utils=full)
    torch.library.opcheck(ops.indexer_quantize_k.default, (ki, 4), test_utils=f8)
    for save in (True, False):
        torch.library.opcheck(ops.indexer_scores_fp8_q.default, (qi, args[2], ksi, wi, 0.125, save),
                              test_utils=f8)
