"""CPU checks of the grouped (MoE) backward oracle.

The reference has no FP8 or backward grouped path, so the oracle applies the dense
FP8MatmulFunction.backward recipe (src/kernels.py:763-794) per expert slice.  It is pinned
here by (1) one expert covering every row reducing exactly to the dense chain
(fp8_linear_ref, itself pinned in test_oracle.py), (2) the padded-axis bookkeeping on known
answers, and (3) the full FP8 SwiGLU-experts forward/backward staying within FP8 error of
an unquantized fp32 autograd computation (catches a wrong silu derivative, a transposed
operand or a swapped expert).
"""
import torch

from oracle import fp8_oracle as orc


def _case(T, D, H, E, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, D, generator=g).to(torch.bfloat16)
    w12 = torch.randn(E, 2 * H, D, generator=g) * 0.02
    w3 = torch.randn(E, D, H, generator=g) * 0.02
    dy = torch.randn(T, D, generator=g) * 1e-3
    return x, w12, w3, dy


def test_padded_offsets_known_answer():
    starts = [0, 300, 300, 301, 500]
    ends = [300, 300, 301, 500, 500]
    assert orc.padded_offsets(starts, ends, 500) == [(0, 3), (384, 0), (384, 1), (512, 2), (768, 0)]
    # ranges are clamped to [0, T)
    assert orc.expert_slices([-5, 10], [10, 99], 50) == [(0, 0, 10), (1, 10, 50)]


def test_single_expert_is_the_dense_chain():
    T, N, K = 384, 256, 256
    g = torch.Generator().manual_seed(1)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16)
    w = torch.randn(N, K, generator=g) * 0.02
    dy = (torch.randn(T, N, generator=g) * 1e-3).to(torch.bfloat16)
    dense = orc.fp8_linear_ref(x, w, dy)
    starts, ends = [0], [T]
    dual = orc.grouped_dual_ref(dy, starts, ends)
    rq, rs, tq, ts = dual[0]
    assert torch.equal(rq.view(torch.uint8), dense["g_fp8"].view(torch.uint8))
    assert torch.equal(tq.view(torch.uint8), dense["g_fp8_t"].view(torch.uint8))
    assert torch.equal(rs, dense["g_scale"]) and torch.equal(ts, dense["g_scale_t"])
    req = orc.grouped_requant_ref(dense["x_fp8"], dense["x_scale"], starts, ends)
    assert torch.equal(req[0][0].view(torch.uint8), dense["xb_fp8"].view(torch.uint8))
    assert torch.equal(req[0][1], dense["xb_scale"])
    dw = orc.grouped_wgrad_ref(dual, req, 1, N, K)
    assert torch.equal(dw[0], dense["dw"])
    wq = dense["w_fp8"].view(torch.uint8)[None]
    dx = orc.grouped_dgrad_ref(rq, rs, wq, dense["w_scale"][None], starts, ends)
    assert torch.equal(dx, dense["dx"])


def test_experts_are_independent_slices():
    """Splitting the rows between experts with identical weights changes only which
    tokens share a quantization chunk, never the dgrad rows of a single-expert run."""
    T, D, H = 256, 256, 256
    x, w12, w3, dy = _case(T, D, H, 1, seed=2)
    one = orc.grouped_experts_ref(x, w12, w3, [0], [T], dy)
    two = orc.grouped_experts_ref(x, w12.repeat(2, 1, 1), w3.repeat(2, 1, 1), [0, 128], [128, T], dy)
    # the forward quantizes rows independently of the expert split
    assert torch.equal(one["out"], two["out"])
    # with 128-aligned boundaries the per-expert chunks are the dense chunks, so the two
    # experts' weight gradients add up to the single expert's (up to fp32 summation order)
    assert orc.normwise_max_rel(two["dw3"].sum(0), one["dw3"][0]) < 1e-6
    assert orc.normwise_max_rel(two["dw12"].sum(0), one["dw12"][0]) < 1e-6


def _autograd_experts(x, w12, w3, starts, ends, dy):
    T, D = x.shape
    H = w3.shape[2]
    xf = x.float().requires_grad_(True)
    a, b = w12.clone().requires_grad_(True), w3.clone().requires_grad_(True)
    out = torch.zeros(T, D)
    for e, s, t in orc.expert_slices(starts, ends, T):
        if t > s:
            h12 = xf[s:t] @ a[e].t()
            h = torch.nn.functional.silu(h12[:, :H]) * h12[:, H:]
            out = out.index_copy(0, torch.arange(s, t), h @ b[e].t())
    out.backward(dy)
    return {"out": out.detach(), "dx": xf.grad, "dw12": a.grad, "dw3": b.grad}


def test_unquantized_experts_are_fp32_autograd():
    """With every quantization switched off, the oracle's composition (slices, transposes,
    silu derivative, expert routing of each gradient) must reproduce autograd."""
    T, D, H, E = 400, 256, 256, 3
    x, w12, w3, dy = _case(T, D, H, E, seed=3)
    x = x.float()
    starts, ends = [0, 150, 150], [150, 150, T]
    r = orc.grouped_experts_ref(x, w12, w3, starts, ends, dy, quantize=False)
    want = _autograd_experts(x, w12, w3, starts, ends, dy)
    for name in ("out", "dx", "dw12", "dw3"):
        assert orc.normwise_max_rel(r[name], want[name]) < 1e-5, name


def test_fp8_experts_within_fp8_error_of_fp32():
    T, D, H, E = 400, 256, 256, 3
    x, w12, w3, dy = _case(T, D, H, E, seed=3)
    starts, ends = [0, 150, 150], [150, 150, T]
    r = orc.grouped_experts_ref(x, w12, w3, starts, ends, dy)
    want = _autograd_experts(x, w12, w3, starts, ends, dy)
    for name in ("out", "dx", "dw12", "dw3"):
        # two chained e4m3 GEMMs: ~7% Frobenius error is the FP8 rounding itself
        assert orc.frob_rel(r[name], want[name]) < 0.1, name
    assert torch.count_nonzero(r["dw12"][1]) == 0 and torch.count_nonzero(r["dw3"][1]) == 0
