"""Device MoE dispatch / combine (GPU) against the oracle's restatement of the reference's
MoE.forward routing block (src/layers.py:126-157).

- Route: perm, counts, starts and ends equal the stable sort exactly; inv is perm's
  inverse.
- Gather-quantize: equals quantize_fp8_rowwise(x[token_indices]) bit for bit.
- Gather-sum and combine: equal the order-exact CPU restatement bit for bit (fp32 adds in
  increasing sorted position, the order of a sequential scatter_add_).
- Combine backward: the row gradient is exact; the score gradient (a 7168-term dot
  product) is within 1e-5 relative of fp64.
- routed_experts end to end: sorted expert outputs (stored in fp16, as the reference's
  fp16 expert GEMMs return them), routed output and weight gradients equal the unfused
  composition (route -> x[token_indices] -> GroupedExperts -> fp16 -> combine); dx and the
  score gradients agree within the stated tolerances.
"""
import pytest
import torch

from cinnamon_amd import kernels, layers, moe
from oracle import fp8_oracle as orc

pytestmark = pytest.mark.gpu


def _routing(T, k, E, seed, zipf=True):
    g = torch.Generator().manual_seed(seed)
    if zipf:
        p = torch.tensor([(e + 1) ** -1.1 for e in range(E)])
        top_idx = torch.multinomial(p.expand(T, E), k, replacement=False, generator=g)
    else:
        top_idx = torch.randint(0, E, (T, k), generator=g)
    scores = torch.rand(T, k, generator=g)
    scores = scores / scores.sum(-1, keepdim=True)
    return top_idx, scores


@pytest.mark.parametrize("T,k,E,zipf", [(16384, 8, 32, True), (1000, 2, 17, True), (77, 1, 5, False),
                                        (3000, 3, 300, False), (5, 4, 2, False)])
def test_route_is_the_stable_sort(dev, T, k, E, zipf):
    top_idx, _ = _routing(T, k, E, seed=T + k, zipf=zipf)
    perm, inv, counts, starts, ends = moe.moe_route(top_idx.to(dev), E)
    order, tok, rc, rs, re_ = orc.moe_dispatch_ref(top_idx, E)
    assert torch.equal(perm.cpu(), order)
    assert torch.equal(counts.cpu(), rc) and torch.equal(starts.cpu(), rs) and torch.equal(ends.cpu(), re_)
    pos = torch.empty(T * k, dtype=torch.int64)
    pos[order] = torch.arange(T * k)
    assert torch.equal(inv.cpu().long(), pos)


def test_route_drops_ids_outside_the_experts(dev):
    top_idx = torch.tensor([[0, 3], [5, 1], [-1, 3], [2, 7]])  # E = 4: 5, -1, 7 are dropped
    perm, inv, counts, starts, ends = moe.moe_route(top_idx.to(dev), 4)
    assert counts.tolist() == [1, 1, 1, 2] and ends.tolist() == [1, 2, 3, 5]
    assert perm.tolist() == [0, 3, 6, 1, 5, -1, -1, -1]
    assert inv.tolist() == [0, 3, -1, 1, -1, 4, 2, -1]


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 7168), (torch.float32, 1100), (torch.float16, 256)])
def test_gather_quantize_equals_quantize_of_gather(dev, dtype, D):
    T, k, E = 700, 4, 11
    top_idx, _ = _routing(T, k, E, seed=3)
    g = torch.Generator().manual_seed(4)
    x = (torch.randn(T, D, generator=g) * 3).to(dtype).to(dev)
    x[5, :300] = 0  # a zero tile
    perm, inv, *_ = moe.moe_route(top_idx.to(dev), E)
    rq, rs = kernels.quantize_fp8_rowwise(x[perm // k])
    for form in (None, inv):  # gather from the sorted side, scatter from the token side
        q, s = moe.moe_gather_quantize(x, perm, k, inv=form)
        assert torch.equal(q.view(torch.uint8), rq.view(torch.uint8)) and torch.equal(s, rs)
    # round_scale path and a strided x
    xs = torch.zeros(T, D + 64, dtype=dtype, device=dev)[:, :D]
    xs.copy_(x)
    rq2, rs2 = kernels.quantize_fp8_rowwise(x[perm // k], round_scale=True)
    for form in (None, inv):
        q2, s2 = moe.moe_gather_quantize(xs, perm, k, round_scale=True, inv=form)
        assert torch.equal(q2.view(torch.uint8), rq2.view(torch.uint8)) and torch.equal(s2, rs2)


def test_gather_quantize_dropped_rows_are_zero(dev):
    x = torch.randn(4, 256, device=dev).to(torch.bfloat16)
    top_idx = torch.tensor([[0, 9], [1, 0], [9, 9], [1, 1]], device=dev)  # 9 is dropped (E = 2)
    perm, inv, *_ = moe.moe_route(top_idx, 2)
    kept = int((perm >= 0).sum())
    assert kept == 5
    rq, rs = kernels.quantize_fp8_rowwise(x[perm[:kept] // 2])
    zq, zs = kernels.quantize_fp8_rowwise(torch.zeros(1, 256, dtype=x.dtype, device=dev))
    for form in (None, inv):
        q, s = moe.moe_gather_quantize(x, perm, 2, inv=form)
        assert torch.equal(q[:kept].view(torch.uint8), rq.view(torch.uint8)) and torch.equal(s[:kept], rs)
        assert int(q[kept:].view(torch.uint8).count_nonzero()) == 0
        assert torch.equal(s[kept:], zs.expand(len(perm) - kept, -1))


def _ordered_token_sums(rows, inv, T, k, weights=None):
    """CPU: out[t] = sum over t's sorted positions (increasing) of rows[r] (* weight), fp32."""
    out = torch.zeros(T, rows.shape[1])
    for t in range(T):
        terms = sorted((int(inv[t * k + j]), j) for j in range(k) if int(inv[t * k + j]) >= 0)
        for r, j in terms:
            term = rows[r] if weights is None else rows[r] * weights[t, j].float()
            out[t] = out[t] + term
    return out


@pytest.mark.parametrize("gdtype,odtype", [(torch.float32, torch.bfloat16), (torch.float32, torch.float32),
                                           (torch.bfloat16, torch.float32)])
def test_gather_sum_in_sorted_order(dev, gdtype, odtype):
    T, k, E, D = 300, 6, 13, 1030
    top_idx, _ = _routing(T, k, E, seed=5)
    perm, inv, *_ = moe.moe_route(top_idx.to(dev), E)
    g = torch.randn(T * k, D, generator=torch.Generator().manual_seed(6)).to(gdtype)
    out = moe.moe_gather_sum(g.to(dev), inv, k, odtype)
    want = _ordered_token_sums(g.float(), inv.cpu(), T, k).to(odtype)
    assert torch.equal(out.cpu(), want)


def _partial_routing(T, k, E, seed):
    """Uniform routing with every 7th token's first assignment outside the experts (dropped),
    so tokens have k or k - 1 rows."""
    top_idx, scores = _routing(T, k, E, seed=seed, zipf=False)
    top_idx[::7, 0] = E + 1
    return top_idx, scores


# Rows whose 16-byte pieces are aligned take the batched loads (up to 8 rows of a token at
# once): k not a multiple of 8, k above 8, dropped assignments, and a last column chunk
# that is partial (1032 = 64 x 16 + 8) or whole (1040).
@pytest.mark.parametrize("k,D,gdtype,odtype", [(6, 1032, torch.bfloat16, torch.float32),
                                               (12, 1040, torch.float32, torch.bfloat16),
                                               (3, 1032, torch.float16, torch.float32),
                                               (9, 1032, torch.float32, torch.float32)])
def test_gather_sum_batched_rows(dev, k, D, gdtype, odtype):
    T, E = 257, 11
    top_idx, _ = _partial_routing(T, k, E, seed=21 + k)
    perm, inv, *_ = moe.moe_route(top_idx.to(dev), E)
    g = torch.randn(T * k, D, generator=torch.Generator().manual_seed(22)).to(gdtype)
    out = moe.moe_gather_sum(g.to(dev), inv, k, odtype)
    want = _ordered_token_sums(g.float(), inv.cpu(), T, k).to(odtype)
    assert torch.equal(out.cpu(), want)


@pytest.mark.parametrize("k,D,ydtype", [(6, 1032, torch.float16), (12, 1032, torch.float32),
                                        (3, 1040, torch.bfloat16), (8, 1032, torch.float16)])
def test_combine_batched_rows(dev, k, D, ydtype):
    T, E = 257, 11
    top_idx, scores = _partial_routing(T, k, E, seed=31 + k)
    perm, inv, *_ = moe.moe_route(top_idx.to(dev), E)
    y = torch.randn(T * k, D, generator=torch.Generator().manual_seed(32)).to(ydtype)
    out = moe.moe_combine(y.to(dev), scores.to(dev), inv)
    want = _ordered_token_sums(y.float(), inv.cpu(), T, k, weights=scores)
    assert torch.equal(out.cpu(), want)


@pytest.mark.parametrize("sdtype,ydtype", [(torch.bfloat16, torch.float32), (torch.float32, torch.float32),
                                           (torch.float32, torch.float16), (torch.bfloat16, torch.float16)])
def test_combine_equals_reference_scatter_add(dev, sdtype, ydtype):
    T, k, E, D = 512, 8, 32, 7168
    top_idx, scores = _routing(T, k, E, seed=7)
    scores = scores.to(sdtype)
    y = torch.randn(T * k, D, generator=torch.Generator().manual_seed(8)).to(ydtype).float()
    perm, inv, *_ = moe.moe_route(top_idx.to(dev), E)
    out = moe.moe_combine(y.to(ydtype).to(dev), scores.to(dev), inv)
    order, *_ = orc.moe_dispatch_ref(top_idx, E)
    want = orc.moe_combine_ref(y, scores, order, T)
    assert torch.equal(out.cpu(), want)


@pytest.mark.parametrize("ydtype", [torch.float32, torch.float16])
def test_combine_backward(dev, ydtype):
    T, k, E, D = 256, 4, 10, 7168
    top_idx, scores = _routing(T, k, E, seed=9)
    scores = scores.to(torch.bfloat16)
    g = torch.Generator().manual_seed(10)
    y = torch.randn(T * k, D, generator=g).to(ydtype).float()
    dout = torch.randn(T, D, generator=g)
    perm, inv, *_ = moe.moe_route(top_idx.to(dev), E)
    dyd, _ = moe.moe_combine_backward(dout.to(dev), y.to(ydtype).to(dev), scores.to(dev), perm, inv)
    assert dyd.dtype == ydtype  # by default the gradient takes sorted_out's dtype
    dy, ds = moe.moe_combine_backward(dout.to(dev), y.to(ydtype).to(dev), scores.to(dev), perm, inv,
                                      dy_dtype=torch.float32 if ydtype == torch.float32 else torch.bfloat16)
    # the row gradient: RNE of the fp32 product, in fp32 for fp32 y and bf16 for 16-bit y
    assert dy.dtype == (torch.float32 if ydtype == torch.float32 else torch.bfloat16)
    # reference autograd of weighted_out = sorted_out * sorted_scores[:, None] + scatter_add_
    order, *_ = orc.moe_dispatch_ref(top_idx, E)
    yr = y.clone().requires_grad_(True)
    sr = scores.float().clone().requires_grad_(True)
    orc.moe_combine_ref(yr, sr, order, T).backward(dout)
    assert torch.equal(dy.cpu(), yr.grad.to(dy.dtype))
    dy16, _ = moe.moe_combine_backward(dout.to(dev), y.to(ydtype).to(dev), scores.to(dev), perm, inv,
                                       dy_dtype=torch.float16)
    assert dy16.dtype == torch.float16 and torch.equal(dy16.cpu(), yr.grad.half())
    assert torch.equal(dyd.cpu(), yr.grad.to(ydtype))
    exact = torch.zeros(T, k, dtype=torch.float64)
    pos = inv.cpu().long().view(T, k)
    for j in range(k):
        exact[:, j] = (dout.double() * y.double()[pos[:, j]]).sum(1)
    assert (ds.cpu().double() - exact).abs().max() <= 1e-5 * exact.abs().max()
    assert (sr.grad.double() - exact).abs().max() <= 1e-5 * exact.abs().max()


def test_combine_backward_keeps_tiny_gradients(dev):
    """dout ~ 1e-6 (a loss averaged over many tokens): the row gradients (~2e-7) are exact
    bf16 roundings of the fp32 products, none flushed; fp16 would hold them as subnormals
    with 1-3 significant bits."""
    T, k, E, D = 512, 8, 32, 2048
    top_idx, scores = _routing(T, k, E, seed=15)
    g = torch.Generator().manual_seed(16)
    y = torch.randn(T * k, D, generator=g).half()
    dout = torch.randn(T, D, generator=g) * 1e-6
    perm, inv, *_ = moe.moe_route(top_idx.to(dev), E)
    dy, _ = moe.moe_combine_backward(dout.to(dev), y.to(dev), scores.to(dev), perm, inv,
                                     dy_dtype=torch.bfloat16)
    assert dy.dtype == torch.bfloat16
    order, *_ = orc.moe_dispatch_ref(top_idx, E)
    exact = dout[order // k] * scores.reshape(-1)[order][:, None]      # fp32 products
    assert torch.equal(dy.cpu(), exact.bfloat16())
    assert int((dy.cpu() == 0).sum()) == int((exact == 0).sum())
    rel = ((dy.cpu().float() - exact).abs() / exact.abs().clamp_min(1e-30)).max().item()
    assert rel <= 2.0 ** -8
    rel16 = ((exact.half().float() - exact).abs() / exact.abs().clamp_min(1e-30)).max().item()
    assert rel16 > 0.1    # what an fp16 row gradient would have lost


class _HalfOutBf16Grad(torch.autograd.Function):
    """Forward: the value rounded to fp16 (the fused block's sorted outputs); backward: the
    gradient rounded to bf16 (the fused combine backward's row gradient)."""

    @staticmethod
    def forward(ctx, t):
        return t.half().float()

    @staticmethod
    def backward(ctx, g):
        return g.bfloat16().float()


@pytest.mark.parametrize("dout_scale", [1.0, 1e-6])
def test_routed_experts_equal_the_unfused_composition(dev, dout_scale):
    torch.manual_seed(11)
    T, k, E, D, H = 1024, 4, 8, 256, 256
    experts = layers.GroupedExperts(E, D, H).to(dev)
    top_idx, scores = _routing(T, k, E, seed=12)
    top_idx, scores = top_idx.to(dev), scores.to(torch.bfloat16).to(dev)
    x = torch.randn(T, D, generator=torch.Generator().manual_seed(13)).to(torch.bfloat16).to(dev)
    dout = (torch.randn(T, D, generator=torch.Generator().manual_seed(14)) * dout_scale).to(dev)

    # fused: route -> gather-quantize -> experts -> combine
    xf = x.clone().requires_grad_(True)
    sf = scores.clone().requires_grad_(True)
    out_f, counts = moe.routed_experts(experts, xf, top_idx, sf)
    out_f.backward(dout)
    gf = (xf.grad.clone(), experts.w12.grad.clone(), experts.w3.grad.clone(), sf.grad.clone())
    experts.w12.grad = experts.w3.grad = None

    # unfused: the reference's block with the same stable permutation
    perm, inv, c2, starts, ends = moe.moe_route(top_idx, E)
    assert torch.equal(counts, c2)
    xu = x.clone().requires_grad_(True)
    su = scores.clone().requires_grad_(True)
    sorted_x = xu[perm // k]
    sorted_out = _HalfOutBf16Grad.apply(experts(sorted_x, starts, ends))
    sorted_scores = su.reshape(-1)[perm]
    weighted = sorted_out * sorted_scores[:, None]
    out_u = torch.zeros(T, D, device=dev, dtype=weighted.dtype)
    out_u.scatter_add_(0, (perm // k).unsqueeze(1).expand_as(weighted), weighted)
    out_u.backward(dout)

    # sorted expert outputs are bit-identical (same codes, same GEMMs); the fused combine
    # adds in sorted order while the GPU scatter_add_ uses atomics
    assert (out_f - out_u).abs().max() <= 1e-5 * out_u.abs().max()
    assert torch.equal(gf[1], experts.w12.grad) and torch.equal(gf[2], experts.w3.grad)
    # dx: fp32 sum of the k row gradients then one rounding, against k bf16 roundings
    assert (gf[0].float() - xu.grad.float()).abs().max() <= 2e-2 * xu.grad.float().abs().max()
    assert orc.frob_rel(gf[0].float().cpu(), xu.grad.float().cpu()) <= 5e-3
    assert (gf[3].float() - su.grad.float()).abs().max() <= 1e-2 * su.grad.float().abs().max()


class _HalfOutGrad(torch.autograd.Function):
    """Forward: the value rounded to fp16; backward: the gradient rounded to grad_dtype."""

    @staticmethod
    def forward(ctx, t, grad_dtype):
        ctx.grad_dtype = grad_dtype
        return t.half().float()

    @staticmethod
    def backward(ctx, g):
        return g.to(ctx.grad_dtype).float(), None


def test_routed_experts_tiny_gradients_against_an_fp32_chain(dev):
    """With dout ~ 1e-6 the expert weight gradients of the fused block stay close to those of
    a chain that keeps the row gradient in fp32; rounding it to fp16 instead (what the
    sorted outputs' own dtype would give) moves them several times further."""
    torch.manual_seed(17)
    T, k, E, D, H = 1024, 4, 8, 256, 256
    experts = layers.GroupedExperts(E, D, H).to(dev)
    top_idx, scores = _routing(T, k, E, seed=18)
    top_idx, scores = top_idx.to(dev), scores.to(torch.bfloat16).to(dev)
    x = torch.randn(T, D, generator=torch.Generator().manual_seed(19)).to(torch.bfloat16).to(dev)
    dout = (torch.randn(T, D, generator=torch.Generator().manual_seed(20)) * 1e-6).to(dev)
    out_f, _ = moe.routed_experts(experts, x, top_idx, scores)
    out_f.backward(dout)
    fused = (experts.w12.grad.clone(), experts.w3.grad.clone())
    perm, inv, _, starts, ends = moe.moe_route(top_idx, E)
    chains = {}
    for gdt in (torch.float32, torch.float16):
        experts.w12.grad = experts.w3.grad = None
        sorted_out = _HalfOutGrad.apply(experts(x[perm // k], starts, ends), gdt)
        weighted = sorted_out * scores.reshape(-1)[perm][:, None]
        out = torch.zeros(T, D, device=dev).scatter_add_(0, (perm // k).unsqueeze(1).expand_as(weighted), weighted)
        out.backward(dout)
        chains[gdt] = (experts.w12.grad.clone(), experts.w3.grad.clone())
    errs = {}
    for i, name in enumerate(("w12", "w3")):
        ref = chains[torch.float32][i].cpu()
        errs[name] = (orc.frob_rel(fused[i].cpu(), ref), orc.frob_rel(chains[torch.float16][i].cpu(), ref))
        print(f"d{name}: fused (bf16 row gradient) {errs[name][0]:.3e}, fp16 row gradient {errs[name][1]:.3e}")
    # The gradients are ~2e-7, below the 1e-4 amax floor, so the FP8 codes sit in e4m3's
    # subnormal range where a perturbation of the input flips codes often: even bf16
    # rounding of the row gradient moves dW12 by ~2.4% (measured), fp16 by ~8.4%.
    for name, (e_fused, e_f16) in errs.items():
        assert e_fused <= 4e-2, name
        assert e_f16 >= 2.5 * e_fused, name
