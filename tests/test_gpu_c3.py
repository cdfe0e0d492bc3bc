"""Config 3 on the GPU: the FP8 grouped GEMMs at the workload of the reference's MoE
(src/layers.py:126-157, src/kernels.py:440-581): 32 experts, d_model 7168, expert hidden
2048, 16384 tokens routed top-8 (131072 sorted rows), expert loads from a Zipf(1.1)
draw without replacement (seed 3), so the ranges are ragged (about 1.3K to 15.8K rows).

At this size the kernels run their long K loops (56 blocks for gate/up, 32 and 56 for the
dgrads, up to 124 for the wgrad's largest expert), which take the XCD-rotated K order,
and every expert has a partial 256-row tile.  The CPU oracle checks:
  * gate/up, down and both dgrads on sampled rows of every expert (first and last row of
    its range, three rows of its partial tile, four random rows), with the GEMM tolerance
    (normwise max relative 2e-3, Frobenius 1e-3, fp32 output);
  * the gate/up and down wgrads of the largest and the smallest expert in full;
  * the sampled rows' operand codes and scales bit-exactly.
Full-size properties: bf16 and fp16 outputs equal the RNE of the fp32 output, and rows
outside every range keep what the output buffer held.

Large inputs come from a seeded CUDA generator; the oracle reads CPU copies of the same
bits.
"""
import pytest
import torch

from cinnamon_amd import layers, moe
from oracle import fp8_oracle as orc

pytestmark = pytest.mark.gpu

E, D, H, T, TOPK = 32, 7168, 2048, 16384, 8
A = T * TOPK
MAX_REL, FROB_REL = 2e-3, 1e-3


def _check(got, want, what):
    mr = orc.normwise_max_rel(got.float().cpu(), want)
    fr = orc.frob_rel(got.float().cpu(), want)
    print(f"{what}: normwise {mr:.2e} frob {fr:.2e}")
    assert mr <= MAX_REL and fr <= FROB_REL, f"{what}: normwise max rel {mr:.3e}, frob rel {fr:.3e}"


def _sample_rows(starts, ends, seed):
    """Per expert: sorted-row indices to check."""
    g = torch.Generator().manual_seed(seed)
    rows = []
    for e in range(E):
        s, t = int(starts[e]), int(ends[e])
        m = t - s
        if m == 0:
            rows.append(torch.empty(0, dtype=torch.int64))
            continue
        tail0 = s + 256 * ((m - 1) // 256)               # the expert's last (partial) 256-row tile
        pick = {s, t - 1, tail0, (tail0 + t - 1) // 2, t - 1}
        pick.update((s + torch.randint(0, m, (4,), generator=g)).tolist())
        rows.append(torch.tensor(sorted(pick), dtype=torch.int64))
    return rows


@pytest.fixture(scope="module")
def c3(kern, dev):
    g = torch.Generator().manual_seed(3)
    p = torch.tensor([(e + 1) ** -1.1 for e in range(E)])
    top_idx = torch.multinomial(p.expand(T, E), TOPK, replacement=False, generator=g)
    gd = torch.Generator(device=dev).manual_seed(3)
    x_tok = torch.randn(T, D, generator=gd, device=dev).to(torch.bfloat16)
    w12 = (torch.randn(E * 2 * H, D, generator=gd, device=dev) * 0.02).to(torch.bfloat16)
    w3 = (torch.randn(E * D, H, generator=gd, device=dev) * 0.02).to(torch.bfloat16)
    h = torch.randn(A, H, generator=gd, device=dev).to(torch.bfloat16)
    dh12 = (torch.randn(A, 2 * H, generator=gd, device=dev) * 1e-3).to(torch.bfloat16)
    dy = (torch.randn(A, D, generator=gd, device=dev) * 1e-3).to(torch.bfloat16)

    perm, inv, counts, starts, ends = moe.moe_route(top_idx.to(dev), E)
    xq, xs = moe.moe_gather_quantize(x_tok, perm, TOPK, inv=inv)
    hq, hs = kern.quantize_fp8_rowwise(h)
    w12q, w12qt, w12s = kern.quantize_fp8_blockwise_t(w12)
    w3q, w3qt, w3s = kern.quantize_fp8_blockwise_t(w3)
    torch.cuda.synchronize()
    c = dict(top_idx=top_idx, x_tok=x_tok, perm=perm, inv=inv, counts=counts, starts=starts, ends=ends,
             xq=xq, xs=xs, h=h, hq=hq, hs=hs, dh12=dh12, dy=dy,
             w12q=w12q.view(E, 2 * H, D), w12qt=w12qt, w12s=w12s.view(E, 2 * H // 128, D // 128),
             w3q=w3q.view(E, D, H), w3qt=w3qt, w3s=w3s.view(E, D // 128, H // 128))
    c["s_cpu"], c["e_cpu"] = starts.cpu(), ends.cpu()
    c["rows"] = _sample_rows(c["s_cpu"], c["e_cpu"], seed=30)
    c["w12q_cpu"] = c["w12q"].view(torch.uint8).cpu()
    c["w12s_cpu"] = c["w12s"].cpu()
    c["w3q_cpu"] = c["w3q"].view(torch.uint8).cpu()
    c["w3s_cpu"] = c["w3s"].cpu()
    m = (c["e_cpu"] - c["s_cpu"])
    print(f"C3 expert rows: max {int(m.max())} min {int(m.min())} total {int(m.sum())}")
    return c


def _rows_cat(c):
    return torch.cat(c["rows"])


def test_c3_route_and_dispatch_codes(c3):
    order, tok, rc, rs, re_ = orc.moe_dispatch_ref(c3["top_idx"], E)
    assert torch.equal(c3["counts"].cpu(), rc) and torch.equal(c3["s_cpu"], rs) and torch.equal(c3["e_cpu"], re_)
    assert int(rc.sum()) == A and int(rc.max()) > 10000 and int(rc.min()) > 0
    r = _rows_cat(c3)
    want_q, want_s = orc.quant_rowwise(c3["x_tok"].cpu()[order[r] // TOPK])
    assert torch.equal(c3["xq"].view(torch.uint8)[r.to(c3["xq"].device)].cpu(), want_q.view(torch.uint8))
    assert torch.equal(c3["xs"][r.to(c3["xs"].device)].cpu(), want_s)


def _grouped_rows_ref(c, a_q, a_s, w_q_cpu, w_s_cpu, transpose_w):
    """Oracle of the sampled rows: per expert, dequantize-then-fp32 matmul with W_e^T (forward)
    or W_e (dgrad)."""
    outs = []
    for e in range(E):
        r = c["rows"][e]
        if r.numel() == 0:
            continue
        rd = r.to(a_q.device)
        aq = a_q.view(torch.uint8)[rd].cpu()
        as_ = a_s[rd].cpu()
        wq, ws = w_q_cpu[e], w_s_cpu[e]
        if transpose_w:
            wq, ws = wq.t().contiguous(), ws.t().contiguous()
        outs.append(orc.gemm_ref(aq, as_, wq, ws))
    return torch.cat(outs)


def test_c3_gate_up(c3):
    c = c3
    args = (c["xq"], c["xs"], c["w12q"], c["w12s"], c["starts"], c["ends"])
    y32 = layers.fp8_grouped_gemm(*args, out_dtype=torch.float32)
    r = _rows_cat(c).to(y32.device)
    want = _grouped_rows_ref(c, c["xq"], c["xs"], c["w12q_cpu"], c["w12s_cpu"], transpose_w=True)
    _check(y32[r], want, "gate/up sampled rows")
    y16 = layers.fp8_grouped_gemm(*args, out_dtype=torch.bfloat16)
    assert torch.equal(y16, y32.to(torch.bfloat16)), "bf16 output is not RNE(fp32)"


def test_c3_rows_outside_every_range_are_untouched(c3):
    """Cut 100 rows off the end of expert 5's range and 37 off the start of expert 20's:
    those rows keep the buffer's NaN; every other row matches the full-range run."""
    c = c3
    starts, ends = c["starts"].clone(), c["ends"].clone()
    ends[5] -= 100
    starts[20] += 37
    full = layers.fp8_grouped_gemm(c["xq"], c["xs"], c["w12q"], c["w12s"], c["starts"], c["ends"],
                                   out_dtype=torch.float32)
    out = torch.full((A, 2 * H), float("nan"), device=full.device)
    layers.fp8_grouped_gemm(c["xq"], c["xs"], c["w12q"], c["w12s"], starts, ends, out=out)
    gap = torch.zeros(A, dtype=torch.bool, device=full.device)
    gap[int(ends[5]):int(c["ends"][5])] = True
    gap[int(c["starts"][20]):int(starts[20])] = True
    assert bool(torch.isnan(out[gap]).all())
    kept = out[~gap]
    assert bool(torch.isfinite(kept).all())
    # the same rows, possibly summed in another K order (tile -> XCD mapping moved)
    assert ((kept - full[~gap]).abs().max() <= 1e-5 * full.abs().max()).item()


def test_c3_down(c3):
    c = c3
    args = (c["hq"], c["hs"], c["w3q"], c["w3s"], c["starts"], c["ends"])
    y32 = layers.fp8_grouped_gemm(*args, out_dtype=torch.float32)
    r = _rows_cat(c)
    want_q, want_s = orc.quant_rowwise(c["h"][r.to(c["h"].device)].cpu())
    assert torch.equal(c["hq"].view(torch.uint8)[r.to(c["hq"].device)].cpu(), want_q.view(torch.uint8))
    want = _grouped_rows_ref(c, c["hq"], c["hs"], c["w3q_cpu"], c["w3s_cpu"], transpose_w=True)
    _check(y32[r.to(y32.device)], want, "down sampled rows")
    y16 = layers.fp8_grouped_gemm(*args, out_dtype=torch.float16)
    assert torch.equal(y16, y32.half()), "fp16 output is not RNE(fp32)"


@pytest.mark.parametrize("which", ["gate_up", "down"])
def test_c3_dgrad(c3, which):
    """dX = dC . W_e per expert (gate/up: dC [A, 4096] -> [A, 7168], 32 K blocks; down:
    dC [A, 7168] -> [A, 2048], 56 K blocks)."""
    c = c3
    if which == "gate_up":
        grad, wqt, ws, w_cpu, ws_cpu, n_red = c["dh12"], c["w12qt"], c["w12s"], c["w12q_cpu"], c["w12s_cpu"], 2 * H
    else:
        grad, wqt, ws, w_cpu, ws_cpu, n_red = c["dy"], c["w3qt"], c["w3s"], c["w3q_cpu"], c["w3s_cpu"], D
    q, s, _, _ = layers.quantize_fp8_dual_grouped(grad, c["starts"], c["ends"])
    r = _rows_cat(c)
    rd = r.to(grad.device)
    want_q, want_s = orc.quant_rowwise(grad[rd].cpu())
    assert torch.equal(q.view(torch.uint8)[rd].cpu(), want_q.view(torch.uint8))
    assert torch.equal(s[rd].cpu(), want_s)
    dx = layers.fp8_grouped_dgrad(q, s, wqt, ws.reshape(-1, ws.shape[-1]), c["starts"], c["ends"], n_red,
                                  out_dtype=torch.float32)
    want = _grouped_rows_ref(c, q, s, w_cpu, ws_cpu, transpose_w=False)
    _check(dx[rd], want, f"{which} dgrad sampled rows")


@pytest.mark.parametrize("which", ["gate_up", "down"])
def test_c3_wgrad_largest_and_smallest_expert(c3, which):
    """dW_e = dC_e^T . X_e over each expert's tokens (the reduction runs over up to 15.8K
    tokens: 124 K blocks), the largest and the smallest expert compared in full."""
    c = c3
    if which == "gate_up":
        grad, xq, xs, N, K = c["dh12"], c["xq"], c["xs"], 2 * H, D
    else:
        grad, xq, xs, N, K = c["dy"], c["hq"], c["hs"], D, H
    _, _, qt, st = layers.quantize_fp8_dual_grouped(grad, c["starts"], c["ends"])
    xbt, xblk = layers.requantize_grouped_t(xq, xs, c["starts"], c["ends"])
    dw = layers.fp8_grouped_wgrad(qt, st, xbt, xblk, c["starts"], c["ends"], A)
    assert dw.shape == (E, N, K)
    m = c["e_cpu"] - c["s_cpu"]
    for e in (int(m.argmax()), int(m.argmin())):
        s, t = int(c["s_cpu"][e]), int(c["e_cpu"][e])
        one = torch.tensor([0]), torch.tensor([t - s])
        dual = orc.grouped_dual_ref(grad[s:t].cpu(), *one)
        req = orc.grouped_requant_ref(xq[s:t].cpu(), xs[s:t].cpu(), *one)
        want = orc.grouped_wgrad_ref(dual, req, 1, N, K)[0]
        _check(dw[e], want, f"{which} wgrad expert {e} ({t - s} tokens)")
