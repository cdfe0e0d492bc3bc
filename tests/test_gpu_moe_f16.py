"""GPU parity of the unquantized grouped GEMM drop-in (moe_grouped_gemm).

The reference kernel rounds both operands to fp16, sums in fp32 and stores fp16
(src/kernels.py:440-523).  The oracle sums the fp16-rounded operands exactly (fp64), so
the device result may differ from it by the fp32 summation error plus the fp16 store:
normwise max relative error <= 1e-3 (the fp16 step is 2^-11 relative).
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import fp8_oracle as orc

pytestmark = pytest.mark.gpu


def test_reference_equivalence(kern, dev):
    """The reference's own test (tests/test_kernels.py:131-155), same shapes and bound."""
    n_experts, d_model, hidden_dim, total_tokens = 8, 512, 128, 256
    g = torch.Generator().manual_seed(0)
    weights = torch.randn(n_experts, hidden_dim, d_model, generator=g).to(torch.bfloat16)
    sorted_x = torch.randn(total_tokens, d_model, generator=g).to(torch.bfloat16)
    per = total_tokens // n_experts
    starts = torch.arange(0, total_tokens, per)[:n_experts]
    ends = torch.cat([starts[1:], torch.tensor([total_tokens])])
    out = kern.moe_grouped_gemm(sorted_x.to(dev), weights.to(dev), starts.to(dev), ends.to(dev))
    assert out.shape == (total_tokens, hidden_dim) and out.dtype == torch.float16
    ref = torch.zeros(total_tokens, hidden_dim)
    for i in range(n_experts):
        s, t = int(starts[i]), int(ends[i])
        ref[s:t] = F.linear(sorted_x[s:t].float(), weights[i].float())
    rel = (ref - out.float().cpu()).abs() / (ref.abs() + 1e-6)
    assert rel.mean().item() < 0.01


@pytest.mark.parametrize("xdt,wdt", [(torch.bfloat16, torch.float32), (torch.float16, torch.float16),
                                     (torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("N,K", [(384, 512), (100, 200)])
def test_grouped_f16_parity(kern, dev, xdt, wdt, N, K):
    counts = [300, 0, 128, 1, 555, 64, 0, 1000]
    ends = torch.tensor(counts).cumsum(0)
    starts = ends - torch.tensor(counts)
    T, E = int(ends[-1]), len(counts)
    g = torch.Generator().manual_seed(N + K)
    x = torch.randn(T, K, generator=g).to(xdt)
    w = (torch.randn(E, N, K, generator=g) * 0.05).to(wdt)
    out = kern.moe_grouped_gemm(x.to(dev), w.to(dev), starts.to(dev), ends.to(dev)).float().cpu()
    ref = orc.grouped_gemm_f16_ref(x, w, starts, ends)
    inside = torch.zeros(T, dtype=torch.bool)
    for _, s, t in orc.expert_slices(starts, ends, T):
        inside[s:t] = True
    got, want = out[inside].double(), ref[inside]
    assert (got - want).abs().max() / want.abs().max() <= 1e-3
