"""FP8 indexer scores (GPU) against the oracle's restatement of the reference's FP8 branch
of DSAIndexer.forward (src/attention.py:288-300).

The codes and scales come from the row-wise quantizer (bit-exact with the oracle, checked
in test_gpu_quant.py), so the scores differ from the oracle only in the code dot products.
Each product of two e4m3 codes is exact in fp32, and the oracle's fp32 einsum is within
1e-7 (normwise) of an exact fp64 evaluation on these inputs. The kernel sums the products
with v_mfma_f32_16x16x32_fp8_fp8, whose 32-product sum inside one instruction is not an
exact fp32 sum: measured at 2.2e-5 of the largest score on the first case. Tolerance: max
|error| <= 1e-4 * max |reference| (normwise) and Frobenius relative error <= 2e-5. These
are 20x and 50x tighter than the FP8 GEMM bar (2e-3 and 1e-3).
"""
import pytest
import torch

from cinnamon_amd import kernels
from oracle import fp8_oracle as orc

pytestmark = pytest.mark.gpu


def _inputs(B, L, S, H, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, L, H, d, generator=g).to(dtype)
    k = torch.randn(B, S, d, generator=g).to(dtype)
    w = torch.randn(B, L, H, generator=g) * H ** -0.5
    return q, k, w


def _check(got, want):
    assert got.shape == want.shape and got.dtype == torch.float32
    normwise = float((got - want).abs().max() / want.abs().max())
    frob = orc.frob_rel(got, want)
    print(f"normwise {normwise:.3g} frobenius {frob:.3g}")
    assert normwise <= 1e-4 and frob <= 2e-5


@pytest.mark.parametrize("B,L,S,H,d,dtype", [
    (2, 1024, 1024, 4, 128, torch.bfloat16),   # the indexer with PoPE (d_rope 64 -> 128)
    (3, 512, 512, 4, 64, torch.bfloat16),      # RoPE, d_indexer_head 64
    (1, 77, 130, 3, 192, torch.float32),       # ragged tiles, two 1x128 tiles per row
    (2, 65, 63, 1, 32, torch.float16),
    (1, 200, 64, 8, 256, torch.bfloat16),
])
def test_scores_match_the_oracle(dev, B, L, S, H, d, dtype):
    q, k, w = _inputs(B, L, S, H, d, dtype, seed=B * 1000 + L + d)
    scale = d ** -0.5
    got = kernels.indexer_scores_fp8(q.to(dev), k.to(dev), w.to(dev), scale).cpu()
    _check(got, orc.indexer_scores_fp8_ref(q, k, w, scale))


def test_zero_rows_and_negative_weights(dev):
    q, k, w = _inputs(2, 100, 96, 4, 64, torch.bfloat16, seed=7)
    q[0, 3] = 0          # all heads of one query: zero row -> floor scale, zero scores
    k[1, 10:20] = 0      # zero keys
    w[:, :, 1] *= -1     # the reference's weights are a signed projection
    got = kernels.indexer_scores_fp8(q.to(dev), k.to(dev), w.to(dev), 0.125).cpu()
    want = orc.indexer_scores_fp8_ref(q, k, w, 0.125)
    _check(got, want)
    assert torch.equal(got[0, 3], torch.zeros(96)) and torch.equal(got[1, :, 10:20], torch.zeros(100, 10))


def test_rejects_unsupported_head_dims(dev):
    q = torch.randn(1, 8, 2, 48, device=dev)
    k = torch.randn(1, 8, 48, device=dev)
    w = torch.randn(1, 8, 2, device=dev)
    with pytest.raises(AssertionError):
        kernels.indexer_scores_fp8(q, k, w, 0.1)
