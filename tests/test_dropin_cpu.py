"""Drop-in functions that run on CPU tensors, as the reference's plain-torch ones do."""
import pytest
import torch

from cinnamon_amd import kernels
from oracle import fp8_oracle as orc


@pytest.mark.parametrize("M,N,block", [(300, 520, 128), (7, 128, 128), (33, 1100, 64), (5, 250, 100)])
def test_dequantize_fp8_rowwise_on_cpu(M, N, block):
    """src/kernels.py:262-281 on CPU tensors: fp32(code) * scale of its tile, tails cut."""
    g = torch.Generator().manual_seed(M + N)
    x = (torch.randn(M, N, generator=g) * 3).to(torch.bfloat16)
    q, s = orc.quant_rowwise(x, block)
    got = kernels.dequantize_fp8_rowwise(q, s, block)
    assert got.dtype == torch.float32 and got.shape == (M, N) and got.device.type == "cpu"
    assert torch.equal(got, orc.dequant_rowwise(q, s, block))
    # every element is the code's value times its tile's scale, exactly
    col_tile = torch.arange(N) // block
    assert torch.equal(got, q.float() * s[:, col_tile])
