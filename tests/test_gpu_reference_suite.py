"""The reference's own FP8 kernel tests (reference tests/test_kernels.py:28-76, :158-182),
run against the drop-in module on the GPU: shapes, dtypes, round trip, outliers and
the row-wise quantizer throughput floor."""
import time

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_rowwise_shapes(kern, dev):
    x = torch.randn(256, 512, dtype=torch.bfloat16, device=dev)
    x_fp8, scales = kern.quantize_fp8_rowwise(x, block_size=128)
    assert x_fp8.shape == x.shape
    assert x_fp8.dtype == torch.float8_e4m3fn
    assert scales.shape == (256, 4)


def test_blockwise_shapes(kern, dev):
    w = torch.randn(512, 512, dtype=torch.bfloat16, device=dev)
    w_fp8, scales = kern.quantize_fp8_blockwise(w, block_m=128, block_n=128)
    assert w_fp8.shape == w.shape
    assert w_fp8.dtype == torch.float8_e4m3fn
    assert scales.shape == (4, 4)


def test_roundtrip_accuracy(kern, dev):
    x = torch.randn(256, 512, dtype=torch.bfloat16, device=dev)
    x_fp8, scales = kern.quantize_fp8_rowwise(x, block_size=128)
    x_rec = kern.dequantize_fp8(x_fp8, scales, block_m=1, block_n=128)
    rel_error = (x.float() - x_rec.float()).abs() / (x.float().abs() + 1e-6)
    assert rel_error.mean().item() < 0.1


def test_outlier_handling(kern, dev):
    x = torch.randn(256, 512, dtype=torch.bfloat16, device=dev)
    x[0, 0] = 1000.0
    x[100, 200] = -500.0
    x_fp8, scales = kern.quantize_fp8_rowwise(x, block_size=128)
    x_rec = kern.dequantize_fp8(x_fp8, scales, block_m=1, block_n=128)
    assert not torch.isnan(x_rec).any()
    assert not torch.isinf(x_rec).any()


def test_non_cuda_input_rejected_like_reference(kern):
    with pytest.raises(AssertionError):
        kern.quantize_fp8_rowwise(torch.randn(4, 128))
    with pytest.raises(AssertionError):
        kern.quantize_fp8_blockwise(torch.randn(4, 128, device="cuda")[0])


def test_rowwise_throughput_floor(kern, dev):
    x = torch.randn(2048, 2048, dtype=torch.bfloat16, device=dev)
    for _ in range(10):
        kern.quantize_fp8_rowwise(x)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(100):
        kern.quantize_fp8_rowwise(x)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / 100
    gbps = x.numel() * x.element_size() / dt / 1e9
    assert gbps > 10, f"{gbps:.1f} GB/s"
