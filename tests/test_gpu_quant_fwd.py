"""GPU parity of the one-launch forward quantizer (cin_quant_fwd): X in 1 x 128 row tiles
and the weight in 128 x 128 blocks, bit-identical to quantize_fp8_rowwise(x, 128,
round_scale) and quantize_fp8_blockwise(weight.float()) (reference src/kernels.py:746-747),
and to the CPU oracle.

The fused launch takes K % 128 == 0 with a 16-bit weight; every other shape and dtype goes
through the entry point's two-launch path, which the same assertions cover.
"""
import pytest
import torch

from oracle import fp8_oracle as orc

from tests.test_gpu_quant import _activations, _assert_codes_equal, _assert_scales_equal, _special_matrix

pytestmark = pytest.mark.gpu

DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _check(kern, dev, x, w, rs, with_rowmajor=True, with_transposed=True, oracle=True):
    xd, wd = x.to(dev), w.to(dev)
    xq, xs, wq, wqt, ws = kern.quantize_fp8_forward(xd, wd, rs, with_rowmajor=with_rowmajor,
                                                     with_transposed=with_transposed)
    assert (wq is None) != with_rowmajor and (wqt is None) != with_transposed
    # the separate quantizers, as the reference forward calls them
    rq, rsx = kern.quantize_fp8_rowwise(xd, 128, rs)
    bq, bqt, bs = kern.quantize_fp8_blockwise_t(wd.float())
    _assert_codes_equal(xq, rq.cpu(), "x codes vs quantize_fp8_rowwise")
    _assert_scales_equal(xs, rsx.cpu(), "x scales vs quantize_fp8_rowwise")
    if with_rowmajor:
        _assert_codes_equal(wq, bq.cpu(), "w codes vs quantize_fp8_blockwise")
    if with_transposed:
        _assert_codes_equal(wqt, bqt.cpu(), "transposed w codes vs quantize_fp8_blockwise_t")
    _assert_scales_equal(ws, bs.cpu(), "w scales vs quantize_fp8_blockwise")
    if oracle:
        oq, osx = orc.quant_rowwise(x, 128, rs)
        owq, ows = orc.quant_blockwise(w.float())
        _assert_codes_equal(xq, oq, "x codes vs oracle")
        _assert_scales_equal(xs, osx, "x scales vs oracle")
        _assert_codes_equal(wq if with_rowmajor else wqt.t(), owq, "w codes vs oracle")
        _assert_scales_equal(ws, ows, "w scales vs oracle")


@pytest.mark.parametrize("xdt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("wdt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("rs", [False, True])
def test_quant_fwd_dtypes(kern, dev, xdt, wdt, rs):
    # (M, K, N) = (300, 1024, 260): ragged M and N, whole K tiles -> fused for 16-bit weights
    x = _activations(300, 1024, seed=11, dtype=DT[xdt])
    w = _activations(260, 1024, seed=12, dtype=DT[wdt], outliers=False, std=0.02)
    _check(kern, dev, x, w, rs)


@pytest.mark.parametrize("layout", [(True, False), (False, True), (True, True)])
def test_quant_fwd_weight_layouts(kern, dev, layout):
    x = _activations(129, 512, seed=13)
    w = _activations(384, 512, seed=14, outliers=False, std=0.02)
    _check(kern, dev, x, w, False, *layout)


@pytest.mark.parametrize("M,K,N", [(1, 128, 1), (70, 200, 130), (3, 1000, 5), (256, 384, 128)])
def test_quant_fwd_shapes(kern, dev, M, K, N):
    # K % 128 != 0 takes the two-launch path; the others run fused
    _check(kern, dev, _activations(M, K, seed=15), _activations(N, K, seed=16, std=0.02), False)


def test_quant_fwd_special_values(kern, dev):
    # zero tiles (floored scale), -0, NaN, Inf and tiny values in both operands
    x = _special_matrix(300, 512, torch.bfloat16, seed=17)
    w = _special_matrix(260, 512, torch.bfloat16, seed=18)
    _check(kern, dev, x, w, False)
    _check(kern, dev, x, w, True)


def test_quant_fwd_strided_rows(kern, dev):
    # rows of X and W taken from wider buffers (row stride > K)
    xb = _activations(200, 640, seed=19).to(dev)
    wb = _activations(300, 768, seed=20, std=0.02).to(dev)
    x, w = xb[:, 64:576], wb[:, 128:640]
    xq, xs, wq, wqt, ws = kern.quantize_fp8_forward(x, w, with_transposed=True)
    rq, rsx = kern.quantize_fp8_rowwise(x.contiguous(), 128)
    bq, bqt, bs = kern.quantize_fp8_blockwise_t(w.contiguous().float())
    _assert_codes_equal(xq, rq.cpu(), "x codes")
    _assert_scales_equal(xs, rsx.cpu(), "x scales")
    _assert_codes_equal(wq, bq.cpu(), "w codes")
    _assert_codes_equal(wqt, bqt.cpu(), "transposed w codes")
    _assert_scales_equal(ws, bs.cpu(), "w scales")


def test_quant_fwd_config2(kern, dev):
    # the config-2 step: X [8192, 7168] bf16 with 1% outliers x20, W [2048, 7168] bf16
    x = _activations(8192, 7168, seed=2)
    w = _activations(2048, 7168, seed=21, outliers=False, std=0.02)
    _check(kern, dev, x, w, False, oracle=False)


def test_quant_fwd_rejects_mismatched_k(kern, dev):
    x = torch.zeros(4, 256, dtype=torch.bfloat16, device=dev)
    w = torch.zeros(4, 384, dtype=torch.bfloat16, device=dev)
    with pytest.raises(AssertionError, match="share K"):
        kern.quantize_fp8_forward(x, w)
