"""Column-major scale matrices (strides (1, rows)) on the GPU.

Every quantizer that writes 1 x 128 row scales can write them column-major, and every kernel
that reads them (the re-quantizers, the GEMMs) takes either layout.  The values are the same
computation in a different place, so each check is bit-exact against the row-major call:
codes, scale values, block scales and GEMM outputs.  Shapes cover each entry point's fast
path and its fallback (partial column blocks, block sizes other than 128, strided input).
"""
import numpy as np
import pytest
import torch

from cinnamon_amd import kernels, layers, moe

pytestmark = pytest.mark.gpu


def _u8(q):
    return q.view(torch.uint8)


def _is_col_major(s):
    R, C = s.shape
    return s.stride(0) == 1 and (C <= 1 or s.stride(1) >= R)


def _same(a, b, what):
    assert torch.equal(a, b), f"{what} differs between the scale layouts"


def _x(M, N, dtype, dev, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, N, generator=g) * 3
    x[torch.rand(M, N, generator=g) < 0.01] *= 50
    if M > 3:
        x[3, : min(N, 128)] = 0  # a zero tile
    return x.to(dtype).to(dev)


@pytest.mark.parametrize("M,N,block,dtype", [
    (300, 1024, 128, torch.bfloat16),   # fast row-wise kernel
    (257, 200, 128, torch.float16),     # partial last column block
    (100, 384, 64, torch.float32),      # generic kernel (block 64)
])
def test_rowwise_col_scales(dev, M, N, block, dtype):
    x = _x(M, N, dtype, dev, seed=M)
    q0, s0 = kernels.quantize_fp8_rowwise(x, block, col_scales=False)
    q1, s1 = kernels.quantize_fp8_rowwise(x, block, col_scales=True)
    assert s0.is_contiguous() and _is_col_major(s1)
    _same(_u8(q0), _u8(q1), "codes")
    _same(s0, s1, "scales")


@pytest.mark.parametrize("M,N,K,wdtype", [
    (512, 384, 1024, torch.bfloat16),   # one launch
    (300, 256, 640, torch.float32),     # fp32 weight: the two quantizers in turn
])
def test_forward_pair_col_scales(dev, M, N, K, wdtype):
    x = _x(M, K, torch.bfloat16, dev, seed=1)
    w = (_x(N, K, torch.float32, dev, seed=2) * 0.01).to(wdtype)
    r0 = kernels.quantize_fp8_forward(x, w, with_transposed=True, col_scales=False)
    r1 = kernels.quantize_fp8_forward(x, w, with_transposed=True, col_scales=True)
    assert _is_col_major(r1[1])
    _same(_u8(r0[0]), _u8(r1[0]), "X codes")
    _same(r0[1], r1[1], "X scales")
    _same(_u8(r0[2]), _u8(r1[2]), "W codes")
    _same(_u8(r0[3]), _u8(r1[3]), "W^T codes")
    _same(r0[4], r1[4], "W scales")


@pytest.mark.parametrize("M,N,strided", [(512, 768, False), (300, 200, False), (256, 384, True)])
def test_dual_col_scales(dev, M, N, strided):
    dy = _x(M, N, torch.bfloat16, dev, seed=3) * 1e-3
    if strided:  # dy as a transposed view: the two generic row-wise passes
        dy = dy.t().contiguous().t()
    a = kernels.quantize_fp8_dual(dy, col_scales=False)
    b = kernels.quantize_fp8_dual(dy, col_scales=True)
    assert _is_col_major(b[1]) and _is_col_major(b[3])
    for i, what in enumerate(("q", "s", "qt", "st")):
        _same(a[i].view(torch.uint8) if i % 2 == 0 else a[i], b[i].view(torch.uint8) if i % 2 == 0 else b[i], what)


@pytest.mark.parametrize("M,K", [(512, 1024), (300, 200)])
@pytest.mark.parametrize("transposed", [False, True])
def test_requant_reads_col_scales(dev, M, K, transposed):
    x = _x(M, K, torch.bfloat16, dev, seed=4)
    q, s_row = kernels.quantize_fp8_rowwise(x)
    _, s_col = kernels.quantize_fp8_rowwise(x, col_scales=True)
    a = kernels.requantize_rowwise_to_blockwise(q, s_row, transposed=transposed)
    b = kernels.requantize_rowwise_to_blockwise(q, s_col, transposed=transposed)
    _same(_u8(a[0]), _u8(b[0]), "block codes")
    _same(a[1], b[1], "block scales")


@pytest.mark.parametrize("M,N,K", [(512, 768, 1024), (384, 200, 256)])
def test_backward_triple_col_scales(dev, M, N, K):
    """The one-launch backward (N, K multiples of 128) and its two-launch fallback."""
    dy = _x(M, N, torch.bfloat16, dev, seed=5) * 1e-3
    x = _x(M, K, torch.bfloat16, dev, seed=6)
    xq, xs_row = kernels.quantize_fp8_rowwise(x)
    _, xs_col = kernels.quantize_fp8_rowwise(x, col_scales=True)
    a = kernels.quantize_fp8_backward(dy, xq, xs_row, col_scales=False)
    b = kernels.quantize_fp8_backward(dy, xq, xs_col, col_scales=True)
    assert _is_col_major(b[1]) and _is_col_major(b[3])
    for i, what in enumerate(("g", "gs", "gt", "gst", "xbt", "xsblk")):
        ta, tb = a[i], b[i]
        if ta.dtype == torch.float8_e4m3fn:
            ta, tb = _u8(ta), _u8(tb)
        _same(ta, tb, what)


@pytest.mark.parametrize("M,N,K", [(512, 768, 1024), (8192, 2176, 384)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_gemm_col_a_scales(dev, M, N, K, out_dtype):
    """One-round (2 x 3 tiles) and persistent (32 x 9 tiles) GEMMs: column-major A scales
    give the same output, bit for bit."""
    x = _x(M, K, torch.bfloat16, dev, seed=7)
    w = _x(N, K, torch.bfloat16, dev, seed=8) * 0.02
    xq, s_row = kernels.quantize_fp8_rowwise(x)
    _, s_col = kernels.quantize_fp8_rowwise(x, col_scales=True)
    wq, ws = kernels.quantize_fp8_blockwise(w)
    a = kernels.fp8_gemm_bs(xq, s_row, wq, ws, out_dtype)
    b = kernels.fp8_gemm_bs(xq, s_col, wq, ws, out_dtype)
    _same(a, b, "GEMM output")


def _ranges(counts, dev):
    ends = torch.tensor(np.cumsum(counts), dtype=torch.int64)
    starts = ends - torch.tensor(counts, dtype=torch.int64)
    return starts.to(dev), ends.to(dev)


@pytest.mark.parametrize("counts,N", [([300, 0, 128, 1, 555], 384), ([700, 260], 200)])
def test_grouped_quantizers_col_scales(dev, counts, N):
    T = int(sum(counts))
    starts, ends = _ranges(counts, dev)
    dy = _x(T, N, torch.bfloat16, dev, seed=9) * 1e-3
    a = layers.quantize_fp8_dual_grouped(dy, starts, ends, col_scales=False)
    b = layers.quantize_fp8_dual_grouped(dy, starts, ends, col_scales=True)
    assert _is_col_major(b[1]) and _is_col_major(b[3])
    # rows outside every range are not written: compare the covered rows of q and s only
    cov = torch.zeros(T, dtype=torch.bool, device=dev)
    for s0, s1 in zip(starts.tolist(), ends.tolist()):
        cov[s0:s1] = True
    _same(_u8(a[0])[cov], _u8(b[0])[cov], "grouped q")
    _same(a[1][cov], b[1][cov], "grouped s")
    # the padded token axis is written up to the experts' padded end; the capacity past it
    # is never touched
    P = int(sum(-(-c // 128) * 128 for c in counts))
    _same(_u8(a[2])[:, :P], _u8(b[2])[:, :P], "grouped qt")
    _same(a[3][:, : P // 128], b[3][:, : P // 128], "grouped st")
    # grouped re-quantization reading either layout of the row scales
    x = _x(T, 512, torch.bfloat16, dev, seed=10)
    xq, xs_row = kernels.quantize_fp8_rowwise(x)
    _, xs_col = kernels.quantize_fp8_rowwise(x, col_scales=True)
    ra = layers.requantize_grouped_t(xq, xs_row, starts, ends)
    rb = layers.requantize_grouped_t(xq, xs_col, starts, ends)
    _same(_u8(ra[0])[:, :P], _u8(rb[0])[:, :P], "grouped block codes")
    _same(ra[1][: P // 128], rb[1][: P // 128], "grouped block scales")


@pytest.mark.parametrize("H", [2048, 200])
def test_silu_mul_col_scales(dev, H):
    h12 = _x(300, 2 * H, torch.bfloat16, dev, seed=11)
    a = layers.silu_mul_quantize_fp8(h12, col_scales=False)
    b = layers.silu_mul_quantize_fp8(h12, col_scales=True)
    assert _is_col_major(b[1])
    _same(_u8(a[0]), _u8(b[0]), "codes")
    _same(a[1], b[1], "scales")


@pytest.mark.parametrize("D", [7168, 1100])
def test_dispatch_quantize_col_scales(dev, D):
    T, k, E = 700, 4, 11
    g = torch.Generator().manual_seed(12)
    top_idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    top_idx[7, 1] = E + 3  # a dropped slot: its sorted row is the zero-row quantization
    x = _x(T, D, torch.bfloat16, dev, seed=13)
    perm, inv, *_ = moe.moe_route(top_idx.to(dev), E)
    for form in (None, inv):  # gather from the sorted side, scatter from the token side
        qa, sa = moe.moe_gather_quantize(x, perm, k, inv=form, col_scales=False)
        qb, sb = moe.moe_gather_quantize(x, perm, k, inv=form, col_scales=True)
        assert _is_col_major(sb)
        _same(_u8(qa), _u8(qb), "dispatch codes")
        _same(sa, sb, "dispatch scales")
