"""GPU parity of the HIP quantizers against the CPU oracle: codes and scales bit-exact.

Inputs are generated on the CPU with seeded generators and copied to the GPU, so both
sides see identical bits.
"""
import os

import numpy as np
import pytest
import torch

from oracle import fp8_oracle as orc

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fp8_golden.npz")


def _u8(t):
    return t.view(torch.uint8).cpu()


def _assert_codes_equal(got, want, what):
    got, want = _u8(got), want.view(torch.uint8)
    if not torch.equal(got, want):
        bad = (got != want).nonzero()
        i = tuple(bad[0].tolist())
        raise AssertionError(f"{what}: {bad.shape[0]} code mismatches, first at {i}: "
                             f"got {got[i]:#x} want {want[i]:#x}")


def _assert_scales_equal(got, want, what):
    got = got.cpu()
    eq = (got == want) | (torch.isnan(got) & torch.isnan(want))
    if not eq.all():
        bad = (~eq).nonzero()
        i = tuple(bad[0].tolist())
        raise AssertionError(f"{what}: {bad.shape[0]} scale mismatches, first at {i}: "
                             f"got {got[i].item()!r} want {want[i].item()!r}")


def _activations(M, N, seed, dtype=torch.bfloat16, outliers=True, std=1.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, N, generator=g) * std
    if outliers:
        x[torch.rand(M, N, generator=g) < 0.01] *= 20
    return x.to(dtype)


# ---------------------------------------------------------------------------
# row-wise 1 x 128
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape,dtype,rs", [
    ((2048, 512), torch.bfloat16, False),     # config 1 activations
    ((8192, 7168), torch.bfloat16, False),    # config 2 activations (1% outliers x20)
    ((16368, 1024), torch.float32, True),     # config 5 MTP rows, fp32 RMSNorm output, round_scale
    ((70, 200), torch.bfloat16, False),       # tails in both dims
    ((3, 1000), torch.float32, False),
    ((1, 128), torch.float16, False),
    ((257, 384), torch.bfloat16, True),
])
def test_rowwise_bit_exact(kern, dev, shape, dtype, rs):
    x = _activations(*shape, seed=1, dtype=dtype)
    q, s = kern.quantize_fp8_rowwise(x.to(dev), 128, rs)
    rq, rs_ = orc.quant_rowwise(x, 128, rs)
    assert q.dtype == torch.float8_e4m3fn and q.shape == shape
    assert s.shape == (shape[0], -(-shape[1] // 128))
    _assert_codes_equal(q, rq, f"codes {shape}")
    _assert_scales_equal(s, rs_, f"scales {shape}")


@pytest.mark.parametrize("block", [32, 64, 100, 256, 1024])
def test_rowwise_other_block_sizes(kern, dev, block):
    x = _activations(96, 1100, seed=2)
    q, s = kern.quantize_fp8_rowwise(x.to(dev), block)
    rq, rs_ = orc.quant_rowwise(x, block)
    _assert_codes_equal(q, rq, f"codes block {block}")
    _assert_scales_equal(s, rs_, f"scales block {block}")


def test_rowwise_strided_input(kern, dev):
    x = _activations(384, 256, seed=3)
    xt = x.to(dev).t()  # non-contiguous [256, 384]
    q, s = kern.quantize_fp8_rowwise(xt)
    rq, rs_ = orc.quant_rowwise(x.t().contiguous())
    _assert_codes_equal(q, rq, "strided codes")
    _assert_scales_equal(s, rs_, "strided scales")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_rowwise_special_tiles(kern, dev, dtype):
    x = torch.randn(8, 512, generator=torch.Generator().manual_seed(4))
    x[0, :128] = 0.0                        # zero tile -> fp32(1e-4) floor
    x[1, 128:256] *= 1e-6                   # tiny tile -> floor active
    x[2, 5] = float("nan")                  # NaN ignored by amax, coded as -448
    x[3, 300] = float("inf")                # inf tile: scale inf, finite -> +-0
    x[4, 0] = -float("inf")
    x[5, 400:512] = float("nan")
    x[6, 7] = 3.0e38 if dtype == torch.float32 else 1e4
    x[7, :64] = -0.0                        # signed zeros keep their sign (code 0x80)
    x[7, 256:384:2] = -0.0
    x = x.to(dtype)
    q, s = kern.quantize_fp8_rowwise(x.to(dev))
    rq, rs_ = orc.quant_rowwise(x)
    _assert_codes_equal(q, rq, f"special codes {dtype}")
    _assert_scales_equal(s, rs_, f"special scales {dtype}")


def test_rowwise_against_golden(kern, dev):
    d = np.load(GOLDEN)
    x = torch.from_numpy(d["x_bf16"].view(np.int16)).view(torch.bfloat16)
    for rs in (0, 1):
        q, s = kern.quantize_fp8_rowwise(x.to(dev), 128, bool(rs))
        _assert_codes_equal(q, torch.from_numpy(d[f"x_row_q_rs{rs}"]), f"golden codes rs{rs}")
        _assert_scales_equal(s, torch.from_numpy(d[f"x_row_s_rs{rs}"]), f"golden scales rs{rs}")


def test_rowwise_deterministic(kern, dev):
    x = _activations(1024, 7168, seed=5).to(dev)
    a = kern.quantize_fp8_rowwise(x)
    b = kern.quantize_fp8_rowwise(x)
    assert torch.equal(_u8(a[0]), _u8(b[0])) and torch.equal(a[1], b[1])


# ---------------------------------------------------------------------------
# block-wise 128 x 128
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape,dtype,std", [
    ((1024, 512), torch.float32, 0.02),    # config 1 weights (fp32 master)
    ((2048, 7168), torch.bfloat16, 0.02),  # config 2 weights
    ((300, 200), torch.float32, 1.0),      # tails
    ((128, 16), torch.bfloat16, 1.0),
])
def test_blockwise_bit_exact(kern, dev, shape, dtype, std):
    w = _activations(*shape, seed=6, dtype=dtype, outliers=False, std=std)
    q, s = kern.quantize_fp8_blockwise(w.to(dev))
    rq, rs_ = orc.quant_blockwise(w)
    _assert_codes_equal(q, rq, f"block codes {shape}")
    _assert_scales_equal(s, rs_, f"block scales {shape}")
    # the variant that also writes the transposed codes for dgrad
    q2, qt, s2 = kern.quantize_fp8_blockwise_t(w.to(dev))
    _assert_codes_equal(q2, rq, "block codes (dual layout)")
    _assert_codes_equal(qt, rq.view(torch.uint8).t().contiguous(), "transposed block codes")
    _assert_scales_equal(s2, rs_, "block scales (dual layout)")


def _special_matrix(M, N, dtype, seed):
    x = torch.randn(M, N, generator=torch.Generator().manual_seed(seed))
    x[:, 0] = -0.0
    x[5, :] = -0.0
    x[:128, 128:256] = 0.0                   # zero block -> floor
    x[130, 131] = float("nan")
    x[200, 300] = float("inf")
    x[3, 260:270] = -0.0
    x[140:150, 140:150] *= 1e-7
    return x.to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_special_values_block_dual_requant(kern, dev, dtype):
    x = _special_matrix(256, 384, dtype, seed=8)
    q, s = kern.quantize_fp8_blockwise(x.to(dev))
    rq, rs_ = orc.quant_blockwise(x)
    _assert_codes_equal(q, rq, f"special block codes {dtype}")
    _assert_scales_equal(s, rs_, f"special block scales {dtype}")
    q, s, qt, st = kern.quantize_fp8_dual(x.to(dev))
    rq, rs_ = orc.quant_rowwise(x)
    rqt, rst = orc.quant_rowwise(x.t().contiguous())
    _assert_codes_equal(q, rq, "special dual row codes")
    _assert_scales_equal(s, rs_, "special dual row scales")
    _assert_codes_equal(qt, rqt, "special dual transposed codes")
    _assert_scales_equal(st, rst, "special dual transposed scales")
    # row-wise codes with signed zeros through the re-quantization (NaN/inf excluded:
    # the reference's requantization takes finite row-wise codes)
    xf = x.float().nan_to_num(0.0, 0.0, 0.0).to(dtype)
    xf[:, 0] = -0.0
    a, sa = orc.quant_rowwise(xf)
    qb, sb = kern.requantize_rowwise_to_blockwise(a.to(dev), sa.to(dev))
    rqb, rsb = orc.quant_blockwise(orc.dequant_rowwise(a, sa))
    _assert_codes_equal(qb, rqb, "special requant codes")
    _assert_scales_equal(sb, rsb, "special requant scales")


@pytest.mark.parametrize("bm,bn,rs", [(64, 64, False), (128, 1, False), (1, 128, True), (32, 256, True)])
def test_blockwise_other_blocks(kern, dev, bm, bn, rs):
    w = _activations(300, 520, seed=7, dtype=torch.float32)
    q, s = kern.quantize_fp8_blockwise(w.to(dev), bm, bn, rs)
    rq, rs_ = orc.quant_blockwise(w, bm, bn, rs)
    _assert_codes_equal(q, rq, f"codes {bm}x{bn}")
    _assert_scales_equal(s, rs_, f"scales {bm}x{bn}")


def test_blockwise_against_golden(kern, dev):
    d = np.load(GOLDEN)
    w = torch.from_numpy(d["w_f32"])
    q, s = kern.quantize_fp8_blockwise(w.to(dev))
    _assert_codes_equal(q, torch.from_numpy(d["w_blk_q"]), "golden block codes")
    _assert_scales_equal(s, torch.from_numpy(d["w_blk_s"]), "golden block scales")


# ---------------------------------------------------------------------------
# dual quantization of gradients (row tiles of dY and of dY^T) — config 4
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape,dtype,rs", [
    ((8192, 2048), torch.bfloat16, False),   # config 4 dY ~ N(0, 1e-3)
    ((8192, 2048), torch.bfloat16, True),
    ((300, 200), torch.bfloat16, False),     # tails
    ((256, 384), torch.float32, True),
])
def test_dual_bit_exact(kern, dev, shape, dtype, rs):
    dy = _activations(*shape, seed=4, dtype=dtype, outliers=False, std=1e-3)
    q, s, qt, st = kern.quantize_fp8_dual(dy.to(dev), rs)
    rq, rs_ = orc.quant_rowwise(dy, 128, rs)
    rqt, rst = orc.quant_rowwise(dy.t().contiguous(), 128, rs)
    _assert_codes_equal(q, rq, "dual row codes")
    _assert_scales_equal(s, rs_, "dual row scales")
    _assert_codes_equal(qt, rqt, "dual transposed codes")
    _assert_scales_equal(st, rst, "dual transposed scales")


def test_dual_against_golden(kern, dev):
    d = np.load(GOLDEN)
    dy = torch.from_numpy(d["dy_bf16"].view(np.int16)).view(torch.bfloat16)
    q, s, qt, st = kern.quantize_fp8_dual(dy.to(dev), True)
    _assert_codes_equal(q, torch.from_numpy(d["dy_row_q"]), "golden dy codes")
    _assert_scales_equal(s, torch.from_numpy(d["dy_row_s"]), "golden dy scales")
    _assert_codes_equal(qt, torch.from_numpy(d["dyt_row_q"]), "golden dy^T codes")
    _assert_scales_equal(st, torch.from_numpy(d["dyt_row_s"]), "golden dy^T scales")


def test_dual_strided_input(kern, dev):
    dy = _activations(256, 384, seed=8, std=1e-3, outliers=False)
    g = dy.to(dev).t()  # [384, 256] non-contiguous
    q, s, qt, st = kern.quantize_fp8_dual(g)
    rq, rs_ = orc.quant_rowwise(dy.t().contiguous())
    rqt, rst = orc.quant_rowwise(dy)
    _assert_codes_equal(q, rq, "strided dual row codes")
    _assert_codes_equal(qt, rqt, "strided dual transposed codes")
    _assert_scales_equal(s, rs_, "strided dual row scales")
    _assert_scales_equal(st, rst, "strided dual transposed scales")


# ---------------------------------------------------------------------------
# row -> block re-quantization (backward X operand) and dequantizers
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape", [(8192, 7168), (300, 200), (128, 128)])
def test_requant_bit_exact(kern, dev, shape):
    x = _activations(*shape, seed=2)
    rq, rs_ = orc.quant_rowwise(x)
    want_q, want_s = orc.quant_blockwise(orc.dequant_rowwise(rq, rs_), 128, 128, False)
    qd, sd = rq.to(dev), rs_.to(dev)
    qb, sb = kern.requantize_rowwise_to_blockwise(qd, sd, transposed=False)
    _assert_codes_equal(qb, want_q, "requant codes")
    _assert_scales_equal(sb, want_s, "requant scales")
    qbt, sbt = kern.requantize_rowwise_to_blockwise(qd, sd, transposed=True)
    _assert_codes_equal(qbt, want_q.view(torch.uint8).t().contiguous(), "requant transposed codes")
    _assert_scales_equal(sbt, want_s, "requant transposed scales")


@pytest.mark.parametrize("M,N,K,dtype,rs", [
    (8192, 2048, 7168, torch.bfloat16, False),   # config 4: one launch
    (300, 256, 384, torch.float16, True),        # one launch, last row block partial
    (1024, 512, 768, torch.bfloat16, False),
    (260, 200, 384, torch.bfloat16, False),      # N % 128 != 0: the two launches
    (256, 256, 200, torch.bfloat16, False),      # K % 128 != 0: the two launches
    (384, 256, 256, torch.float32, False),       # fp32 dY: the two launches
])
def test_backward_triple_bit_exact(kern, dev, M, N, K, dtype, rs):
    """quantize_fp8_backward (the backward's three quantizations in one launch) against the
    oracle chain (src/kernels.py:771, :781-787), with specials in dY's first tile."""
    dy = _activations(M, N, seed=M + N, dtype=torch.float32, std=1e-3)
    dy[0, :4] = torch.tensor([float("nan"), float("inf"), -0.0, 0.0])
    dy = dy.to(dtype)
    x = _activations(M, K, seed=K)
    rq, rs_ = orc.quant_rowwise(x)
    gq, gs = orc.quant_rowwise(dy, 128, rs)
    gqt, gst = orc.quant_rowwise(dy.t().contiguous(), 128, rs)
    bq, bs = orc.quant_blockwise(orc.dequant_rowwise(rq, rs_), 128, 128, False)
    got = kern.quantize_fp8_backward(dy.to(dev), rq.to(dev), rs_.to(dev), rs)
    torch.cuda.synchronize()
    for g, w, what in zip(got[0::2], (gq, gqt, bq.view(torch.uint8).t().contiguous()),
                          ("dY codes", "dY^T codes", "X^T block codes")):
        _assert_codes_equal(g, w, what)
    for g, w, what in zip(got[1::2], (gs, gst, bs), ("dY scales", "dY^T scales", "X block scales")):
        _assert_scales_equal(g, w, what)


def test_requant_against_golden(kern, dev):
    d = np.load(GOLDEN)
    q = torch.from_numpy(d["xc_row_q"]).to(dev)
    s = torch.from_numpy(d["xc_row_s"]).to(dev)
    qb, sb = kern.requantize_rowwise_to_blockwise(q, s)
    _assert_codes_equal(qb, torch.from_numpy(d["xc_blk_q"]), "golden requant codes")
    _assert_scales_equal(sb, torch.from_numpy(d["xc_blk_s"]), "golden requant scales")


def test_dequantizers(kern, dev):
    x = _activations(300, 520, seed=9)
    rq, rs_ = orc.quant_rowwise(x)
    got = kern.dequantize_fp8_rowwise(rq.to(dev), rs_.to(dev))
    assert got.dtype == torch.float32
    assert torch.equal(got.cpu(), orc.dequant_rowwise(rq, rs_))
    got = kern.dequantize_fp8(rq.to(dev), rs_.to(dev), block_m=1, block_n=128)
    assert got.dtype == torch.bfloat16
    assert torch.equal(got.cpu(), orc.dequant_block_bf16(rq, rs_, 1, 128))
    bq, bs = orc.quant_blockwise(x.float())
    got = kern.dequantize_fp8(bq.to(dev), bs.to(dev))
    assert torch.equal(got.cpu(), orc.dequant_block_bf16(bq, bs))


# ---------------------------------------------------------------------------
# 128 x 128 tile kernels: many tiles per workgroup, ragged last row block and column
# block (the column edge runs as a launch of its own)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("M,N,dtype", [
    (1000, 1100, torch.bfloat16),
    (2050, 4100, torch.float16),
    (4096, 640, torch.float32),
    (12000, 8300, torch.float32),   # ~6000 tiles: several per workgroup in the fp32 one-set walk
])
def test_tile_kernels_ragged_many_tiles(kern, dev, M, N, dtype):
    x = _activations(M, N, seed=11, dtype=dtype)
    rq, rs_ = orc.quant_blockwise(x)
    q2, qt, s2 = kern.quantize_fp8_blockwise_t(x.to(dev))
    _assert_codes_equal(q2, rq, "block codes")
    _assert_codes_equal(qt, rq.view(torch.uint8).t().contiguous(), "block transposed codes")
    _assert_scales_equal(s2, rs_, "block scales")
    q, s, qt, st = kern.quantize_fp8_dual(x.to(dev))
    rq, rs_ = orc.quant_rowwise(x)
    rqt, rst = orc.quant_rowwise(x.t().contiguous())
    _assert_codes_equal(q, rq, "dual row codes")
    _assert_scales_equal(s, rs_, "dual row scales")
    _assert_codes_equal(qt, rqt, "dual transposed codes")
    _assert_scales_equal(st, rst, "dual transposed scales")
    want_q, want_s = orc.quant_blockwise(orc.dequant_rowwise(rq, rs_), 128, 128, False)
    qbt, sbt = kern.requantize_rowwise_to_blockwise(q.view(torch.float8_e4m3fn), s, transposed=True)
    _assert_codes_equal(qbt, want_q.view(torch.uint8).t().contiguous(), "requant transposed codes")
    _assert_scales_equal(sbt, want_s, "requant scales")


def test_requant_every_code(kern, dev):
    """All 256 e4m3fn codes (NaN codes included) through the re-quantization: the
    hardware code -> fp32 conversion against torch's, with row scales spanning many
    binades and one infinite row scale (its tile's scale is inf: finite values -> +-0,
    inf and NaN -> NaN -> -448)."""
    g = torch.Generator().manual_seed(21)
    M, K = 384, 512
    codes = torch.stack([torch.randperm(256, generator=g)[: K // 2].repeat(2) for _ in range(M)])
    codes = codes.to(torch.uint8).view(torch.float8_e4m3fn)
    scales = torch.exp2(torch.randint(-20, 20, (M, K // 128), generator=g).float())
    scales *= 1 + torch.rand(M, K // 128, generator=g)
    scales[300, 2] = float("inf")
    want_q, want_s = orc.quant_blockwise(orc.dequant_rowwise(codes, scales), 128, 128, False)
    qb, sb = kern.requantize_rowwise_to_blockwise(codes.to(dev), scales.to(dev), transposed=False)
    _assert_codes_equal(qb, want_q, "every-code requant codes")
    _assert_scales_equal(sb, want_s, "every-code requant scales")
    qbt, sbt = kern.requantize_rowwise_to_blockwise(codes.to(dev), scales.to(dev), transposed=True)
    _assert_codes_equal(qbt, want_q.view(torch.uint8).t().contiguous(), "every-code requant^T codes")
    _assert_scales_equal(sbt, want_s, "every-code requant^T scales")


# ---------------------------------------------------------------------------
# the hardware e4m3 cast, exhaustively: every fp32 in the 21 binades that round
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("e", list(range(-12, 9)))
def test_e4m3_cast_exhaustive_through_rowwise(kern, dev, e):
    """Every fp32 of both signs in binade 2^e (e = -12 .. 8, the binades where the e4m3fn
    cast rounds), quantized by quantize_fp8_rowwise with a 448 pivot at the head of each
    tile: the scale is 448 / 448 = 1 and x / 1 = x, so each code is the cast of x itself.
    Compared with torch's CPU cast, which tests/test_oracle.py pins to the textbook OCP
    round-to-nearest-even on the same binades.  In binade 8 only |x| <= 448 is reachable
    (the quantizer clamps to +-448 before the cast)."""
    n = 1 << 23
    if e == 8:
        n = 3 * (1 << 21) + 1          # 256 * (1 + m / 2^23) <= 448
    m = torch.arange(0, n, dtype=torch.int64)
    bits = ((e + 127) << 23) | m
    for sign in (0, 1):
        b = bits | (sign << 31)
        v = (b - (1 << 32) * (b >= (1 << 31)).long()).to(torch.int32).view(torch.float32)
        rows = -(-n // 127)
        tiles = torch.zeros(rows * 127, dtype=torch.float32)
        tiles[:n] = v
        x = torch.cat([torch.full((rows, 1), 448.0), tiles.view(rows, 127)], dim=1)
        q, s = kern.quantize_fp8_rowwise(x.to(dev))
        assert bool((s == 1.0).all())
        got = q.view(torch.uint8)[:, 1:].reshape(-1)[:n].cpu()
        want = v.to(torch.float8_e4m3fn).view(torch.uint8)
        bad = (got != want).nonzero()
        assert bad.numel() == 0, f"binade {e} sign {sign}: {bad.numel()} codes differ, first x = {v[bad[0]].item()!r}"
        assert bool((q.view(torch.uint8)[:, 0] == 0x7E).all())
