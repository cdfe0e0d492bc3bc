"""CPU pins of the oracle (oracle/fp8_oracle.py) — no GPU needed.

Each test checks the oracle against something that does not restate it: the OCP
e4m3fn spec (textbook RNE), a correctly rounded log2, hand-derived known answers,
identities between different oracle functions, and brute force on tiny inputs.
"""
import os

import numpy as np
import pytest
import torch

from oracle import fp8_oracle as orc


def _bits(e, m, sign=0):
    return np.uint32(sign) | (np.uint32(e + 127) << np.uint32(23)) | np.asarray(m, dtype=np.uint32)


# ---------------------------------------------------------------------------
# e4m3 cast (torch float8_e4m3fn, used by the oracle) == textbook OCP RNE
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("e", list(range(-12, 9)))
def test_e4m3_cast_exhaustive_per_binade(e):
    """Every fp32 of both signs in binade 2^e (e covers all non-trivial rounding)."""
    m = np.arange(0, 1 << 23, dtype=np.uint32)
    for sign in (0, 0x80000000):
        v = _bits(e, m, sign).view(np.float32)
        want = orc.e4m3_rne_np(v)
        got = torch.from_numpy(v.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, f"binade {e} sign {sign:#x}: first mismatches {v[bad[:4]]}"


def test_e4m3_cast_specials():
    v = np.array([0.0, -0.0, 1e-30, -1e-30, 2.0**-10, 2.0**-10 * 1.0000001, 448.0, 460.0, 464.0,
                  464.00003, -448.0, np.inf, -np.inf, np.nan, 1.0625, 1.1875, 2.0**-126],
                 dtype=np.float32)
    want = orc.e4m3_rne_np(v)
    got = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert (got == want).all()
    # hand-derived: RNE ties go to even mantissa; 1.0625 -> 1.0 (0x38), 1.1875 -> 1.25 (0x3A)
    assert list(want[[0, 1, 6, 10, 14, 15]]) == [0x00, 0x80, 0x7E, 0xFE, 0x38, 0x3A]
    assert want[4] == 0x00 and want[5] == 0x01  # 2^-10 is the tie between 0 and 2^-9
    assert want[8] == 0x7E and want[9] == 0x7F  # 464 ties to 448; above it is NaN


# ---------------------------------------------------------------------------
# round_scale: torch exp2(ceil(log2(v))) == ceil of the correctly rounded fp32 log2,
# == the integer threshold rule the HIP kernel uses (cin_common.h compute_scale)
# ---------------------------------------------------------------------------
def _kernel_rule_exponent(k, m):
    """The HIP kernel's rule, restated: exponent of the round_scale result."""
    if m == 0:
        return k
    a = k if k > 0 else (-k - 1 if k < 0 else 0)
    j = a.bit_length() - 1 if a else -1
    t = 1 if j <= 1 else {2: 2, 3: 3, 4: 6, 5: 12}.get(j, 23)
    return k + 1 if m >= t else k


def test_round_scale_thresholds_all_exponents():
    # every exponent reachable from amax in [fp32(1e-4), fp32 max] / 448
    ms = np.concatenate([np.arange(0, 64, dtype=np.uint32),
                         np.random.default_rng(0).integers(64, 1 << 23, 512, dtype=np.uint32),
                         np.array([(1 << 23) - 1], dtype=np.uint32)])
    for k in range(-23, 120):
        v = _bits(k, ms).view(np.float32)
        got = torch.exp2(torch.ceil(torch.log2(torch.from_numpy(v.copy())))).numpy()
        cr = np.exp2(np.ceil(np.log2(v.astype(np.float64)).astype(np.float32).astype(np.float64)))
        assert (got == cr.astype(np.float32)).all(), k
        rule = np.array([2.0 ** _kernel_rule_exponent(k, int(mm)) for mm in ms], dtype=np.float32)
        assert (got == rule).all(), (k, ms[got != rule][:4])


@pytest.mark.slow
def test_round_scale_exhaustive():
    """All 2^23 mantissas for every reachable exponent (long; run with -m slow)."""
    m = np.arange(0, 1 << 23, dtype=np.uint32)
    for k in range(-23, 120):
        v = torch.from_numpy(_bits(k, m).view(np.float32).copy())
        eq_k = (torch.log2(v) == float(k)).numpy()
        thr = int(np.nonzero(~eq_k[1:])[0][0]) + 1
        assert eq_k[1:thr].all() and not eq_k[thr:].any()
        assert _kernel_rule_exponent(k, thr) == k + 1 and _kernel_rule_exponent(k, thr - 1) in (k, k + 1)
        if thr > 1:
            assert _kernel_rule_exponent(k, thr - 1) == k


# ---------------------------------------------------------------------------
# Quantizer known answers and invariants
# ---------------------------------------------------------------------------
def test_rowwise_known_answers_fp32():
    x = torch.zeros(1, 128)
    x[0, :4] = torch.tensor([448.0, 1.0, -1.0, 0.5])
    q, s = orc.quant_rowwise(x)
    assert s.item() == 1.0  # 448 / 448
    assert q.view(torch.uint8)[0, :5].tolist() == [0x7E, 0x38, 0xB8, 0x30, 0x00]
    x = torch.zeros(1, 128)
    x[0, :2] = torch.tensor([896.0, 3.0])
    q, s = orc.quant_rowwise(x)
    assert s.item() == 2.0 and q.view(torch.uint8)[0, :2].tolist() == [0x7E, 0x3C]  # 3/2 = 1.5


_TRITON_FLOOR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "triton_floor.npz")
_FLOOR_DTYPES = (("bf16", torch.bfloat16), ("f16", torch.float16), ("f32", torch.float32))


def _from_bits(b, dt):
    return torch.from_numpy(b.view(np.int32) if dt == torch.float32 else b.view(np.int16)).view(dt)


def test_zero_tile_scale_known_answer_every_dtype():
    # Triton's interpreter printed 2.2321428616578487e-07 = fp32(1e-4) / 448 for zero
    # bf16, fp16 and fp32 tiles alike (tests/golden/gen_triton_floor.py).
    for dt in (torch.bfloat16, torch.float16, torch.float32):
        for fn in (lambda x: orc.quant_rowwise(x), lambda x: orc.quant_blockwise(x)):
            q, s = fn(torch.zeros(130, 256, dtype=dt))
            assert (s == 2.2321428616578487e-07).all(), dt
            assert (q.view(torch.uint8) == 0).all()


@pytest.mark.parametrize("name,dt", _FLOOR_DTYPES)
def test_floor_matches_triton_typing(name, dt):
    """Scales and codes of zero, tiny (N(0, 2e-5)), floor-edge and ordinary tiles against
    what Triton itself computed for the same inputs (tests/golden/triton_floor.npz).

    The fixture's codes are Triton's fp32 quotient cast by torch's RNE cast (pinned to the
    textbook cast above).  Elements whose input is NaN are left out of the code
    comparison: the interpreter lowers tl.maximum's maxnumf to np.maximum, which keeps
    NaN, while compiled Triton emits maxnumf and maps NaN to -448 (code 0xFE); the scale
    of a tile holding a NaN is compared like every other."""
    d = np.load(_TRITON_FLOOR)
    x = _from_bits(d[f"row_x_{name}"], dt)
    nan = torch.isnan(x.float()).numpy()
    assert nan.sum() == 1
    floored = 0
    for rs in (0, 1):
        q, s = orc.quant_rowwise(x, 128, bool(rs))
        want_s = d[f"row_s_{name}_rs{rs}"]
        assert np.array_equal(s.numpy().view(np.uint32), want_s.view(np.uint32))
        got = q.view(torch.uint8).numpy()
        assert np.array_equal(got[~nan], d[f"row_q_{name}_rs{rs}"][~nan])
        floored += int((want_s == np.float32(1e-4) / np.float32(448.0)).sum())
    assert floored >= 20   # most tiles of this input take the floor
    xb = _from_bits(d[f"blk_x_{name}"], dt)
    nan = torch.isnan(xb.float()).numpy()
    q, s = orc.quant_blockwise(xb, 128, 128, False)
    assert np.array_equal(s.numpy().view(np.uint32), d[f"blk_s_{name}"].view(np.uint32))
    assert np.array_equal(q.view(torch.uint8).numpy()[~nan], d[f"blk_q_{name}"][~nan])


def test_nan_and_inf_follow_maxnum_semantics():
    x = torch.zeros(1, 128)
    x[0, 0] = float("nan")
    x[0, 1] = 2.0
    x[0, 2] = -1.0
    q, s = orc.quant_rowwise(x)
    assert s.item() == np.float32(2.0) / np.float32(448.0)  # NaN ignored by the amax
    c = q.view(torch.uint8)[0]
    assert c[0].item() == 0xFE and c[1].item() == 0x7E  # NaN -> maxnum(NaN, -448) = -448
    x = torch.zeros(1, 128)
    x[0, 0] = float("inf")
    x[0, 1] = -3.0
    q, s = orc.quant_rowwise(x)
    c = q.view(torch.uint8)[0]
    assert s.item() == float("inf") and c[0].item() == 0xFE and c[1].item() == 0x80


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_quant_invariants_random(dtype):
    g = torch.Generator().manual_seed(7)
    x = torch.randn(64, 1000, generator=g)
    x[torch.rand(64, 1000, generator=g) < 0.01] *= 20
    x = x.to(dtype)
    q, s = orc.quant_rowwise(x)
    c = q.view(torch.uint8)
    assert s.shape == (64, 8)
    # the tile's amax element maps to +-448 and no code is NaN
    for t in range(8):
        tile = c[:, t * 128:(t + 1) * 128]
        assert ((tile & 0x7F).amax(dim=1) == 0x7E).all()
    assert not ((c & 0x7F) == 0x7F).any()
    # |dequant - x| <= half an e4m3 spacing (times the scale) everywhere
    y = x.float() / s.repeat_interleave(128, dim=1)[:, :1000]
    deq = q.float()
    spacing = torch.where(deq.abs() >= 2.0 ** -6, torch.exp2(torch.floor(torch.log2(deq.abs().clamp_min(2.0 ** -6)))) / 8,
                          torch.full_like(deq, 2.0 ** -9))
    assert ((deq - y).abs() <= spacing / 2 * (1 + 1e-6)).all()


def test_column_tiles_equal_rowwise_of_transpose():
    # quant_rowwise(dY^T) (src/kernels.py:781-783) == 128x1 column tiles of dY
    g = torch.Generator().manual_seed(3)
    dy = (torch.randn(300, 200, generator=g) * 1e-3).to(torch.bfloat16)
    qt, st = orc.quant_rowwise(dy.t().contiguous())
    qc, sc = orc.quant_blockwise(dy, 128, 1)
    assert torch.equal(qt.view(torch.uint8), qc.view(torch.uint8).t())
    assert torch.equal(st, sc.t())


def test_blockwise_1xN_equals_rowwise():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(50, 300, generator=g).to(torch.bfloat16)
    q1, s1 = orc.quant_rowwise(x, 128)
    q2, s2 = orc.quant_blockwise(x, 1, 128)
    assert torch.equal(q1.view(torch.uint8), q2.view(torch.uint8)) and torch.equal(s1, s2)


# ---------------------------------------------------------------------------
# GEMM oracle vs brute force (src/kernels.py:634-660 loop order, fp64)
# ---------------------------------------------------------------------------
def test_gemm_oracle_vs_bruteforce():
    g = torch.Generator().manual_seed(5)
    M, N, K = 3, 130, 256
    a, sa = orc.quant_rowwise(torch.randn(M, K, generator=g))
    w, sw = orc.quant_blockwise(torch.randn(N, K, generator=g) * 0.02)
    b = w.view(torch.uint8).t().contiguous()   # [K, N]
    sb = sw.t().contiguous()                   # [kb, nb]
    got = orc.gemm_ref(a, sa, b, sb)
    af, bf = a.float().double(), b.view(torch.float8_e4m3fn).float().double()
    want = torch.zeros(M, N, dtype=torch.float64)
    for kb in range(K // 128):
        ks = slice(kb * 128, (kb + 1) * 128)
        for n in range(N):
            an = af[:, ks] * sa[:, kb:kb + 1].double()
            bn = bf[ks, n] * sb[kb, n // 128].double()
            want[:, n] += an @ bn
    assert orc.frob_rel(got, want) < 1e-6 and orc.normwise_max_rel(got, want) < 1e-6


def test_fp8_linear_exact_on_representable_inputs():
    """Inputs on the e4m3 grid with tile amax 448*2^j quantize exactly, so the whole
    forward/backward chain must equal the float64 matmuls (catches any operand or
    transpose mix-up in the oracle's restatement of src/kernels.py:739-794)."""
    g = torch.Generator().manual_seed(9)
    M, N, K = 256, 256, 384
    grid_vals = torch.tensor([0.0, 0.5, 1.0, -1.0, 2.0, -3.0, 448.0])

    def make(rows, cols, scale):
        idx = torch.randint(0, 6, (rows, cols), generator=g)
        v = grid_vals[idx]
        v[:, ::128] = 448.0  # every 1x128 row tile holds 448 ...
        v[::128, :] = 448.0  # ... and every 128x1 column tile too
        return v * scale

    x = make(M, K, 2.0 ** -4)
    w = make(N, K, 2.0 ** -10)
    dy = make(M, N, 2.0 ** -12)
    r = orc.fp8_linear_ref(x, w, dy)
    xd, wd, dyd = x.double(), w.double(), dy.double()
    # quantization is exact here; only fp32 summation rounding remains
    for got, want in [(r["y"], xd @ wd.t()), (r["dx"], dyd @ wd), (r["dw"], dyd.t() @ xd)]:
        assert orc.normwise_max_rel(got, want) < 1e-6
    # and the saved codes dequantize back to the inputs bit-exactly
    assert torch.equal(orc.dequant_rowwise(r["x_fp8"], r["x_scale"]), x)
    assert torch.equal(orc.dequant_block(r["w_fp8"], r["w_scale"]), w)
    assert torch.equal(orc.dequant_rowwise(r["g_fp8_t"], r["g_scale_t"]), dy.t())
    assert torch.equal(orc.dequant_block(r["xb_fp8"], r["xb_scale"]), x)


def test_grouped_oracle_e1_equals_dense():
    g = torch.Generator().manual_seed(11)
    T, N, K = 200, 256, 256
    a, sa = orc.quant_rowwise(torch.randn(T, K, generator=g).to(torch.bfloat16))
    w, sw = orc.quant_blockwise(torch.randn(N, K, generator=g) * 0.02)
    got = orc.grouped_gemm_ref(a, sa, w.view(torch.uint8)[None], sw[None], [0], [T])
    want = orc.gemm_ref(a, sa, w.view(torch.uint8).t().contiguous(), sw.t().contiguous())
    assert torch.equal(got, want)


# ---------------------------------------------------------------------------
# The HIP quantizers compute x / s without a division: q = RN(x * r), r = RN(1/s),
# then STEPS corrections q = fma(-fma(q, s, -x), r, q) (cin_common.h div_by_scale),
# one step for bf16/fp16 inputs and two for fp32.  Check on the CPU that this equals
# the IEEE quotient: exhaustively over bf16 mantissa pairs, on a large fp16 sample and
# on random plus midpoint-planted fp32 inputs.  The fp32 fma is emulated with one
# rounding in float64 (TwoSum + midpoint fix-up), itself checked against exact
# rational arithmetic.
# ---------------------------------------------------------------------------
def _fma32(a, b, c):
    a, b, c = a.astype(np.float64), b.astype(np.float64), c.astype(np.float64)
    p = a * b                                       # exact: 24 x 24 bits
    hi = p + c
    bb = hi - p
    lo = (p - (hi - bb)) + (c - bb)                 # p + c == hi + lo exactly
    f = hi.astype(np.float32)
    fd = f.astype(np.float64)
    nb = np.where(fd <= hi, np.nextafter(f, np.float32(np.inf)),
                  np.nextafter(f, np.float32(-np.inf))).astype(np.float64)
    lower, upper = np.minimum(fd, nb), np.maximum(fd, nb)
    tie = (hi == (lower + upper) / 2) & (lo != 0)   # double rounding only on a tie
    return np.where(tie, np.where(lo > 0, upper, lower), fd).astype(np.float32)


def _div_by_scale(x, s, r, steps):
    q = (x * r).astype(np.float32)
    for _ in range(steps):
        q = _fma32(-_fma32(q, s, -x), r, q)
    return q


def test_fma32_emulation_is_single_rounding():
    from fractions import Fraction
    rng = np.random.default_rng(5)
    n = 3000
    a = (rng.standard_normal(n) * 2.0 ** rng.integers(-20, 20, n)).astype(np.float32)
    b = (rng.standard_normal(n) * 2.0 ** rng.integers(-20, 20, n)).astype(np.float32)
    # c close to -a*b so that cancellation and ties are exercised
    c = np.where(rng.random(n) < 0.5, -(a.astype(np.float64) * b).astype(np.float32),
                 rng.standard_normal(n).astype(np.float32))
    got = _fma32(a, b, c)
    for i in range(n):
        exact = Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i]))
        f = np.float32(float(exact))                # float() is correctly rounded to double
        # correct rounding to fp32: pick the nearer of the two fp32 neighbours of exact
        lo_ = f if Fraction(float(f)) <= exact else np.nextafter(f, np.float32(-np.inf))
        hi_ = np.nextafter(lo_, np.float32(np.inf)) if Fraction(float(lo_)) != exact else lo_
        dlo, dhi = exact - Fraction(float(lo_)), Fraction(float(hi_)) - exact
        want = lo_ if (dlo < dhi or (dlo == dhi and (lo_.view(np.uint32) & 1) == 0)) else hi_
        assert got[i] == want or (got[i] == 0 and want == 0), (a[i], b[i], c[i])


def _mantissa_pairs(bits, gaps, rng=None, sample=None):
    m = np.arange(1 << bits, 1 << (bits + 1), dtype=np.float64)
    for d in gaps:
        mx, ma = np.meshgrid(m, m, indexing="ij")
        x, amax = (mx * 2.0 ** d).ravel(), ma.ravel()
        if sample is not None:
            k = rng.choice(x.size, sample, replace=False)
            x, amax = x[k], amax[k]
        keep = x <= amax
        yield x[keep].astype(np.float32), amax[keep].astype(np.float32)


@pytest.mark.parametrize("bits,sample", [(7, None), (10, 40000)])
def test_division_free_quotient_16bit_inputs(bits, sample):
    """bf16 (7 stored mantissa bits): every (x, amax) pair; fp16 (10 bits): a sample."""
    rng = np.random.default_rng(bits)
    for x, amax in _mantissa_pairs(bits, range(-30, 1), rng, sample):
        s = (amax / np.float32(448.0)).astype(np.float32)
        r = (np.float32(1.0) / s).astype(np.float32)
        for xs in (x, -x):
            assert np.array_equal(_div_by_scale(xs, s, r, 1), (xs / s).astype(np.float32))


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_division_free_quotient_floored_16bit_tiles(dt):
    """A floored 16-bit tile divides by s = RN(fp32(1e-4) / 448), which no 16-bit amax
    produces: one correction step is still exact for every value of the dtype below the
    floor (all of them, both signs)."""
    every = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(dt).float().numpy()
    floor = np.float32(1e-4)
    x = every[np.isfinite(every) & (np.abs(every) < floor)]
    assert x.size > 3000
    s = np.full_like(x, np.float32(floor / np.float32(448.0)))
    r = (np.float32(1.0) / s).astype(np.float32)
    want = (x / s).astype(np.float32)
    assert np.array_equal(_div_by_scale(x, s, r, 1).view(np.uint32), want.view(np.uint32))


def test_division_free_quotient_fp32_inputs():
    rng = np.random.default_rng(123)
    n = 1_000_000
    amax = np.exp(rng.uniform(np.log(1e-4), np.log(1e30), n)).astype(np.float32)
    s = (amax / np.float32(448.0)).astype(np.float32)
    x = (amax * rng.uniform(-1, 1, n).astype(np.float32)).astype(np.float32)
    # quotients planted on and next to every e4m3 rounding midpoint (+-6 fp32 steps)
    vals = torch.arange(0, 0x7F, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    mids = ((vals[:-1].astype(np.float64) + vals[1:]) / 2).astype(np.float32)
    k = np.arange(-6, 7, dtype=np.int64)
    planted = (mids.view(np.uint32)[:, None].astype(np.int64) + k[None, :]).astype(np.uint32).view(np.float32).ravel()
    planted = np.tile(planted, 200)
    sp = s[: planted.size]
    xp = (planted.astype(np.float64) * sp).astype(np.float32)
    x = np.concatenate([x, xp, -xp])
    s = np.concatenate([s, sp, sp])
    r = (np.float32(1.0) / s).astype(np.float32)
    exact = (x / s).astype(np.float32)
    assert np.array_equal(_div_by_scale(x, s, r, 2), exact)
    # signed zeros keep their sign (the reference maps -0 to code 0x80)
    z = np.array([0.0, -0.0], dtype=np.float32)
    for steps in (1, 2):
        q = _div_by_scale(z, s[:2], r[:2], steps)
        assert np.array_equal(np.signbit(q), [False, True])
    # the bare product is not enough: without a correction step codes differ
    y0 = (x * r).astype(np.float32)
    assert not np.array_equal(y0, exact)


# ---------------------------------------------------------------------------
# Reference names outside the FP8 path (torch restatements in cinnamon_amd.kernels)
# ---------------------------------------------------------------------------
def test_sparse_attention_matches_brute_force():
    from cinnamon_amd import kernels
    g = torch.Generator().manual_seed(3)
    B, H, L, D, Kk = 2, 3, 9, 8, 4
    q, k, v = (torch.randn(B, H, L, D, generator=g) for _ in range(3))
    idx = torch.randint(0, L, (B, L, Kk), generator=g)
    out, p = kernels.sparse_attention(q, k, v, idx, 0.5)
    for b in range(B):
        for h in range(H):
            for t in range(L):
                sel = [j for j in idx[b, t].tolist()]
                s = torch.tensor([float(q[b, h, t] @ k[b, h, j]) * 0.5 if j <= t else float("-inf") for j in sel])
                w = torch.softmax(s, 0) if torch.isfinite(s).any() else torch.zeros(Kk)
                assert torch.allclose(p[b, h, t], w, atol=1e-6)
                o = sum(w[i] * v[b, h, sel[i]] for i in range(Kk))
                assert torch.allclose(out[b, h, t], o, atol=1e-5)


def test_grouped_f16_oracle_single_expert_is_matmul():
    g = torch.Generator().manual_seed(4)
    a = torch.randn(70, 40, generator=g).to(torch.bfloat16)
    w = torch.randn(1, 30, 40, generator=g)
    got = orc.grouped_gemm_f16_ref(a, w, [0], [70])
    want = a.to(torch.float16).double() @ w[0].to(torch.float16).double().t()
    assert torch.equal(got, want)
