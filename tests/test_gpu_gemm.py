"""GPU parity of the block-scaled FP8 GEMMs (dense, dgrad/wgrad, grouped) against the
oracle's dequantize-then-fp32-matmul.

Tolerance (stated for the fp32 epilogue, compared in float64):
  normwise max relative  max|Y - Yref| / max|Yref|  <= 2e-3
  Frobenius relative     ||Y - Yref|| / ||Yref||     <= 1e-3
and the production bf16 output must equal the round-to-nearest-even of the fp32 output.
"""
import os

import numpy as np
import pytest
import torch

from oracle import fp8_oracle as orc

pytestmark = pytest.mark.gpu

MAX_REL = 2e-3
FROB_REL = 1e-3
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fp8_golden.npz")


def _check(got, want, what):
    mr = orc.normwise_max_rel(got.cpu(), want)
    fr = orc.frob_rel(got.cpu(), want)
    assert mr <= MAX_REL and fr <= FROB_REL, f"{what}: normwise max rel {mr:.3e}, frob rel {fr:.3e}"
    return mr, fr


def _operands(M, N, K, seed, outliers=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    if outliers:
        x[torch.rand(M, K, generator=g) < 0.01] *= 20
    x = x.to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    xq, xs = orc.quant_rowwise(x)
    wq, ws = orc.quant_blockwise(w)
    return xq, xs, wq, ws


def _run_fp32_and_bf16(kern, dev, xq, xs, wq, ws):
    a, sa, b, sb = xq.to(dev), xs.to(dev), wq.to(dev), ws.to(dev)
    y32 = kern.fp8_gemm_bs(a, sa, b, sb, torch.float32)
    y16 = kern.fp8_gemm_bs(a, sa, b, sb, torch.bfloat16)
    torch.cuda.synchronize()
    return y32, y16


@pytest.mark.parametrize("M,N,K", [
    (2048, 1024, 512),    # config 1
    (8192, 2048, 7168),   # config 2 (DeepSeek-V3 projection)
    (70, 200, 384),       # M/N tails
    (129, 257, 144),      # K not a multiple of 128
    (1, 128, 128),
    (16368, 1024, 1024),  # config 5 MTP rows
    (4100, 4224, 512),    # more 256 x 256 tiles than CUs (persistent walk), last row and column shifted
    (2304, 7296, 4096),   # persistent walk with the XCD-rotated K order (32 K blocks)
    (8192, 2176, 384),    # 288 tiles (persistent walk), N % 256 = 128: the last column tile shifted back
    (6400, 5376, 256),    # 525 tiles: XCD-major ranges of 65 and 66 tiles, three rounds
    (2560, 6912, 256),    # 270 tiles: ranges of 33 and 34 tiles, the last partly empty
])
def test_gemm_parity(kern, dev, M, N, K):
    xq, xs, wq, ws = _operands(M, N, K, seed=M + N + K)
    y32, y16 = _run_fp32_and_bf16(kern, dev, xq, xs, wq, ws)
    want = orc.gemm_ref(xq, xs, wq.view(torch.uint8).t().contiguous(), ws.t().contiguous())
    _check(y32, want, f"gemm {M}x{N}x{K}")
    assert y16.dtype == torch.bfloat16
    assert torch.equal(y16.cpu(), y32.cpu().to(torch.bfloat16)), "bf16 output is not RNE(fp32 output)"


def test_gemm_against_golden(kern, dev):
    d = np.load(GOLDEN)
    a = torch.from_numpy(d["xc_row_q"]).to(dev)
    sa = torch.from_numpy(d["xc_row_s"]).to(dev)
    b = torch.from_numpy(d["w_blk_q"]).to(dev)
    sb = torch.from_numpy(d["w_blk_s"]).to(dev)
    y = kern.fp8_gemm_bs(a, sa, b, sb, torch.float32)
    _check(y, torch.from_numpy(d["y_f32"]), "golden gemm")


def test_fp8_matmul_dsv3_api(kern, dev):
    """The reference signature: b is [K, N] (contiguous or a transposed view)."""
    xq, xs, wq, ws = _operands(512, 384, 640, seed=3)
    b_kn = wq.view(torch.uint8).t().contiguous()
    sb_kn = ws.t().contiguous()
    want = orc.gemm_ref(xq, xs, b_kn, sb_kn)
    y32 = kern.fp8_gemm_bs(xq.to(dev), xs.to(dev), wq.to(dev), ws.to(dev), torch.float32)
    _check(y32, want, "fp8_gemm_bs")
    for b in (b_kn.to(dev), wq.to(dev).view(torch.uint8).t()):
        y = kern.fp8_matmul_dsv3(xq.to(dev), b.view(torch.float8_e4m3fn), xs.to(dev), sb_kn.to(dev))
        assert y.dtype == torch.bfloat16 and y.shape == (512, 384)
        # bf16 output = RNE of the fp32 epilogue
        assert torch.equal(y, y32.to(torch.bfloat16))


def test_gemm_deterministic(kern, dev):
    xq, xs, wq, ws = _operands(1024, 1024, 2048, seed=12)
    a, sa, b, sb = xq.to(dev), xs.to(dev), wq.to(dev), ws.to(dev)
    y1 = kern.fp8_gemm_bs(a, sa, b, sb, torch.float32)
    y2 = kern.fp8_gemm_bs(a, sa, b, sb, torch.float32)
    assert torch.equal(y1, y2)


# ---------------------------------------------------------------------------
# FP8MatmulFunction forward + backward at config-4 shapes
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("M,N,K,rs", [(8192, 2048, 7168, False), (300, 256, 384, True), (16368, 384, 256, False)])
def test_fp8_linear_fwd_bwd(kern, dev, M, N, K, rs):
    g = torch.Generator().manual_seed(4)
    x = torch.randn(M, K, generator=g)
    x[torch.rand(M, K, generator=g) < 0.01] *= 20
    x = x.to(torch.bfloat16)
    w = torch.randn(N, K, generator=g) * 0.02          # fp32 master weight
    dy = (torch.randn(M, N, generator=g) * 1e-3).to(torch.bfloat16)
    ref = orc.fp8_linear_ref(x, w, dy, round_scale=rs)

    xd = x.to(dev).requires_grad_(True)
    wd = w.to(dev).requires_grad_(True)
    y = kern.FP8MatmulFunction.apply(xd, wd, rs)
    y.backward(dy.to(dev))
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16 and xd.grad.dtype == torch.bfloat16 and wd.grad.dtype == torch.float32
    # outputs are bf16 roundings of fp32 values: compare against the fp32 oracle with the
    # bf16 rounding allowance (2^-8 relative per element) added to the GEMM tolerance
    for name, got in (("y", y), ("dx", xd.grad), ("dw", wd.grad)):
        mr = orc.normwise_max_rel(got.float().cpu(), ref[name])
        fr = orc.frob_rel(got.float().cpu(), ref[name])
        assert mr <= MAX_REL + 2 ** -8 and fr <= FROB_REL + 2 ** -8, f"{name}: {mr:.3e} {fr:.3e}"


@pytest.mark.parametrize("which", ["dgrad", "wgrad"])
def test_config4_backward_gemms_tight(kern, dev, which):
    """Config 4's two GEMMs at their exact shapes, at the GEMM bar (2e-3 normwise, 1e-3
    Frobenius, fp32 epilogue), fed the operands the backward itself produces on the GPU:
    - dgrad dX[8192, 7168] = dY . W (src/kernels.py:774): A = the dual quantizer's dY row
      tiles, B = the forward quantizer's transposed weight codes Wt[7168, 2048] with the
      weight's block scales read transposed (the persistent walk, 16 K blocks per tile);
    - wgrad dW[2048, 7168] = dY^T . X (src/kernels.py:781-788): A = the dual quantizer's
      dY^T row tiles [2048, 8192], B = the re-quantized X codes, transposed to [7168, 8192]
      (one round of 256 x 256 tiles, 64 K blocks, XCD-rotated K order).
    Those operands are checked bit-exact against the oracle's chain first, and the bf16
    output must equal RNE of the fp32 output."""
    M, N, K = 8192, 2048, 7168
    g = torch.Generator().manual_seed(44)
    x = torch.randn(M, K, generator=g)
    x[torch.rand(M, K, generator=g) < 0.01] *= 20
    x = x.to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    dy = (torch.randn(M, N, generator=g) * 1e-3).to(torch.bfloat16)
    x_fp8, x_s, w_fp8, w_fp8_t, w_s = kern.quantize_fp8_forward(
        x.to(dev), w.to(dev), False, with_rowmajor=True, with_transposed=True)
    g_fp8, g_s, g_fp8_t, g_s_t = kern.quantize_fp8_dual(dy.to(dev))
    u8 = lambda t: t.view(torch.uint8).cpu()  # noqa: E731
    if which == "dgrad":
        rq, rs = orc.quant_rowwise(dy)
        wq, ws = orc.quant_blockwise(w.float())
        assert torch.equal(u8(g_fp8), rq.view(torch.uint8)) and torch.equal(g_s.cpu(), rs)
        assert torch.equal(u8(w_fp8_t), wq.view(torch.uint8).t()) and torch.equal(w_s.cpu(), ws)
        y32 = kern.fp8_gemm_bs(g_fp8, g_s, w_fp8_t, w_s.t(), torch.float32)
        y16 = kern.fp8_gemm_bs(g_fp8, g_s, w_fp8_t, w_s.t(), torch.bfloat16)
        want = orc.gemm_ref(rq, rs, wq, ws)                            # [M, K]
    else:
        xb_t, xb_s = kern.requantize_rowwise_to_blockwise(x_fp8, x_s, transposed=True)
        rq, rs = orc.quant_rowwise(dy.t().contiguous())
        xq, xs = orc.quant_rowwise(x)
        xb, xbs = orc.quant_blockwise(orc.dequant_rowwise(xq, xs, 128))
        assert torch.equal(u8(g_fp8_t), rq.view(torch.uint8)) and torch.equal(g_s_t.cpu(), rs)
        assert torch.equal(u8(xb_t), xb.view(torch.uint8).t()) and torch.equal(xb_s.cpu(), xbs)
        y32 = kern.fp8_gemm_bs(g_fp8_t, g_s_t, xb_t, xb_s.t(), torch.float32)
        y16 = kern.fp8_gemm_bs(g_fp8_t, g_s_t, xb_t, xb_s.t(), torch.bfloat16)
        want = orc.gemm_ref(rq, rs, xb, xbs)                            # [N, K]
    torch.cuda.synchronize()
    mr, fr = _check(y32, want, f"config-4 {which}")
    print(f"\nconfig-4 {which} {tuple(y32.shape)}: normwise max rel {mr:.2e}, frob rel {fr:.2e}", flush=True)
    assert torch.equal(y16.cpu(), y32.cpu().to(torch.bfloat16)), "bf16 output is not RNE(fp32 output)"


def test_fp8_linear_backward_operands_bit_exact(kern, dev):
    """The quantized operands the backward GEMMs consume are bit-exact to the reference chain."""
    M, N, K = 1024, 512, 768
    g = torch.Generator().manual_seed(14)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = torch.randn(N, K, generator=g) * 0.02
    dy = (torch.randn(M, N, generator=g) * 1e-3).to(torch.bfloat16)
    ref = orc.fp8_linear_ref(x, w, dy)
    xq, xs = kern.quantize_fp8_rowwise(x.to(dev))
    q, s, qt, st = kern.quantize_fp8_dual(dy.to(dev))
    xbt, xbs = kern.requantize_rowwise_to_blockwise(xq, xs, transposed=True)
    assert torch.equal(q.view(torch.uint8).cpu(), ref["g_fp8"].view(torch.uint8))
    assert torch.equal(qt.view(torch.uint8).cpu(), ref["g_fp8_t"].view(torch.uint8))
    assert torch.equal(st.cpu(), ref["g_scale_t"]) and torch.equal(s.cpu(), ref["g_scale"])
    assert torch.equal(xbt.view(torch.uint8).cpu(), ref["xb_fp8"].view(torch.uint8).t())
    assert torch.equal(xbs.cpu(), ref["xb_scale"])


# ---------------------------------------------------------------------------
# grouped GEMM (one launch over all experts, device-side tile table)
# ---------------------------------------------------------------------------
def _grouped_case(counts, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    T = int(sum(counts))
    x = torch.randn(T, K, generator=g).to(torch.bfloat16)
    E = len(counts)
    w = (torch.randn(E, N, K, generator=g) * 0.02)
    xq, xs = orc.quant_rowwise(x)
    wq, ws = orc.quant_blockwise(w.reshape(E * N, K))
    wq = wq.view(torch.uint8).view(E, N, K)
    ws = ws.view(E, -(-N // 128), -(-K // 128))
    ends = torch.tensor(np.cumsum(counts), dtype=torch.int64)
    starts = ends - torch.tensor(counts, dtype=torch.int64)
    return xq, xs, wq, ws, starts, ends


@pytest.mark.parametrize("counts,N,K", [
    ([300, 0, 128, 1, 555, 64, 0, 1000], 384, 512),
    ([128] * 8, 256, 256),
    ([4000], 512, 1024),
])
def test_grouped_gemm_parity(kern, dev, counts, N, K):
    from cinnamon_amd import layers
    xq, xs, wq, ws, starts, ends = _grouped_case(counts, N, K, seed=len(counts))
    want = orc.grouped_gemm_ref(xq, xs, wq, ws, starts, ends)
    out = layers.fp8_grouped_gemm(xq.to(dev), xs.to(dev), wq.to(dev), ws.to(dev), starts.to(dev),
                                  ends.to(dev), out_dtype=torch.float32)
    _check(out, want, f"grouped {counts}")
    out16 = layers.fp8_grouped_gemm(xq.to(dev), xs.to(dev), wq.to(dev), ws.to(dev), starts.to(dev),
                                    ends.to(dev), out_dtype=torch.bfloat16)
    assert torch.equal(out16.cpu(), out.cpu().to(torch.bfloat16))


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_grouped_gemm_leaves_rows_outside_ranges(kern, dev, out_dtype):
    """Expert ranges with gaps between them (rows no expert covers), a partial last n-tile
    (N = 640) and partial expert tiles: every covered element equals the fp32 result
    rounded to the output type, and every other element of a NaN-filled output stays NaN
    (16-bit outputs take the fixed-count epilogue, whose out-of-tile lanes write elsewhere)."""
    from cinnamon_amd import layers
    N, K = 640, 512
    xq, xs, wq, ws, _, _ = _grouped_case([520, 300, 900, 280], N, K, seed=31)
    starts = torch.tensor([0, 600, 1000, 1900], dtype=torch.int64)
    ends = torch.tensor([420, 870, 1850, 2000], dtype=torch.int64)
    want = orc.grouped_gemm_ref(xq, xs, wq, ws, starts, ends)
    ref32 = layers.fp8_grouped_gemm(xq.to(dev), xs.to(dev), wq.to(dev), ws.to(dev), starts.to(dev),
                                    ends.to(dev), out_dtype=torch.float32)
    out = torch.full((2000, N), float("nan"), dtype=out_dtype, device=dev)
    layers.fp8_grouped_gemm(xq.to(dev), xs.to(dev), wq.to(dev), ws.to(dev), starts.to(dev), ends.to(dev),
                            out_dtype=out_dtype, out=out)
    torch.cuda.synchronize()
    covered = torch.zeros(2000, dtype=torch.bool)
    for s0, s1 in zip(starts.tolist(), ends.tolist()):
        covered[s0:s1] = True
    got = out.cpu()
    assert bool(torch.isnan(got[~covered].float()).all())
    assert torch.equal(got[covered], ref32.cpu()[covered].to(out_dtype))
    _check(ref32.cpu()[covered], want[covered], "grouped with gaps")


def test_grouped_equals_dense_for_one_expert(kern, dev):
    from cinnamon_amd import layers
    xq, xs, wq, ws, starts, ends = _grouped_case([1000], 256, 384, seed=21)
    a = layers.fp8_grouped_gemm(xq.to(dev), xs.to(dev), wq.to(dev), ws.to(dev), starts.to(dev),
                                ends.to(dev), out_dtype=torch.float32)
    b = kern.fp8_gemm_bs(xq.to(dev), xs.to(dev), wq[0].to(dev), ws[0].to(dev), torch.float32)
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gemm_empty_reduction_zeroes_c(dev, dtype):
    """K = 0: C[:M, :N] = 0 (the reference's zero accumulator), written by a kernel; the
    columns past N in each row of a strided C are left alone."""
    from cinnamon_amd import _lib
    M, N, ld = 300, 136, 160
    c = torch.full((M, ld), float("nan"), dtype=dtype, device=dev)
    a = torch.zeros(M, 16, dtype=torch.uint8, device=dev)
    b = torch.zeros(N, 16, dtype=torch.uint8, device=dev)
    s = torch.ones(M, 1, dtype=torch.float32, device=dev)
    _lib.call("cin_gemm_fp8_bs", _lib.ptr(a), 16, _lib.ptr(s), 1, 1, _lib.ptr(b), 16, _lib.ptr(s), 1, 1,
              M, N, 0, _lib.ptr(c), _lib.dtype_code(c), ld, _lib.stream_of(c))
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(c[:, :N].float())) == 0
    assert bool(torch.isnan(c[:, N:].float()).all())


def test_gemm_rows_past_32bit_tile_offsets(kern, dev):
    """Row strides past the 256 x 256 kernel's 32-bit tile offsets (255 * ld + K >= 2^32)
    take the 128 x 128 kernel, which addresses in 64 bits: results within tolerance."""
    M, N, K = 256, 256, 256
    ld = (1 << 24) + 256  # bytes per row of A and of B
    xq, xs, wq, ws = _operands(M, N, K, seed=77)
    a = torch.empty(M, ld, dtype=torch.uint8, device=dev)[:, :K]
    b = torch.empty(N, ld, dtype=torch.uint8, device=dev)[:, :K]
    a.copy_(xq.view(torch.uint8).to(dev))
    b.copy_(wq.view(torch.uint8).to(dev))
    y = kern.fp8_gemm_bs(a.view(torch.float8_e4m3fn), xs.to(dev), b.view(torch.float8_e4m3fn), ws.to(dev),
                         torch.float32)
    torch.cuda.synchronize()
    want = orc.gemm_ref(xq, xs, wq.view(torch.uint8).t().contiguous(), ws.t().contiguous())
    _check(y, want, "gemm with 16 MiB rows")
    del a, b


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("pad", [1, 2, 4])
def test_persistent_gemm_into_strided_c(kern, dev, out_dtype, pad):
    """More tiles than CUs (9 x 29): the persistent walk, whose epilogue depends on C's
    alignment (fixed-count 16-bit or fp32 stores, or direct stores for rows that are not
    aligned).  A C with row stride N + pad gets the same values as a contiguous C, bit for
    bit (same kernel, same K order), and the padding columns are left alone."""
    M, N, K = 2304, 7296, 512
    g = torch.Generator(device=dev).manual_seed(21)
    xq, xs = kern.quantize_fp8_rowwise(torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16))
    wq, ws = kern.quantize_fp8_blockwise((torch.randn(N, K, device=dev, generator=g) * 0.02).to(torch.bfloat16))
    want = kern.fp8_gemm_bs(xq, xs, wq, ws, out_dtype)
    big = torch.full((M, N + pad), 7.0, dtype=out_dtype, device=dev)
    got = kern.fp8_gemm_bs(xq, xs, wq, ws, out_dtype, out=big[:, :N])
    torch.cuda.synchronize()
    assert torch.equal(got, want), f"strided C (ldc = N + {pad}) differs from contiguous C"
    assert bool((big[:, N:] == 7.0).all()), "padding columns were written"


def _bf16_rne_bits(u32):
    """fp32 bit patterns -> bf16 bit patterns: round to nearest even; a NaN keeps its sign
    and upper payload with the quiet bit set (the integer formula the epilogue follows)."""
    u = u32.astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    return np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r).astype(np.uint16)


def _special_scale_patterns():
    """fp32 bit patterns for the row scales: ties below and above an even bf16 mantissa,
    one ulp either side of a tie, fp32 denormals, values next to FLT_MAX (some round to inf
    in bf16), infinities, NaNs with payloads, signed zeros and plain random values."""
    rng = np.random.default_rng(5)
    hi = rng.integers(0, 1 << 16, size=96, dtype=np.uint64) << 16
    pats = []
    for low in (0x8000, 0x7FFF, 0x8001, 0x0000, 0xFFFF):
        pats.append(hi | low)
    pats.append(rng.integers(0x00000001, 0x00800000, size=64, dtype=np.uint64))  # denormals
    pats.append(rng.integers(0x80000001, 0x80800000, size=32, dtype=np.uint64))  # negative denormals
    pats.append(np.array([0x7F7FFFFF, 0x7F7F8000, 0x7F7F7FFF, 0x7F7E8000, 0xFF7FFFFF, 0xFF7F8000,
                          0x7F800000, 0xFF800000, 0x7FC00000, 0x7FC12345, 0xFFC0ABCD, 0x7F812345,
                          0x00000000, 0x80000000, 0x3F808000, 0x3F818000], dtype=np.uint64))
    pats.append(rng.integers(0, 1 << 32, size=400, dtype=np.uint64))
    p = np.concatenate(pats).astype(np.uint32)
    return p


@pytest.mark.parametrize("M,N", [(512, 512), (4352, 4096)])
@pytest.mark.parametrize("path", ["dense_bf16", "grouped_bf16", "grouped_f16"])
def test_gemm_half_output_rounding_special_values(kern, dev, M, N, path):
    """The 16-bit epilogues round the fp32 result exactly as the fp32 output rounded to
    nearest even.  Dense: the one-round LDS-staged tile at 2 x 2 tiles, the persistent
    16-byte stores and its last-tile LDS path at 17 x 16 tiles; grouped (one expert over
    every row): the persistent walk at both sizes, bf16 and fp16.  One K block in which row
    m of A and row n of B hold a single non-zero code, so C[m, n] = b_n * sa[m] with b_n
    mostly a power of two, which carries the chosen scale bit patterns (ties, denormals,
    overflow, NaN payloads) into C unchanged.  bf16: bit-exact against the integer RNE of
    the fp32 output bits, NaN payloads included; fp16: bit-exact against numpy's IEEE
    conversion of the fp32 output, NaNs by position."""
    from cinnamon_amd import layers
    K = 128
    pats = _special_scale_patterns()
    sa_bits = np.resize(pats, M).astype(np.uint32)
    sa = torch.from_numpy(sa_bits.view(np.float32).copy()).reshape(M, 1).to(dev)
    # e4m3 codes of b_n: 1, 2, 0.5, 4, 0.25, -1, 256, 2^-6 (powers of two) and 1.125, 3.5
    codes_b = np.array([0x38, 0x40, 0x30, 0x48, 0x28, 0xB8, 0x78, 0x08, 0x39, 0x46], dtype=np.uint8)
    a = torch.zeros(M, K, dtype=torch.uint8)
    a[:, 0] = 0x38  # 1.0
    b = torch.zeros(N, K, dtype=torch.uint8)
    b[:, 0] = torch.from_numpy(np.resize(codes_b, N))
    sb = torch.ones(N // 128, 1, device=dev)
    a8, b8 = a.view(torch.float8_e4m3fn).to(dev), b.view(torch.float8_e4m3fn).to(dev)
    out_dtype = torch.float16 if path == "grouped_f16" else torch.bfloat16
    if path == "dense_bf16":
        y32 = kern.fp8_gemm_bs(a8, sa, b8, sb, torch.float32)
        y16 = kern.fp8_gemm_bs(a8, sa, b8, sb, out_dtype)
    else:
        starts = torch.zeros(1, dtype=torch.int64, device=dev)
        ends = torch.full((1,), M, dtype=torch.int64, device=dev)
        w8, ws = b8.unsqueeze(0).contiguous(), sb.unsqueeze(0).contiguous()
        y32 = layers.fp8_grouped_gemm(a8, sa, w8, ws, starts, ends, out_dtype=torch.float32)
        y16 = layers.fp8_grouped_gemm(a8, sa, w8, ws, starts, ends, out_dtype=out_dtype)
    torch.cuda.synchronize()
    f32 = y32.cpu().numpy()
    u32 = f32.view(np.uint32)
    # the construction reached the cases it is meant to reach
    assert int(((u32 & 0xFFFF) == 0x8000).sum()) > 1000, "no exact bf16 ties in C"
    assert int(((np.abs(f32) < np.float32(1.1754944e-38)) & (f32 != 0)).sum()) > 100, "no denormals in C"
    assert bool(np.isnan(f32).any()) and bool(np.isinf(f32).any())
    got = y16.cpu().view(torch.int16).numpy().view(np.uint16)
    if out_dtype == torch.bfloat16:
        want = _bf16_rne_bits(u32)
        bad = np.argwhere(got != want)
        if bad.size:
            r, c = bad[0]
            raise AssertionError(f"{len(bad)} bf16 values differ from RNE; first at ({r}, {c}): fp32 "
                                 f"{u32[r, c]:08x} got {got[r, c]:04x} want {want[r, c]:04x}")
    else:
        with np.errstate(over="ignore"):  # values past fp16's range become inf, as intended
            want16 = f32.astype(np.float16)
        nan = np.isnan(want16)
        assert bool((np.isnan(got.view(np.float16)) == nan).all()), "fp16 NaN positions differ"
        bad = np.argwhere((got != want16.view(np.uint16)) & ~nan)
        if bad.size:
            r, c = bad[0]
            raise AssertionError(f"{len(bad)} fp16 values differ from RNE; first at ({r}, {c}): fp32 "
                                 f"{u32[r, c]:08x} got {got[r, c]:04x} want {want16.view(np.uint16)[r, c]:04x}")
