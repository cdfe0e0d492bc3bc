"""CPU oracle: a torch-CPU restatement of the reference FP8 path (shyampathak22/cinnamon,
src/kernels.py) used as the parity checker.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the checker (or the timed CPU
baseline), never as the thing measured or shipped.  The product path
(cinnamon_amd) never calls it.

Third-party arithmetic the reference relies on (not vendored in /root/reference):
  * Triton 3.5.1 (uv.lock:2385-2386): scalar type promotion makes
    tl.maximum(bf16_tile, 1e-4) a bf16 op (floor = bf16(1e-4)) while tl.maximum /
    tl.minimum / tl.max lower to maxnum (NaN ignored); fp32 '/' is IEEE division.
  * torch 2.9.1 (uv.lock:2308-2309): the float8_e4m3fn dtype and its RNE cast;
    torch.log2 (used for round_scale).
Both are pinned by tests/test_oracle.py: the cast against a textbook OCP e4m3fn
round-to-nearest-even (e4m3_rne_np, written from the OCP FP8 spec), and log2 by
enumeration against a correctly rounded fp32 log2.

Functions and the reference lines they restate:
  quant_rowwise           src/kernels.py:38-71   (+ wrapper :178-216)
  quant_blockwise         src/kernels.py:94-132  (+ wrapper :219-259)
  dequant_rowwise         src/kernels.py:262-281
  dequant_block_bf16      src/kernels.py:149-173, :284-314
  gemm_ref                src/kernels.py:618-664 as dequantize-then-fp32-matmul
  fp8_linear_ref          src/kernels.py:739-794 (FP8MatmulFunction fwd/bwd)
  grouped_gemm_ref        src/layers.py:79-86 loop semantics on FP8 operands
"""
from __future__ import annotations

import numpy as np
import torch

FP8_MAX = 448.0
_FP8_MAX_T = torch.tensor(FP8_MAX, dtype=torch.float32)


# ---------------------------------------------------------------------------
# Scalar semantics
# ---------------------------------------------------------------------------
def amax_floor(dtype: torch.dtype) -> torch.Tensor:
    """1e-4 in the input dtype, widened to fp32 (src/kernels.py:53, :114 under Triton typing)."""
    if dtype in (torch.bfloat16, torch.float16):
        return torch.tensor(1e-4, dtype=dtype).float()
    return torch.tensor(1e-4, dtype=torch.float32)


def scale_from_amax(amax: torch.Tensor, round_scale: bool) -> torch.Tensor:
    """src/kernels.py:54-57 / :115-118 in fp32."""
    v = amax / _FP8_MAX_T
    if round_scale:
        v = torch.exp2(torch.ceil(torch.log2(v)))
    return v


def _quantize_tiles(t: torch.Tensor, floor: torch.Tensor, round_scale: bool):
    """t: [..., tile] fp32 (zero padded).  Returns (codes uint8 [..., tile], scales [...])."""
    a = t.abs()
    a = torch.where(torch.isnan(a), torch.zeros_like(a), a)  # maxnum reduction ignores NaN
    amax = torch.fmax(a.amax(dim=-1), floor)                 # tl.maximum(abs_max, 1e-4)
    s = scale_from_amax(amax, round_scale)
    y = t / s.unsqueeze(-1)                                   # IEEE fp32 division
    y = torch.fmin(torch.fmax(y, -_FP8_MAX_T), _FP8_MAX_T)     # maxnum/minnum clamp: NaN -> -448
    return y.to(torch.float8_e4m3fn).view(torch.uint8), s


# ---------------------------------------------------------------------------
# Quantizers
# ---------------------------------------------------------------------------
def quant_rowwise(x: torch.Tensor, block_size: int = 128, round_scale: bool = False):
    """(codes float8_e4m3fn [M, N], scales fp32 [M, ceil(N/bs)])  — src/kernels.py:38-71."""
    M, N = x.shape
    nb = -(-N // block_size)
    floor = amax_floor(x.dtype)
    xf = x.float()
    pad = nb * block_size - N
    if pad:
        xf = torch.nn.functional.pad(xf, (0, pad))  # masked loads read 0.0
    codes, s = _quantize_tiles(xf.view(M, nb, block_size), floor, round_scale)
    codes = codes.view(M, nb * block_size)[:, :N].contiguous()
    return codes.view(torch.float8_e4m3fn), s.contiguous()


def quant_blockwise(x: torch.Tensor, block_m: int = 128, block_n: int = 128,
                    round_scale: bool = False):
    """(codes [M, N], scales [ceil(M/bm), ceil(N/bn)])  — src/kernels.py:94-132."""
    M, N = x.shape
    nbm, nbn = -(-M // block_m), -(-N // block_n)
    floor = amax_floor(x.dtype)
    xf = torch.nn.functional.pad(x.float(), (0, nbn * block_n - N, 0, nbm * block_m - M))
    tiles = xf.view(nbm, block_m, nbn, block_n).permute(0, 2, 1, 3).reshape(nbm, nbn, block_m * block_n)
    codes, s = _quantize_tiles(tiles, floor, round_scale)
    codes = codes.view(nbm, nbn, block_m, block_n).permute(0, 2, 1, 3).reshape(nbm * block_m, nbn * block_n)
    return codes[:M, :N].contiguous().view(torch.float8_e4m3fn), s.contiguous()


# ---------------------------------------------------------------------------
# Dequantizers
# ---------------------------------------------------------------------------
def dequant_rowwise(codes: torch.Tensor, scales: torch.Tensor, block_size: int = 128) -> torch.Tensor:
    """fp32(code) * scale[row, col // bs] in fp32  — src/kernels.py:262-281."""
    M, N = codes.shape
    idx = torch.arange(N) // block_size
    return codes.view(torch.float8_e4m3fn).float() * scales[:, idx]


def dequant_block(codes: torch.Tensor, scales: torch.Tensor, block_m: int = 128,
                  block_n: int = 128) -> torch.Tensor:
    """fp32(code) * scale[row // bm, col // bn] in fp32 (the fp32 value before the bf16 store)."""
    M, N = codes.shape
    ri = torch.arange(M) // block_m
    ci = torch.arange(N) // block_n
    nbn = -(-N // block_n)
    flat = scales.reshape(-1)
    s = flat[(ri[:, None] * nbn + ci[None, :]).reshape(-1)].view(M, N)
    return codes.view(torch.float8_e4m3fn).float() * s


def dequant_block_bf16(codes, scales, block_m=128, block_n=128) -> torch.Tensor:
    """src/kernels.py:168-173: bf16 RNE of the fp32 product."""
    return dequant_block(codes, scales, block_m, block_n).to(torch.bfloat16)


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------
def gemm_ref(a_codes, a_scales, b_codes_kn, b_scales_kn, dtype=torch.float32) -> torch.Tensor:
    """Dequantize-then-matmul oracle of fp8_gemm_kernel (src/kernels.py:618-664).

    a_codes [M, K] with row-wise scales [M, ceil(K/128)]; b_codes_kn [K, N] with block
    scales [ceil(K/128), ceil(N/128)].  Returns the unrounded product in `dtype`.
    """
    a = dequant_rowwise(a_codes, a_scales, 128).to(dtype)
    K, N = b_codes_kn.shape
    b = dequant_block(b_codes_kn, b_scales_kn, 128, 128).to(dtype)
    return a @ b


def normwise_max_rel(got: torch.Tensor, want: torch.Tensor) -> float:
    """max|got - want| / max|want| (0 if want is all zero and got equals it)."""
    got, want = got.double(), want.double()
    den = want.abs().max().item()
    num = (got - want).abs().max().item()
    return num / den if den > 0 else num


def frob_rel(got: torch.Tensor, want: torch.Tensor) -> float:
    got, want = got.double(), want.double()
    den = torch.linalg.vector_norm(want).item()
    num = torch.linalg.vector_norm(got - want).item()
    return num / den if den > 0 else num


# ---------------------------------------------------------------------------
# FP8MatmulFunction forward/backward (src/kernels.py:739-794)
# ---------------------------------------------------------------------------
def fp8_linear_ref(x: torch.Tensor, w: torch.Tensor, dy: torch.Tensor | None,
                   round_scale: bool = False) -> dict:
    """The reference forward and backward operand chain, with fp32 GEMMs.

    x [M, K] (bf16/fp32), w [N, K] (master weights, quantized as w.float()),
    dy [M, N].  Returns a dict with every intermediate code/scale tensor and the fp32
    values y [M, N], dx [M, K], dw [N, K] before their bf16 rounding.
    """
    out = {}
    x_fp8, x_s = quant_rowwise(x, 128, round_scale)                        # :746
    w_fp8, w_s = quant_blockwise(w.float(), 128, 128, False)               # :747
    out.update(x_fp8=x_fp8, x_scale=x_s, w_fp8=w_fp8, w_scale=w_s)
    out["y"] = gemm_ref(x_fp8, x_s, w_fp8.view(torch.uint8).t().contiguous(), w_s.t().contiguous())  # :748-752
    if dy is None:
        return out
    g_fp8, g_s = quant_rowwise(dy, 128, round_scale)                       # :771
    out.update(g_fp8=g_fp8, g_scale=g_s)
    out["dx"] = gemm_ref(g_fp8, g_s, w_fp8, w_s)                           # :774
    g_fp8_t, g_s_t = quant_rowwise(dy.t().contiguous(), 128, round_scale)  # :781-783
    x_deq = dequant_rowwise(x_fp8, x_s, 128)                               # :784
    xb_fp8, xb_s = quant_blockwise(x_deq, 128, 128, False)                 # :785-787
    out.update(g_fp8_t=g_fp8_t, g_scale_t=g_s_t, xb_fp8=xb_fp8, xb_scale=xb_s)
    out["dw"] = gemm_ref(g_fp8_t, g_s_t, xb_fp8, xb_s)                     # :788
    return out


# ---------------------------------------------------------------------------
# Grouped GEMM (src/layers.py:79-86 loop semantics, FP8 operands)
# ---------------------------------------------------------------------------
def grouped_gemm_ref(a_codes, a_scales, w_codes, w_scales, starts, ends) -> torch.Tensor:
    """Per-expert block-scaled product on dequantized operands.

    a_codes [T, K] row-wise quantized (scales [T, ceil(K/128)]); w_codes [E, N, K] with
    per-expert 128x128 block scales w_scales [E, ceil(N/128), ceil(K/128)].  Rows
    outside every expert range are returned as 0.  Output fp32 [T, N].
    """
    T, K = a_codes.shape
    E, N, _ = w_codes.shape
    a = dequant_rowwise(a_codes, a_scales, 128)
    out = torch.zeros(T, N, dtype=torch.float32)
    for e in range(E):
        s, t = int(starts[e]), int(ends[e])
        if t > s:
            we = dequant_block(w_codes[e], w_scales[e], 128, 128)
            out[s:t] = a[s:t] @ we.t()
    return out


# ---------------------------------------------------------------------------
# Textbook OCP e4m3fn round-to-nearest-even (numpy; independent of torch)
# ---------------------------------------------------------------------------
def e4m3_rne_np(x: np.ndarray) -> np.ndarray:
    """OCP FP8 E4M3FN encoding of fp32 values with RNE and NaN for |x| >= 464 or NaN.

    Written from the OCP 8-bit floating point specification (bias 7, 3 mantissa bits,
    subnormal step 2^-9, max finite 448 = S.1111.110, NaN = S.1111.111, no infinities).
    """
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    sign = ((u >> 24) & 0x80).astype(np.uint8)
    a = u & np.uint32(0x7FFFFFFF)
    out = np.zeros(a.shape, dtype=np.uint32)
    nan = a > 0x7F800000
    big = (a > 0x43E80000) & ~nan            # > 464: rounds past 448 -> NaN (non-saturating)
    sub = a < 0x3C800000                      # < 2^-6: e4m3 subnormal range
    norm = ~(nan | big | sub)
    an = a[norm]
    r = (an + np.uint32(0x7FFFF) + ((an >> 20) & 1)) >> 20
    out[norm] = r - np.uint32(960)            # (127 - 7) << 3
    # subnormals: round(|x| * 2^9) to nearest even integer in [0, 8]
    t = a[sub].view(np.float32).astype(np.float64) * 512.0
    out[sub] = np.rint(t).astype(np.uint32)   # rint = round half to even
    out[nan | big] = 0x7F
    return (out.astype(np.uint8) | sign)
