"""CPU oracle: a torch-CPU restatement of the reference FP8 path (shyampathak22/cinnamon,
src/kernels.py) used as the parity checker.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the checker (or the timed CPU
baseline), never as the thing measured or shipped.  The product path
(cinnamon_amd) never calls it.

Third-party arithmetic the reference relies on (not vendored in /root/reference):
  * Triton 3.5.1 (uv.lock:2385-2386): tl.max widens bf16/fp16 tiles to fp32 before
    reducing (language/standard.py, max) and tl.maximum promotes both operands, so
    tl.maximum(tl.max(tl.abs(x)), 1e-4) floors at fp32(1e-4) for every input dtype;
    tl.maximum / tl.minimum / tl.max lower to maxnum (NaN ignored); fp32 '/' is IEEE
    division.
  * torch 2.9.1 (uv.lock:2308-2309): the float8_e4m3fn dtype and its RNE cast;
    torch.log2 (used for round_scale).
Both are pinned by tests/test_oracle.py: the floor against scales and codes that
Triton's own interpreter produced for zero and tiny bf16/fp16/fp32 tiles
(tests/golden/triton_floor.npz, written by tests/golden/gen_triton_floor.py), the
cast against a textbook OCP e4m3fn round-to-nearest-even (e4m3_rne_np, written from
the OCP FP8 spec), and log2 by enumeration against a correctly rounded fp32 log2.

Functions and the reference lines they restate:
  quant_rowwise           src/kernels.py:38-71   (+ wrapper :178-216)
  quant_blockwise         src/kernels.py:94-132  (+ wrapper :219-259)
  dequant_rowwise         src/kernels.py:262-281
  dequant_block_bf16      src/kernels.py:149-173, :284-314
  gemm_ref                src/kernels.py:618-664 as dequantize-then-fp32-matmul
  fp8_linear_ref          src/kernels.py:739-794 (FP8MatmulFunction fwd/bwd)
  grouped_gemm_ref        src/layers.py:79-86 loop semantics on FP8 operands
  moe_dispatch_ref        src/layers.py:133-148 (sort, token_indices, bincount, cumsum)
  moe_combine_ref         src/layers.py:151-154 (gated scatter_add_ of sorted rows)
  indexer_scores_fp8_ref  src/attention.py:288-300 (DSA indexer scoring on FP8 q / k)
The MoE functions are pinned by tests/test_oracle_moe.py; indexer_scores_fp8_ref by
tests/test_oracle_indexer.py (the reference's non-FP8 formula on lossless inputs, the
first-scale rule, the ReLU, power-of-two homogeneity).
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
    """fp32(1e-4) for every input dtype (src/kernels.py:53, :114 under Triton typing:
    the tile amax of a bf16/fp16 tile is already fp32 when it meets the floor)."""
    del dtype
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


def grouped_gemm_f16_ref(a: torch.Tensor, w: torch.Tensor, starts, ends) -> torch.Tensor:
    """Unquantized grouped GEMM of the reference (src/kernels.py:440-523): operands rounded
    to fp16 (a.to(tl.float16), b.to(tl.float16)), exact products summed in fp64 here.
    Returns the fp64 result [T, N] before the fp16 store; rows outside every range are 0."""
    T, K = a.shape
    E, N, _ = w.shape
    out = torch.zeros(T, N, dtype=torch.float64)
    a16 = a.to(torch.float16).double()
    for e, s, t in expert_slices(starts, ends, T):
        if t > s:
            out[s:t] = a16[s:t] @ w[e].to(torch.float16).double().t()
    return out


# ---------------------------------------------------------------------------
# Grouped (MoE) backward: the FP8MatmulFunction.backward recipe (src/kernels.py:763-794)
# applied to each expert's row slice.  The reference has no grouped backward, so these
# are defined here and pinned by the dense chain (one expert covering every row is the
# dense backward) and by per-expert brute force in the tests.
# ---------------------------------------------------------------------------
def expert_slices(starts, ends, T):
    """[(e, s, t)] with the range clamped to [0, T) (empty ranges have t == s)."""
    out = []
    for e in range(len(starts)):
        s = min(max(int(starts[e]), 0), T)
        t = min(max(int(ends[e]), s), T)
        out.append((e, s, t))
    return out


def padded_offsets(starts, ends, T):
    """Padded token-axis offset p_e and chunk count of each expert (128-token chunks)."""
    p, offs = 0, []
    for e, s, t in expert_slices(starts, ends, T):
        n = -(-(t - s) // 128)
        offs.append((p, n))
        p += 128 * n
    return offs


def grouped_dual_ref(dc: torch.Tensor, starts, ends, round_scale: bool = False):
    """Per expert: (codes, scales) of quant_rowwise(dC[s:t]) (the dgrad operand, rows
    s..t-1) and of quant_rowwise(dC[s:t].t().contiguous()) (the wgrad operand)."""
    out = []
    for e, s, t in expert_slices(starts, ends, dc.shape[0]):
        if t == s:
            out.append(None)
            continue
        rq, rs = quant_rowwise(dc[s:t], 128, round_scale)                      # :771
        tq, ts = quant_rowwise(dc[s:t].t().contiguous(), 128, round_scale)     # :781-783
        out.append((rq, rs, tq, ts))
    return out


def grouped_requant_ref(x_codes: torch.Tensor, x_scales: torch.Tensor, starts, ends):
    """Per expert: quant_blockwise(dequant_rowwise(x)[s:t]) (src/kernels.py:784-787)."""
    xd = dequant_rowwise(x_codes, x_scales, 128)
    out = []
    for e, s, t in expert_slices(starts, ends, x_codes.shape[0]):
        out.append(None if t == s else quant_blockwise(xd[s:t], 128, 128, False))
    return out


def grouped_dgrad_ref(g_codes, g_scales, w_codes, w_scales, starts, ends) -> torch.Tensor:
    """dA[s:t] = dC[s:t] . W_e on dequantized operands (src/kernels.py:774 per expert).
    w_codes [E, N, K], w_scales [E, N/128, K/128]; fp32 [T, K], 0 outside every range."""
    T = g_codes.shape[0]
    E, N, K = w_codes.shape
    out = torch.zeros(T, K, dtype=torch.float32)
    for e, s, t in expert_slices(starts, ends, T):
        if t > s:
            out[s:t] = gemm_ref(g_codes[s:t], g_scales[s:t], w_codes[e], w_scales[e])
    return out


def grouped_wgrad_ref(dual, requant, E, N, K) -> torch.Tensor:
    """dW_e = dC_e^T . Xb_e (src/kernels.py:788 per expert) from grouped_dual_ref and
    grouped_requant_ref outputs; fp32 [E, N, K], zeros for experts without rows."""
    out = torch.zeros(E, N, K, dtype=torch.float32)
    for e in range(E):
        if dual[e] is not None:
            _, _, tq, ts = dual[e]
            xb, xbs = requant[e]
            out[e] = gemm_ref(tq, ts, xb, xbs)
    return out


def grouped_experts_ref(x: torch.Tensor, w12: torch.Tensor, w3: torch.Tensor, starts, ends,
                        g_out: torch.Tensor | None = None, quantize: bool = True) -> dict:
    """FP8 SwiGLU experts (src/layers.py:69-75 with FP8 GEMMs), forward and backward.

    x [T, D], w12 [E, 2H, D], w3 [E, D, H] (fp32 masters), g_out [T, D] fp32.  Every GEMM
    is dequantize-then-fp32-matmul (gemm_ref) on operands quantized as the device path
    does: activations and gradients 1x128 row-wise, weights 128x128, the wgrad operands
    per expert (gradient 128x1 column tiles, inputs re-quantized to 128x128 blocks of the
    dequantized row-wise codes); h12 is rounded to bf16 as the device stores it.  With
    quantize=False every quantization (and the bf16 rounding) is the identity, which
    turns this into plain fp32 SwiGLU experts and their exact gradients.
    Returns fp32 out [T, D] and, with g_out, dx [T, D], dw12 [E, 2H, D], dw3 [E, D, H].
    """
    T, D = x.shape
    E, H2, _ = w12.shape
    H = H2 // 2
    if quantize:
        rowq = lambda t: dequant_rowwise(*quant_rowwise(t))                       # noqa: E731
        blkq = lambda t: dequant_block(*quant_blockwise(t))                       # noqa: E731
        colq = lambda t: dequant_rowwise(*quant_rowwise(t.t().contiguous())).t()  # noqa: E731
        bf16 = lambda t: t.to(torch.bfloat16).float()                             # noqa: E731
    else:
        rowq = blkq = colq = bf16 = lambda t: t.float()                           # noqa: E731
    sl = [(s, t) for _, s, t in expert_slices(starts, ends, T)]
    r = {}
    xd = rowq(x)
    w12d = blkq(w12.float().reshape(E * H2, D)).view(E, H2, D)
    w3d = blkq(w3.float().reshape(E * D, H)).view(E, D, H)
    h12 = torch.zeros(T, H2)
    for e, (s, t) in enumerate(sl):
        if t > s:
            h12[s:t] = bf16(xd[s:t] @ w12d[e].t())
    h1, h2 = h12[:, :H], h12[:, H:]
    h = (torch.nn.functional.silu(h1) * h2).to(x.dtype)
    hd = rowq(h)
    out = torch.zeros(T, D)
    for e, (s, t) in enumerate(sl):
        if t > s:
            out[s:t] = hd[s:t] @ w3d[e].t()
    r["out"] = out
    if g_out is None:
        return r
    g_row = rowq(g_out)
    dh = torch.zeros(T, H)
    r["dw3"] = torch.zeros(E, D, H)
    for e, (s, t) in enumerate(sl):
        if t > s:
            dh[s:t] = g_row[s:t] @ w3d[e]                                    # dgrad (:774)
            r["dw3"][e] = colq(g_out[s:t]).t() @ blkq(hd[s:t])              # wgrad (:781-788)
    sig = torch.sigmoid(h1)
    dh12 = torch.cat([dh * h2 * (sig * (1.0 + h1 * (1.0 - sig))), dh * (h1 * sig)], dim=-1)
    d_row = rowq(dh12)
    r["dx"] = torch.zeros(T, D)
    r["dw12"] = torch.zeros(E, H2, D)
    for e, (s, t) in enumerate(sl):
        if t > s:
            r["dx"][s:t] = d_row[s:t] @ w12d[e]
            r["dw12"][e] = colq(dh12[s:t]).t() @ blkq(xd[s:t])
    return r


# ---------------------------------------------------------------------------
# DSA indexer scoring in FP8 (reference src/attention.py:288-300)
# ---------------------------------------------------------------------------
def indexer_scores_fp8_ref(q: torch.Tensor, k: torch.Tensor, weights: torch.Tensor,
                           softmax_scale: float) -> torch.Tensor:
    """The reference's FP8 index scores (src/attention.py:288-300) on the CPU:
    q [B, L, H, d], k [B, S, d] quantized row-wise in 1x128 tiles (the first scale of each
    row is used, :296-297), logits = einsum('bthd,bsd->bths') of the codes in fp32,
    relu(logits) * (q_scale * weights * softmax_scale), summed over the heads, times
    k_scale.  weights [B, L, H] fp32.  Returns scores [B, L, S] fp32 (before the mask)."""
    B, L, H, d = q.shape
    S = k.shape[1]
    q_fp8, q_scale = quant_rowwise(q.reshape(-1, d).contiguous(), block_size=128)
    k_fp8, k_scale = quant_rowwise(k.reshape(-1, d).contiguous(), block_size=128)
    q_fp8 = q_fp8.view(B, L, H, d)
    k_fp8 = k_fp8.view(B, S, d)
    q_scale = q_scale.view(B, L, H, -1)[..., 0]
    k_scale = k_scale.view(B, S, -1)[..., 0]
    logits = torch.einsum('bthd,bsd->bths', q_fp8.float(), k_fp8.float())
    logits = torch.relu(logits) * (q_scale * weights * softmax_scale).unsqueeze(-1)
    return logits.sum(dim=2) * k_scale.unsqueeze(1)


# ---------------------------------------------------------------------------
# MoE dispatch / combine (reference src/layers.py:126-157)
# ---------------------------------------------------------------------------
def moe_dispatch_ref(top_idx: torch.Tensor, n_experts: int):
    """The reference's routing bookkeeping (src/layers.py:133-148) on the CPU:
    expanded_idx = top_idx.view(-1); sorted_idx, sort_order = expanded_idx.sort();
    token_indices = sort_order // top_k; expert_counts = bincount; expert_ends = cumsum;
    expert_starts = [0, ends[:-1]].  The sort is the stable one (the reference's torch.sort
    may order equal ids differently; the build's device sort is stable).
    Returns (sort_order, token_indices, counts, starts, ends), all int64."""
    k = top_idx.shape[1]
    expanded_idx = top_idx.reshape(-1).to(torch.int64)
    _, sort_order = torch.sort(expanded_idx, stable=True)
    token_indices = sort_order // k
    counts = torch.bincount(expanded_idx, minlength=n_experts)
    ends = counts.cumsum(0)
    starts = torch.cat([torch.zeros(1, dtype=torch.long), ends[:-1]])
    return sort_order, token_indices, counts, starts, ends


def moe_combine_ref(sorted_out: torch.Tensor, top_scores: torch.Tensor, sort_order: torch.Tensor,
                    n_tokens: int) -> torch.Tensor:
    """The reference's gated combine (src/layers.py:137,151-154): sorted_scores =
    top_scores.view(-1)[sort_order]; weighted_out = sorted_out * sorted_scores[:, None];
    routed_out = zeros(n_tokens, d, dtype=weighted_out.dtype).scatter_add_(0,
    token_indices[:, None].expand_as(weighted_out), weighted_out).  On the CPU, scatter_add_
    adds the rows in index order, i.e. each token's terms in increasing sorted position."""
    k = top_scores.shape[1]
    sorted_scores = top_scores.reshape(-1)[sort_order]
    token_indices = sort_order // k
    weighted_out = sorted_out * sorted_scores[:, None]
    out = torch.zeros(n_tokens, sorted_out.shape[1], dtype=weighted_out.dtype)
    out.scatter_add_(0, token_indices.unsqueeze(1).expand_as(weighted_out), weighted_out)
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
