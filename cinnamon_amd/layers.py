"""FP8 routed-expert layer for MI355X: grouped GEMM over experts in one launch.

Counterpart of the reference's moe_grouped_gemm (src/kernels.py:526-581) and
GroupedExperts (src/layers.py:34-87).  The reference grouped GEMM computes in fp16;
this module runs it in FP8 with the reference's quantization recipe (1x128
activation tiles, 128x128 weight blocks per expert) and the reference's per-expert
loop semantics (src/layers.py:79-86).
"""
from __future__ import annotations

import torch

from ._lib import call, dtype_code, ptr, stream_of
from .kernels import _cdiv, _kcontig, _require


def fp8_grouped_gemm(a_codes: torch.Tensor, a_scales: torch.Tensor, w_codes: torch.Tensor,
                     w_scales: torch.Tensor, expert_starts: torch.Tensor,
                     expert_ends: torch.Tensor, out_dtype: torch.dtype = torch.bfloat16,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """out[r] = A[r] x W_e^T for every row r in [starts[e], ends[e]), all experts in one launch.

    a_codes [T, K] e4m3 (1x128 scales a_scales [T, ceil(K/128)]), w_codes [E, N, K] e4m3
    (per-expert 128x128 block scales w_scales [E, ceil(N/128), ceil(K/128)]), expert
    ranges as int64 device tensors (no host sync).  Rows outside every range are left
    untouched (as in the reference, whose output is torch.empty).
    """
    _require(a_codes.is_cuda and w_codes.is_cuda, "Input must be on CUDA")
    T, K = a_codes.shape
    E, N, K2 = w_codes.shape
    _require(K == K2, f"Dimension mismatch: {K} vs {K2}")
    _require(K % 16 == 0, "grouped GEMM needs K % 16 == 0")
    aq, _ = _kcontig(a_codes, K)
    wq = w_codes.view(torch.uint8) if w_codes.dtype == torch.float8_e4m3fn else w_codes
    if wq.stride(2) != 1 or wq.stride(1) % 16 or wq.stride(0) % 16 or wq.data_ptr() % 16:
        wq = wq.contiguous()
    _require(w_scales.shape[0] == E and w_scales.shape[1] >= _cdiv(N, 128)
             and w_scales.shape[2] >= _cdiv(K, 128), "w_scales must be [E, ceil(N/128), ceil(K/128)]")
    starts = expert_starts.to(torch.int64)
    ends = expert_ends.to(torch.int64)
    _require(starts.numel() == E and ends.numel() == E, "expert ranges must have E entries")
    if out is None:
        out = torch.empty((T, N), dtype=out_dtype, device=a_codes.device)
    _require(out.stride(1) == 1, "out must have unit column stride")
    call("cin_grouped_gemm_fp8", ptr(aq), aq.stride(0), ptr(a_scales), a_scales.stride(0),
         a_scales.stride(1), ptr(wq), wq.stride(0), wq.stride(1), ptr(w_scales),
         w_scales.stride(0), w_scales.stride(1), w_scales.stride(2), ptr(starts), ptr(ends), E, T,
         N, K, ptr(out), dtype_code(out), out.stride(0), stream_of(aq))
    return out
