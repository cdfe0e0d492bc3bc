"""Drop-in replacement of the reference's FP8 ``kernels`` module for MI355X.

Same public names, signatures, defaults, output dtypes/shapes and argument
checks as reference src/kernels.py; every operator launches hand-written HIP
kernels (gfx950) through the C ABI in include/cinnamon_fp8.h.  There is no
Triton and no fallback: device tensors are required exactly where the reference
requires CUDA tensors, and a missing native library raises.  The one CPU path is
the reference's own: dequantize_fp8_rowwise is plain torch there (:262-281) and runs
on CPU tensors here too.

Replaced reference items (src/kernels.py):
  quantize_fp8_rowwise      :178-216  -> cin_quant_rowwise
  quantize_fp8_blockwise    :219-259  -> cin_quant_blockwise
  dequantize_fp8_rowwise    :262-281  -> cin_dequant (fp32 out)
  dequantize_fp8            :284-314  -> cin_dequant (bf16 out)
  fp8_matmul_dsv3           :667-702  -> cin_gemm_fp8_bs
  FP8MatmulFunction         :731-794  -> cin_quant_fwd + cin_quant_dual + cin_requant_row_to_block + GEMMs
  FP8Linear                 :797-840
  convert_to_fp8            :843-905
  moe_grouped_gemm          :526-581  -> cin_grouped_gemm_f16 (unquantized, fp16 MFMA)

Every launch is registered as a torch operator (namespace ``cinnamon_amd``) with a
shape function, so torch.compile traces through these functions (the reference
compiles its training model, src/train.py:703) instead of breaking the graph at a
native call; the public functions keep the reference's argument checks in front.

Two reference names outside the FP8 path are kept so that imports resolve
(src/attention.py:6, tests/test_kernels.py:14): lightning_indexer_fused (:392-432) and
sparse_attention (:1292-1320).  They are plain torch on the GPU, not part of this build's
kernels.
"""
from __future__ import annotations

import torch
from torch.utils._python_dispatch import _get_current_dispatch_mode

from . import _lib
from ._lib import call, dtype_code, ptr, stream_of

FP8_E4M3_MAX = 448.0

__all__ = [
    "FP8_E4M3_MAX",
    "quantize_fp8_rowwise",
    "quantize_fp8_blockwise",
    "dequantize_fp8_rowwise",
    "dequantize_fp8",
    "fp8_matmul_dsv3",
    "fp8_gemm_bs",
    "quantize_fp8_forward",
    "quantize_fp8_dual",
    "quantize_fp8_backward",
    "requantize_rowwise_to_blockwise",
    "FP8MatmulFunction",
    "FP8Linear",
    "convert_to_fp8",
    "set_weight_cache",
    "indexer_scores_fp8",
    "moe_grouped_gemm",
    "lightning_indexer_fused",
    "sparse_attention",
]


# operator -> the launch function it was made from (see _run)
_LAUNCH: dict = {}


def custom_op(name: str, schema: str):
    """Register the decorated launch as the torch operator cinnamon_amd::<name> with an
    explicit schema; the caller attaches its shape function with ``register_fake``.  The
    operators allocate their outputs and never mutate their inputs."""
    def deco(fn):
        op = torch.library.custom_op(f"cinnamon_amd::{name}", fn, mutates_args=(), schema=schema)
        _LAUNCH[op] = fn
        return op
    return deco


def _plain_eager(*tensors) -> bool:
    """True outside tracing: no torch.compile, no dispatch mode (FakeTensor, make_fx,
    functionalization), no functorch transform, and plain tensors."""
    return (not torch.compiler.is_compiling() and _get_current_dispatch_mode() is None
            and not torch._C._are_functorch_transforms_active()
            and all(type(t) is torch.Tensor for t in tensors))


def _run(op, *args):
    """op(*args); in plain eager mode its launch function is called directly instead: the
    same kernels on the same arguments, without torch's dispatcher, whose host cost per call
    exceeds the device time of a small launch.  Only for operators without an autograd
    formula (these run inside the autograd Functions, or where no gradient is defined)."""
    if _plain_eager(*(a for a in args if isinstance(a, torch.Tensor))):
        return _LAUNCH[op](*args)
    return op(*args)


def _require(cond: bool, msg: str) -> None:
    # The reference checks these conditions with `assert`; keep AssertionError.
    if not cond:
        raise AssertionError(msg)


def _cdiv(a: int, b: int) -> int:
    return (a + b - 1) // b


def _codes_u8(t: torch.Tensor) -> torch.Tensor:
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8)
    _require(t.dtype == torch.uint8, f"expected float8_e4m3fn codes, got {t.dtype}")
    return t


def _scales_2d(sc: torch.Tensor) -> torch.Tensor:
    """A 2-D fp32 scale tensor the kernels can address with (row, column) strides: itself
    when it is row-major (unit column stride, rows not overlapping) or column-major (unit row
    stride), else a row-major copy."""
    R, C = sc.shape
    if sc.dtype == torch.float32 and ((sc.stride(1) == 1 and sc.stride(0) >= max(C, 1)) or
                                      (sc.stride(0) == 1 and sc.stride(1) >= max(R, 1))):
        return sc
    return sc.to(torch.float32).contiguous()


def _rows8(q: torch.Tensor) -> torch.Tensor:
    """2-D uint8 codes with unit column stride and 8-byte aligned rows (the tile kernels
    read 8 codes at a time): q itself when it qualifies, else a copy whose rows are padded
    to a multiple of 8 bytes."""
    if q.stride(1) == 1 and q.stride(0) % 8 == 0 and q.data_ptr() % 8 == 0:
        return q
    M, K = q.shape
    buf = torch.empty((M, _cdiv(max(K, 1), 8) * 8), dtype=torch.uint8, device=q.device)
    buf[:, :K].copy_(q)
    return buf[:, :K]


# ---------------------------------------------------------------------------
# Quantization (reference src/kernels.py:178-259)
# ---------------------------------------------------------------------------
def _scale_buf(like: torch.Tensor, rows: int, cols: int, col_major: bool) -> torch.Tensor:
    """An fp32 [rows, cols] scale tensor, row-major (the reference's layout) or column-major
    (strides (1, rows): the scales of one 128-column block of consecutive rows side by
    side, which the GEMM reads as one run per K block).  ``like`` gives the device (or the
    fake-tensor mode)."""
    if col_major:
        return like.new_empty((cols, rows), dtype=torch.float32).t()
    return like.new_empty((rows, cols), dtype=torch.float32)


def quantize_fp8_rowwise(x: torch.Tensor, block_size: int = 128,
                         round_scale: bool = False,
                         col_scales: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """1 x block_size e4m3 quantization -> (codes [M, N] float8_e4m3fn, scales [M, ceil(N/bs)] fp32).

    col_scales: the scales come back column-major (same values, strides (1, M)); the
    reference's layout is row-major."""
    _require(x.is_cuda, "Input must be on CUDA")
    _require(x.ndim == 2, "Input must be 2D for now")
    return _run(_quant_rowwise_op, x, int(block_size), bool(round_scale), bool(col_scales))


@custom_op("quant_rowwise", "(Tensor x, int block_size, bool round_scale, bool col_scales) -> (Tensor, Tensor)")
def _quant_rowwise_op(x, block_size, round_scale, col_scales):
    M, N = x.shape
    x_fp8 = torch.empty((M, N), dtype=torch.float8_e4m3fn, device=x.device)
    scales = _scale_buf(x, M, _cdiv(N, block_size), col_scales)
    call("cin_quant_rowwise", ptr(x), dtype_code(x), M, N, x.stride(0), x.stride(1), block_size,
         int(round_scale), ptr(x_fp8), x_fp8.stride(0), ptr(scales), scales.stride(0),
         scales.stride(1), stream_of(x))
    return x_fp8, scales


@_quant_rowwise_op.register_fake
def _(x, block_size, round_scale, col_scales):
    M, N = x.shape
    return (x.new_empty((M, N), dtype=torch.float8_e4m3fn),
            _scale_buf(x, M, _cdiv(N, block_size), col_scales))


def quantize_fp8_blockwise(x: torch.Tensor, block_m: int = 128, block_n: int = 128,
                           round_scale: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """block_m x block_n e4m3 quantization -> (codes [M, N], scales [ceil(M/bm), ceil(N/bn)] fp32)."""
    _require(x.is_cuda, "Input must be on CUDA")
    _require(x.ndim == 2, "Input must be 2D")
    return _run(_quant_blockwise_op, x, int(block_m), int(block_n), bool(round_scale))


@custom_op("quant_blockwise",
           "(Tensor x, int block_m, int block_n, bool round_scale) -> (Tensor, Tensor)")
def _quant_blockwise_op(x, block_m, block_n, round_scale):
    M, N = x.shape
    x_fp8 = torch.empty((M, N), dtype=torch.float8_e4m3fn, device=x.device)
    scales = torch.empty((_cdiv(M, block_m), _cdiv(N, block_n)), dtype=torch.float32, device=x.device)
    call("cin_quant_blockwise", ptr(x), dtype_code(x), M, N, x.stride(0), x.stride(1), block_m,
         block_n, int(round_scale), ptr(x_fp8), x_fp8.stride(0), ptr(None), 0, ptr(scales),
         scales.stride(0), stream_of(x))
    return x_fp8, scales


@_quant_blockwise_op.register_fake
def _(x, block_m, block_n, round_scale):
    M, N = x.shape
    return (x.new_empty((M, N), dtype=torch.float8_e4m3fn),
            x.new_empty((_cdiv(M, block_m), _cdiv(N, block_n)), dtype=torch.float32))


def quantize_fp8_blockwise_t(x: torch.Tensor, round_scale: bool = False,
                             with_rowmajor: bool = True):
    """128x128 block quantization that also emits the transposed codes [N, M].

    Returns (codes [M, N] or None, codes_t [N, M], scales [ceil(M/128), ceil(N/128)]).
    The transposed codes are the K-contiguous B operand of the dgrad GEMM.
    """
    _require(x.is_cuda, "Input must be on CUDA")
    _require(x.ndim == 2, "Input must be 2D")
    q, qt, scales = _run(_quant_blockwise_t_op, x, bool(round_scale), bool(with_rowmajor))
    return (q if with_rowmajor else None), qt, scales


@custom_op("quant_blockwise_t",
           "(Tensor x, bool round_scale, bool with_rowmajor) -> (Tensor, Tensor, Tensor)")
def _quant_blockwise_t_op(x, round_scale, with_rowmajor):
    # without the row-major codes the first output is an empty [0, N] placeholder
    M, N = x.shape
    q = torch.empty((M if with_rowmajor else 0, N), dtype=torch.float8_e4m3fn, device=x.device)
    qt = torch.empty((N, M), dtype=torch.float8_e4m3fn, device=x.device)
    scales = torch.empty((_cdiv(M, 128), _cdiv(N, 128)), dtype=torch.float32, device=x.device)
    call("cin_quant_blockwise", ptr(x), dtype_code(x), M, N, x.stride(0), x.stride(1), 128, 128,
         int(round_scale), ptr(q) if with_rowmajor else ptr(None), N, ptr(qt), qt.stride(0),
         ptr(scales), scales.stride(0), stream_of(x))
    return q, qt, scales


@_quant_blockwise_t_op.register_fake
def _(x, round_scale, with_rowmajor):
    M, N = x.shape
    return (x.new_empty((M if with_rowmajor else 0, N), dtype=torch.float8_e4m3fn),
            x.new_empty((N, M), dtype=torch.float8_e4m3fn),
            x.new_empty((_cdiv(M, 128), _cdiv(N, 128)), dtype=torch.float32))


def quantize_fp8_forward(x: torch.Tensor, weight: torch.Tensor, round_scale: bool = False,
                         with_rowmajor: bool = True, with_transposed: bool = False,
                         col_scales: bool = False):
    """Both quantizations of the FP8 linear forward in one launch (reference
    src/kernels.py:746-747): x [M, K] in 1 x 128 row tiles with round_scale as given, and
    weight [N, K] in 128 x 128 blocks with round_scale off.  Bit-identical to
    quantize_fp8_rowwise(x, 128, round_scale) and quantize_fp8_blockwise(weight.float());
    a 16-bit weight is read as it is, without the fp32 copy.

    Returns (x_fp8 [M, K], x_scale [M, ceil(K/128)], w_fp8 [N, K] or None,
    w_fp8_t [K, N] or None, w_scale [ceil(N/128), ceil(K/128)]); x_scale column-major with
    col_scales.
    """
    _require(x.is_cuda and weight.is_cuda, "Inputs must be on CUDA")
    _require(x.ndim == 2 and weight.ndim == 2, "Inputs must be 2D")
    _require(x.shape[1] == weight.shape[1], "x and weight must share K")
    _require(with_rowmajor or with_transposed, "at least one layout of the weight codes")
    xq, xs, wq, wqt, ws = _run(_quant_fwd_op, x, weight, bool(round_scale), bool(with_rowmajor),
                                        bool(with_transposed), bool(col_scales))
    return xq, xs, (wq if with_rowmajor else None), (wqt if with_transposed else None), ws


@custom_op("quant_fwd", "(Tensor x, Tensor weight, bool round_scale, bool with_rowmajor, "
           "bool with_transposed, bool col_scales) -> (Tensor, Tensor, Tensor, Tensor, Tensor)")
def _quant_fwd_op(x, weight, round_scale, with_rowmajor, with_transposed, col_scales):
    # a weight layout not asked for comes back as an empty [0, ...] placeholder
    x = x if x.stride(1) == 1 else x.contiguous()
    weight = weight if weight.stride(1) == 1 else weight.contiguous()
    (M, K), N = x.shape, weight.shape[0]
    dev = x.device
    xq = torch.empty((M, K), dtype=torch.float8_e4m3fn, device=dev)
    xs = _scale_buf(x, M, _cdiv(K, 128), col_scales)
    wq = torch.empty((N if with_rowmajor else 0, K), dtype=torch.float8_e4m3fn, device=dev)
    wqt = torch.empty((K if with_transposed else 0, N), dtype=torch.float8_e4m3fn, device=dev)
    ws = torch.empty((_cdiv(N, 128), _cdiv(K, 128)), dtype=torch.float32, device=dev)
    call("cin_quant_fwd", ptr(x), dtype_code(x), M, K, x.stride(0), int(round_scale), ptr(xq), K,
         ptr(xs), xs.stride(0), xs.stride(1), ptr(weight), dtype_code(weight), N, weight.stride(0),
         ptr(wq) if with_rowmajor else ptr(None), K, ptr(wqt) if with_transposed else ptr(None), N,
         ptr(ws), ws.stride(0), stream_of(x))
    return xq, xs, wq, wqt, ws


@_quant_fwd_op.register_fake
def _(x, weight, round_scale, with_rowmajor, with_transposed, col_scales):
    (M, K), N = x.shape, weight.shape[0]
    return (x.new_empty((M, K), dtype=torch.float8_e4m3fn),
            _scale_buf(x, M, _cdiv(K, 128), col_scales),
            x.new_empty((N if with_rowmajor else 0, K), dtype=torch.float8_e4m3fn),
            x.new_empty((K if with_transposed else 0, N), dtype=torch.float8_e4m3fn),
            x.new_empty((_cdiv(N, 128), _cdiv(K, 128)), dtype=torch.float32))


def quantize_fp8_dual(dy: torch.Tensor, round_scale: bool = False, col_scales: bool = False):
    """Row tiles of dy and of dy^T from one read (reference src/kernels.py:771, :781-783).

    Returns (q [M, N], s [M, ceil(N/128)], qt [N, M], st [N, ceil(M/128)]), bit-identical to
    quantize_fp8_rowwise(dy) and quantize_fp8_rowwise(dy.t().contiguous()); s and st
    column-major with col_scales.
    """
    _require(dy.is_cuda, "Input must be on CUDA")
    _require(dy.ndim == 2, "Input must be 2D")
    return _run(_quant_dual_op, dy, bool(round_scale), bool(col_scales))


@custom_op("quant_dual", "(Tensor dy, bool round_scale, bool col_scales) -> (Tensor, Tensor, Tensor, Tensor)")
def _quant_dual_op(dy, round_scale, col_scales):
    M, N = dy.shape
    q = torch.empty((M, N), dtype=torch.float8_e4m3fn, device=dy.device)
    s = _scale_buf(dy, M, _cdiv(N, 128), col_scales)
    qt = torch.empty((N, M), dtype=torch.float8_e4m3fn, device=dy.device)
    st = _scale_buf(dy, N, _cdiv(M, 128), col_scales)
    call("cin_quant_dual", ptr(dy), dtype_code(dy), M, N, dy.stride(0), dy.stride(1),
         int(round_scale), ptr(q), q.stride(0), ptr(s), s.stride(0), s.stride(1), ptr(qt),
         qt.stride(0), ptr(st), st.stride(0), st.stride(1), stream_of(dy))
    return q, s, qt, st


@_quant_dual_op.register_fake
def _(dy, round_scale, col_scales):
    M, N = dy.shape
    return (dy.new_empty((M, N), dtype=torch.float8_e4m3fn),
            _scale_buf(dy, M, _cdiv(N, 128), col_scales),
            dy.new_empty((N, M), dtype=torch.float8_e4m3fn),
            _scale_buf(dy, N, _cdiv(M, 128), col_scales))


def requantize_rowwise_to_blockwise(x_fp8: torch.Tensor, x_scale: torch.Tensor,
                                    transposed: bool = False):
    """quantize_fp8_blockwise(dequantize_fp8_rowwise(x_fp8, x_scale), round_scale=False)
    without the fp32 temporary (reference src/kernels.py:784-787).

    Returns (codes, scales [ceil(M/128), ceil(K/128)]); codes are [M, K], or [K, M] when
    ``transposed`` (the K-contiguous B operand of the wgrad GEMM).
    """
    _require(x_fp8.is_cuda, "Input must be on CUDA")
    M, K = x_fp8.shape
    _require(x_fp8.dtype in (torch.float8_e4m3fn, torch.uint8),
             f"expected float8_e4m3fn codes, got {x_fp8.dtype}")
    _require(x_scale.shape == (M, _cdiv(K, 128)), "row scales must be [M, ceil(K/128)]")
    return _run(_requant_op, x_fp8, x_scale, bool(transposed))


@custom_op("requant_row_to_block", "(Tensor x_fp8, Tensor x_scale, bool transposed) -> (Tensor, Tensor)")
def _requant_op(x_fp8, x_scale, transposed):
    M, K = x_fp8.shape
    q = _rows8(_codes_u8(x_fp8))
    xs = _scales_2d(x_scale)
    sblk = torch.empty((_cdiv(M, 128), _cdiv(K, 128)), dtype=torch.float32, device=x_fp8.device)
    if transposed:
        out = torch.empty((K, M), dtype=torch.float8_e4m3fn, device=x_fp8.device)
        call("cin_requant_row_to_block", ptr(q), M, K, q.stride(0), ptr(xs), xs.stride(0),
             xs.stride(1), ptr(None), 0, ptr(out), out.stride(0), ptr(sblk), sblk.stride(0),
             stream_of(q))
    else:
        # the kernel stores 8 codes at a time: rows of a K that is not a multiple of 8 go
        # to a padded buffer, and the caller gets a contiguous copy
        K8 = _cdiv(K, 8) * 8
        out = torch.empty((M, K8), dtype=torch.float8_e4m3fn, device=x_fp8.device)
        call("cin_requant_row_to_block", ptr(q), M, K, q.stride(0), ptr(xs), xs.stride(0),
             xs.stride(1), ptr(out), out.stride(0), ptr(None), 0, ptr(sblk), sblk.stride(0),
             stream_of(q))
        if K8 != K:
            out = out[:, :K].contiguous()
    return out, sblk


@_requant_op.register_fake
def _(x_fp8, x_scale, transposed):
    M, K = x_fp8.shape
    return (x_fp8.new_empty((K, M) if transposed else (M, K), dtype=torch.float8_e4m3fn),
            x_fp8.new_empty((_cdiv(M, 128), _cdiv(K, 128)), dtype=torch.float32))


def quantize_fp8_backward(grad: torch.Tensor, x_fp8: torch.Tensor, x_scale: torch.Tensor,
                          round_scale: bool = False, col_scales: bool = False):
    """The three quantizations of FP8MatmulFunction.backward in one launch (reference
    src/kernels.py:771, :781-783, :784-787): dY [M, N] in 1 x 128 row tiles, dY^T in row
    tiles, and the saved row-wise X codes [M, K] re-quantized into 128 x 128 blocks, stored
    transposed.  Bit-identical to quantize_fp8_dual(grad, round_scale) followed by
    requantize_rowwise_to_blockwise(x_fp8, x_scale, transposed=True).

    Returns (g_fp8 [M, N], g_scale, g_fp8_t [N, M], g_scale_t, x_blk_t [K, M], x_sblk);
    g_scale and g_scale_t column-major with col_scales.  x_scale may have either layout.
    """
    _require(grad.is_cuda and x_fp8.is_cuda, "Inputs must be on CUDA")
    _require(grad.ndim == 2 and x_fp8.ndim == 2, "Inputs must be 2D")
    M, K = x_fp8.shape
    _require(grad.shape[0] == M, "grad and x_fp8 must share M")
    _require(x_fp8.dtype in (torch.float8_e4m3fn, torch.uint8),
             f"expected float8_e4m3fn codes, got {x_fp8.dtype}")
    _require(x_scale.shape == (M, _cdiv(K, 128)), "row scales must be [M, ceil(K/128)]")
    return _run(_quant_bwd_op, grad, x_fp8, x_scale, bool(round_scale), bool(col_scales))


@custom_op("quant_bwd", "(Tensor grad, Tensor x_fp8, Tensor x_scale, bool round_scale, bool col_scales) -> "
           "(Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)")
def _quant_bwd_op(grad, x_fp8, x_scale, round_scale, col_scales):
    dy = grad if grad.stride(1) == 1 else grad.contiguous()
    M, N = dy.shape
    K = x_fp8.shape[1]
    dev = dy.device
    xq = _rows8(_codes_u8(x_fp8))
    xs = _scales_2d(x_scale)
    q = torch.empty((M, N), dtype=torch.float8_e4m3fn, device=dev)
    s = _scale_buf(dy, M, _cdiv(N, 128), col_scales)
    qt = torch.empty((N, M), dtype=torch.float8_e4m3fn, device=dev)
    st = _scale_buf(dy, N, _cdiv(M, 128), col_scales)
    xbt = torch.empty((K, M), dtype=torch.float8_e4m3fn, device=dev)
    sblk = torch.empty((_cdiv(M, 128), _cdiv(K, 128)), dtype=torch.float32, device=dev)
    call("cin_quant_backward", ptr(dy), dtype_code(dy), M, N, dy.stride(0), int(round_scale), ptr(q),
         q.stride(0), ptr(s), s.stride(0), s.stride(1), ptr(qt), qt.stride(0), ptr(st), st.stride(0),
         st.stride(1), ptr(xq), K, xq.stride(0), ptr(xs), xs.stride(0), xs.stride(1), ptr(xbt),
         xbt.stride(0), ptr(sblk), sblk.stride(0), stream_of(dy))
    return q, s, qt, st, xbt, sblk


@_quant_bwd_op.register_fake
def _(grad, x_fp8, x_scale, round_scale, col_scales):
    M, N = grad.shape
    K = x_fp8.shape[1]
    return (grad.new_empty((M, N), dtype=torch.float8_e4m3fn),
            _scale_buf(grad, M, _cdiv(N, 128), col_scales),
            grad.new_empty((N, M), dtype=torch.float8_e4m3fn),
            _scale_buf(grad, N, _cdiv(M, 128), col_scales),
            grad.new_empty((K, M), dtype=torch.float8_e4m3fn),
            grad.new_empty((_cdiv(M, 128), _cdiv(K, 128)), dtype=torch.float32))


# ---------------------------------------------------------------------------
# Dequantization (reference src/kernels.py:262-314)
# ---------------------------------------------------------------------------
def dequantize_fp8_rowwise(x_fp8: torch.Tensor, scales: torch.Tensor,
                           block_size: int = 128) -> torch.Tensor:
    """fp32(code) * scale[row, col // block_size] -> fp32 [M, N].

    The reference's function is plain torch (src/kernels.py:262-281) and so runs on CPU
    tensors too; a CPU tensor takes the same product here (pad to whole tiles, one fp32
    multiply per element, drop the padding).  GPU tensors run the HIP dequantizer."""
    if x_fp8.device.type == "cpu":
        M, N = x_fp8.shape
        nb = scales.shape[1]
        x = x_fp8.float()          # exact: every e4m3 code is an fp32 value
        pad = nb * block_size - N
        if pad > 0:
            x = torch.nn.functional.pad(x, (0, pad))
        x = (x.view(M, nb, block_size) * scales.view(M, nb, 1)).view(M, nb * block_size)
        return x[:, :N] if pad > 0 else x
    _require(x_fp8.is_cuda, "Input must be on CUDA")
    _codes_u8(x_fp8)
    return _run(_dequant_rowwise_op, x_fp8, scales, int(block_size))


@custom_op("dequant_rowwise", "(Tensor x_fp8, Tensor scales, int block_size) -> Tensor")
def _dequant_rowwise_op(x_fp8, scales, block_size):
    M, N = x_fp8.shape
    q = _codes_u8(x_fp8)
    out = torch.empty((M, N), dtype=torch.float32, device=x_fp8.device)
    call("cin_dequant", ptr(q), M, N, q.stride(0), q.stride(1), ptr(scales), scales.stride(0),
         scales.stride(1), 1, block_size, ptr(out), _lib.CIN_DT_F32, out.stride(0), stream_of(q))
    return out


@_dequant_rowwise_op.register_fake
def _(x_fp8, scales, block_size):
    return x_fp8.new_empty(x_fp8.shape, dtype=torch.float32)


def dequantize_fp8(x_fp8: torch.Tensor, scales: torch.Tensor, block_m: int = 128,
                   block_n: int = 128) -> torch.Tensor:
    """bf16(fp32(code) * scale[block]) -> bf16 [M, N]; block_m = 1 reads row-wise scales."""
    _require(x_fp8.is_cuda, "Input must be on CUDA")
    M, N = x_fp8.shape
    _codes_u8(x_fp8)
    _require(scales.numel() >= _cdiv(M, block_m) * _cdiv(N, block_n),
             "scales too small for the block grid")
    return _run(_dequant_op, x_fp8, scales, int(block_m), int(block_n))


@custom_op("dequant", "(Tensor x_fp8, Tensor scales, int block_m, int block_n) -> Tensor")
def _dequant_op(x_fp8, scales, block_m, block_n):
    M, N = x_fp8.shape
    q = _codes_u8(x_fp8)
    # the reference indexes scales.flatten() as [row_block * ceil(N/bn) + col_block]
    flat = scales.reshape(-1)
    if flat.stride(0) != 1:
        flat = flat.contiguous()
    nbn = _cdiv(N, block_n)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=x_fp8.device)
    call("cin_dequant", ptr(q), M, N, q.stride(0), q.stride(1), ptr(flat), nbn, 1, block_m,
         block_n, ptr(out), _lib.CIN_DT_BF16, out.stride(0), stream_of(q))
    return out


@_dequant_op.register_fake
def _(x_fp8, scales, block_m, block_n):
    return x_fp8.new_empty(x_fp8.shape, dtype=torch.bfloat16)


# ---------------------------------------------------------------------------
# Block-scaled FP8 GEMM (reference src/kernels.py:588-702)
# ---------------------------------------------------------------------------
def _kcontig(codes: torch.Tensor, K: int) -> tuple[torch.Tensor, int]:
    """Return a [R, Kp] K-contiguous, 16-byte aligned uint8 view/copy and Kp (K padded to 16)."""
    q = _codes_u8(codes)
    Kp = _cdiv(K, 16) * 16
    if Kp == K and q.stride(1) == 1 and q.stride(0) % 16 == 0 and q.data_ptr() % 16 == 0:
        return q, K
    out = torch.zeros((q.shape[0], Kp), dtype=torch.uint8, device=q.device)
    out[:, :K].copy_(q)
    return out, Kp


def fp8_gemm_bs(a: torch.Tensor, a_scales: torch.Tensor, b_t: torch.Tensor,
                b_scales_nk: torch.Tensor, out_dtype: torch.dtype = torch.bfloat16,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """C[M, N] = block-scaled a[M, K] x b_t[N, K]^T.

    a_scales indexed [m, kb] (1 x 128 tiles of a); b_scales_nk indexed [n // 128, kb]
    (128 x 128 blocks of b_t).  out_dtype bf16 (RNE of the fp32 epilogue) or fp32.
    """
    _require(a.is_cuda and b_t.is_cuda, "Input must be on CUDA")
    M, K = a.shape
    N, K2 = b_t.shape
    _require(K == K2, f"Dimension mismatch: {K} vs {K2}")
    _require(a_scales.shape[0] >= M and a_scales.shape[1] >= _cdiv(K, 128), "a_scales too small")
    _require(b_scales_nk.shape[0] >= _cdiv(N, 128) and b_scales_nk.shape[1] >= _cdiv(K, 128),
             "b_scales too small")
    if out is None:
        _require(out_dtype in (torch.bfloat16, torch.float32), "out_dtype must be bf16 or fp32")
        return _run(_gemm_bs_op, a, a_scales, b_t, b_scales_nk, out_dtype)
    _require(out.dtype in (torch.bfloat16, torch.float32) and out.stride(1) == 1,
             "out must be bf16/fp32 with unit column stride")
    return _gemm_bs_into(a, a_scales, b_t, b_scales_nk, out)


def _gemm_bs_into(a, a_scales, b_t, b_scales_nk, out):
    M, K = a.shape
    N = b_t.shape[0]
    aq, Kp = _kcontig(a, K)
    bq, _ = _kcontig(b_t, K)
    call("cin_gemm_fp8_bs", ptr(aq), aq.stride(0), ptr(a_scales), a_scales.stride(0),
         a_scales.stride(1), ptr(bq), bq.stride(0), ptr(b_scales_nk), b_scales_nk.stride(0),
         b_scales_nk.stride(1), M, N, Kp, ptr(out), dtype_code(out), out.stride(0), stream_of(aq))
    return out


@custom_op("gemm_fp8_bs",
           "(Tensor a, Tensor a_scales, Tensor b_t, Tensor b_scales_nk, ScalarType out_dtype) -> Tensor")
def _gemm_bs_op(a, a_scales, b_t, b_scales_nk, out_dtype):
    out = torch.empty((a.shape[0], b_t.shape[0]), dtype=out_dtype, device=a.device)
    return _gemm_bs_into(a, a_scales, b_t, b_scales_nk, out)


@_gemm_bs_op.register_fake
def _(a, a_scales, b_t, b_scales_nk, out_dtype):
    return a.new_empty((a.shape[0], b_t.shape[0]), dtype=out_dtype)


def fp8_matmul_dsv3(a: torch.Tensor, b: torch.Tensor, a_scales: torch.Tensor,
                    b_scales: torch.Tensor) -> torch.Tensor:
    """C = A @ B with A [M, K] row-wise 1x128 scaled, B [K, N] 128x128 block scaled -> bf16."""
    M, K = a.shape
    K2, N = b.shape
    _require(K == K2, f"Dimension mismatch: {K} vs {K2}")
    _require(a.is_cuda and b.is_cuda, "Input must be on CUDA")
    # the GEMM wants B^T [N, K] K-contiguous: a transposed view of such a tensor is free,
    # otherwise transpose the codes on the device
    bq = _codes_u8(b)
    if bq.stride(0) == 1 and bq.stride(1) % 16 == 0 and bq.data_ptr() % 16 == 0 and K % 16 == 0:
        b_t = bq.t()
    else:
        b_t = _run(_transpose_u8_op, bq)
    # b_scales is [kb, nb]; the GEMM reads it as [nb, kb] through swapped strides
    return fp8_gemm_bs(a, a_scales, b_t, b_scales.t(), torch.bfloat16)


@custom_op("transpose_u8", "(Tensor src) -> Tensor")
def _transpose_u8_op(src):
    R, C = src.shape
    s = src if src.stride(1) == 1 else src.contiguous()
    out = torch.empty((C, R), dtype=torch.uint8, device=src.device)
    call("cin_transpose_u8", ptr(s), R, C, s.stride(0), ptr(out), out.stride(0), stream_of(s))
    return out


@_transpose_u8_op.register_fake
def _(src):
    return src.new_empty((src.shape[1], src.shape[0]), dtype=torch.uint8)


# ---------------------------------------------------------------------------
# Autograd function / module / conversion (reference src/kernels.py:731-905)
# ---------------------------------------------------------------------------
class FP8MatmulFunction(torch.autograd.Function):
    """DeepSeek-V3 style FP8 matmul: y = x @ weight^T with 1x128 activation tiles and
    128x128 weight blocks (reference src/kernels.py:731-794).

    Forward quantizes x row-wise and the weight block-wise (emitting the transposed
    weight codes for dgrad) and runs one GEMM.  Backward quantizes dY once into row
    tiles and dY^T row tiles and re-quantizes the saved x codes into transposed 128x128
    blocks, all in one launch (cin_quant_backward), and runs the dgrad and wgrad GEMMs,
    with the same operands and rounding steps as the reference.
    """

    @staticmethod
    def forward(ctx, x, weight, round_scale, weight_fp8=None):
        # weight_fp8: optional (codes, transposed codes, scales) of this weight from
        # quantize_fp8_blockwise_t, e.g. FP8Linear's weight cache
        x_shape = x.shape
        x_flat = x.reshape(-1, x_shape[-1])
        M, K = x_flat.shape
        N = weight.shape[0]
        if weight_fp8 is None:
            # x row tiles and weight blocks in one launch; the weight's 16-bit values are
            # exact in fp32, so this equals quantizing weight.float() as the reference does
            x_fp8, x_scale, w_fp8, w_fp8_t, w_scale = quantize_fp8_forward(
                x_flat, weight, round_scale, with_rowmajor=True, with_transposed=True, col_scales=True)
        else:
            x_fp8, x_scale = quantize_fp8_rowwise(x_flat, block_size=128, round_scale=round_scale,
                                                  col_scales=True)
            w_fp8, w_fp8_t, w_scale = weight_fp8
        out = fp8_gemm_bs(x_fp8, x_scale, w_fp8, w_scale, torch.bfloat16)
        ctx.save_for_backward(x_fp8, x_scale, w_fp8_t, w_scale)
        ctx.x_shape = x_shape
        ctx.round_scale = round_scale
        return out.reshape(*x_shape[:-1], N)

    @staticmethod
    def backward(ctx, grad_output):
        x_fp8, x_scale, w_fp8_t, w_scale = ctx.saved_tensors
        x_shape = ctx.x_shape
        grad_flat = grad_output.reshape(-1, grad_output.shape[-1])
        # dY row tiles, dY^T row tiles and X^T blocks in one launch
        g_fp8, g_scale, g_fp8_t, g_scale_t, x_blk_t, x_sblk = quantize_fp8_backward(
            grad_flat, x_fp8, x_scale, ctx.round_scale, col_scales=True)
        # dgrad: dX[M, K] = dY[M, N] . W[N, K]; B^T = W^T [K, N], block scales read as [kb, nb]
        grad_x = fp8_gemm_bs(g_fp8, g_scale, w_fp8_t, w_scale.t(), torch.bfloat16)
        # wgrad: dW[N, K] = dY^T[N, M] . X[M, K]; B^T = X^T block codes [K, M]
        grad_w = fp8_gemm_bs(g_fp8_t, g_scale_t, x_blk_t, x_sblk.t(), torch.bfloat16)
        return grad_x.reshape(x_shape), grad_w, None, None


class WeightCache:
    """Quantized copies of a parameter, rebuilt only when the parameter changes.

    The key is the parameter's version counter (bumped by every in-place update: optimizer
    steps, copy_, load_state_dict), its storage pointer (re-assignment) and its dtype/shape.
    Writes through ``param.data`` do not bump the version counter; callers that update
    weights that way must call ``clear()``.  Never used while torch.compile traces."""

    def __init__(self):
        self.key = None
        self.value = None

    def get(self, params, build):
        key = tuple((p._version, p.data_ptr(), p.dtype, tuple(p.shape)) for p in params)
        if key != self.key:
            self.value = None  # release the old copies before building the new ones
            self.value = build()
            self.key = key
        return self.value

    def clear(self):
        self.key = self.value = None


def _weight_cache_active(module) -> bool:
    return module.cache_weights and not torch.compiler.is_compiling()


class FP8Linear(torch.nn.Module):
    """Linear layer with DeepSeek-V3 FP8 quantization (reference src/kernels.py:797-840).

    Keeps an fp32 master ``weight`` [out, in] (init N(0, 0.02)) and an optional bias
    added after the FP8 matmul.  On non-GPU tensors the reference runs F.linear, and so
    does this module.  With ``cache_weights`` (off by default; see set_weight_cache) the
    weight's codes are kept between forwards until the weight changes, instead of
    re-quantizing on every forward as the reference does (src/kernels.py:747-749): with
    gradient accumulation the weight is quantized once per optimizer step.
    """

    def __init__(self, in_features: int, out_features: int, bias: bool = False,
                 round_scale: bool = False):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.round_scale = round_scale
        self.cache_weights = False
        self._wcache = WeightCache()
        self.weight = torch.nn.Parameter(torch.empty(out_features, in_features))
        torch.nn.init.normal_(self.weight, mean=0.0, std=0.02)
        if bias:
            self.bias = torch.nn.Parameter(torch.zeros(out_features))
        else:
            self.register_parameter("bias", None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.is_cuda:
            wq = None
            if _weight_cache_active(self):
                w = self.weight.detach()
                wq = self._wcache.get([self.weight], lambda: quantize_fp8_blockwise_t(
                    w if w.dtype == torch.float32 else w.float(), round_scale=False))
            out = FP8MatmulFunction.apply(x, self.weight, self.round_scale, wq)
        else:
            out = torch.nn.functional.linear(x, self.weight, None)
        if self.bias is not None:
            out = out + self.bias
        return out

    @classmethod
    def from_linear(cls, linear: torch.nn.Linear, round_scale: bool = False) -> "FP8Linear":
        fp8_linear = cls(linear.in_features, linear.out_features, bias=linear.bias is not None,
                         round_scale=round_scale)
        fp8_linear.weight = torch.nn.Parameter(linear.weight.data.clone())
        if linear.bias is not None:
            fp8_linear.bias = torch.nn.Parameter(linear.bias.data.clone())
        return fp8_linear


def set_weight_cache(model: torch.nn.Module, enabled: bool = True) -> torch.nn.Module:
    """Turn the quantized-weight cache of every FP8Linear and FP8 expert layer in ``model``
    on or off (off clears it).  With the cache on, weights are quantized once per change
    (per optimizer step) instead of once per forward."""
    for m in model.modules():
        if hasattr(m, "cache_weights") and hasattr(m, "_wcache"):
            m.cache_weights = bool(enabled)
            if not enabled:
                m._wcache.clear()
    return model


_DEFAULT_EXCLUDE = ["embedding", "lm_head", "router", "norm", "attn", "indexer"]
_ROUND_SCALE_NAMES = ["w_out", "w1", "w2"]


def convert_to_fp8(model: torch.nn.Module, exclude_names: list | None = None) -> torch.nn.Module:
    """Swap eligible nn.Linear modules for FP8Linear (reference src/kernels.py:843-905).

    Skips names containing embedding/lm_head/router/norm/attn/indexer (plus
    ``exclude_names``) and layers with a dimension under 128; names containing
    w_out/w1/w2 get power-of-two activation and gradient scales.
    """
    exclude = (exclude_names or []) + _DEFAULT_EXCLUDE
    for name, module in list(model.named_modules()):
        if not isinstance(module, torch.nn.Linear):
            continue
        if any(ex in name for ex in exclude):
            continue
        if module.in_features < 128 or module.out_features < 128:
            print(f"[FP8] Auto-excluding {name}: shape ({module.out_features}, "
                  f"{module.in_features}) < 128")
            continue
        parts = name.rsplit(".", 1)
        if len(parts) == 2:
            parent = model.get_submodule(parts[0])
            attr = parts[1]
        else:
            parent, attr = model, name
        round_scale = any(key in name for key in _ROUND_SCALE_NAMES)
        setattr(parent, attr, FP8Linear.from_linear(module, round_scale=round_scale))
    return model


# ---------------------------------------------------------------------------
# Unquantized grouped GEMM (reference src/kernels.py:526-581)
# ---------------------------------------------------------------------------
def moe_grouped_gemm(sorted_x: torch.Tensor, weights: torch.Tensor, expert_starts: torch.Tensor,
                     expert_ends: torch.Tensor, max_expert_tokens: int | None = None) -> torch.Tensor:
    """C[r] = fp16(fp16(sorted_x[r]) . fp16(weights[e])^T) for the rows r of each expert e.

    sorted_x [T, d_in], weights [E, d_out, d_in] (bf16, fp16 or fp32), expert ranges as
    device tensors -> fp16 [T, d_out].  One launch covers every expert with a device-side
    tile table, so max_expert_tokens (a host value in the reference) is not needed and
    is ignored.  Rows outside every range are left unset (torch.empty, as the reference).
    """
    _require(sorted_x.is_cuda and weights.is_cuda, "Input must be on CUDA")
    _require(sorted_x.ndim == 2 and weights.ndim == 3, "sorted_x must be 2D and weights 3D")
    T, d_in = sorted_x.shape
    E, d_out, d_in2 = weights.shape
    _require(d_in == d_in2, f"Dimension mismatch: {d_in} vs {d_in2}")
    a = sorted_x if sorted_x.stride(1) == 1 else sorted_x.contiguous()
    w = weights if weights.stride(2) == 1 else weights.contiguous()
    starts = expert_starts.to(device=a.device, dtype=torch.int64).contiguous()
    ends = expert_ends.to(device=a.device, dtype=torch.int64).contiguous()
    _require(starts.numel() == E and ends.numel() == E, "expert ranges must have n_experts entries")
    return _run(_grouped_f16_op, a, w, starts, ends)


@custom_op("grouped_gemm_f16", "(Tensor a, Tensor w, Tensor starts, Tensor ends) -> Tensor")
def _grouped_f16_op(a, w, starts, ends):
    T, d_in = a.shape
    E, d_out, _ = w.shape
    out = torch.empty((T, d_out), dtype=torch.float16, device=a.device)
    call("cin_grouped_gemm_f16", ptr(a), dtype_code(a), a.stride(0), ptr(w), dtype_code(w),
         w.stride(0), w.stride(1), ptr(starts), ptr(ends), E, T, d_out, d_in, ptr(out),
         out.stride(0), stream_of(a))
    return out


@_grouped_f16_op.register_fake
def _(a, w, starts, ends):
    return a.new_empty((a.shape[0], w.shape[1]), dtype=torch.float16)


# ---------------------------------------------------------------------------
# DSA indexer scoring on FP8 q / k (reference src/attention.py:288-300)
# ---------------------------------------------------------------------------
def indexer_scores_fp8(q: torch.Tensor, k: torch.Tensor, weights: torch.Tensor,
                       softmax_scale: float) -> torch.Tensor:
    """The FP8 branch of DSAIndexer.forward up to the mask (reference
    src/attention.py:288-300): q [B, L, H, d] and k [B, S, d] quantized row-wise (1x128,
    the first scale of each row), scores [B, L, S] fp32 = k_scale * sum_h
    relu(q_codes . k_codes) * (q_scale * weights * softmax_scale).  Two launches: k's
    quantization, then one scoring kernel that quantizes q itself (H <= 4 for d <= 128,
    H <= 2 above; with more heads both quantizations run first, in one launch, and the
    scoring kernel takes the codes).  Scores, codes and scales are the same either way; the
    reference's [B, L, H, S] fp32 logits are never written.  weights [B, L, H]; d a multiple
    of 32 up to 256.

    Differentiable in `weights` only, as the reference's branch is: its q and k pass through
    the quantizer, which carries no gradient (the scores feed the indexer's KL loss,
    src/attention.py:480-502, whose gradient reaches weights_proj alone)."""
    _require(q.is_cuda and k.is_cuda and weights.is_cuda, "Input must be on CUDA")
    _require(q.ndim == 4 and k.ndim == 3 and weights.shape == q.shape[:3],
             "q must be [B, L, H, d], k [B, S, d], weights [B, L, H]")
    B, L, H, d = q.shape
    _require(k.shape[0] == B and k.shape[2] == d, "k must be [B, S, d] with q's B and d")
    _require(d % 32 == 0 and 32 <= d <= 256, "head dim must be a multiple of 32 in [32, 256]")
    S = k.shape[1]
    w = weights.float().contiguous()
    if H <= (4 if d <= 128 else 2):
        # the q codes are kept only for the weights' gradient
        save_q = torch.is_grad_enabled() and w.requires_grad
        if _plain_eager(q, k, w):
            return _IndexerScoresQ.apply(q.detach(), k.detach(), w, float(softmax_scale), save_q)
        k8, ks = _indexer_quant_k_op(k.detach(), H)
        return _indexer_q_op(q.detach(), k8, ks, w, float(softmax_scale), save_q)[0]
    q8, qs, k8, ks = _indexer_quant_op(q.detach(), k.detach())
    return _indexer_op(q8, qs, k8, ks, w, float(softmax_scale))


def _aligned16(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


@custom_op("indexer_quantize", "(Tensor q, Tensor k) -> (Tensor, Tensor, Tensor, Tensor)")
def _indexer_quant_op(q, k):
    """Both row-wise 1x128 quantizations of the indexer (src/attention.py:292-297) in one
    call, keeping only each row's first scale: (q codes [B, L, H, d], q_scale [B, L, H],
    k codes [B, S, d], k_scale [B, S]), bit-identical to quantize_fp8_rowwise."""
    B, L, H, d = q.shape
    S = k.shape[1]
    q, k = _aligned16(q), _aligned16(k)
    q8 = torch.empty((B, L, H, d), dtype=torch.float8_e4m3fn, device=q.device)
    k8 = torch.empty((B, S, d), dtype=torch.float8_e4m3fn, device=q.device)
    qs = torch.empty((B, L, H), dtype=torch.float32, device=q.device)
    ks = torch.empty((B, S), dtype=torch.float32, device=q.device)
    call("cin_indexer_quantize", ptr(q), dtype_code(q), ptr(k), dtype_code(k), B, L, S, H, d, ptr(q8),
         ptr(qs), ptr(k8), ptr(ks), stream_of(q))
    return q8, qs, k8, ks


@_indexer_quant_op.register_fake
def _(q, k):
    B, L, H, d = q.shape
    S = k.shape[1]
    return (q.new_empty((B, L, H, d), dtype=torch.float8_e4m3fn), q.new_empty((B, L, H), dtype=torch.float32),
            q.new_empty((B, S, d), dtype=torch.float8_e4m3fn), q.new_empty((B, S), dtype=torch.float32))


def _launch_quant_k(k, H):
    B, S, d = k.shape
    k = _aligned16(k)
    k8 = torch.empty((B, S, d), dtype=torch.float8_e4m3fn, device=k.device)
    ks = torch.empty((B, S), dtype=torch.float32, device=k.device)
    # (L = 0: no q rows; q's pointer and dtype are k's)
    call("cin_indexer_quantize", ptr(k), dtype_code(k), ptr(k), dtype_code(k), B, 0, S, H, d, None, None,
         ptr(k8), ptr(ks), stream_of(k))
    return k8, ks


def _launch_scores_q(q, k8, k_scale, weights, softmax_scale, save_q):
    B, L, H, d = q.shape
    S = k8.shape[1]
    q = _aligned16(q)
    kc = _codes_u8(k8).contiguous()
    out = torch.empty((B, L, S), dtype=torch.float32, device=q.device)
    q8 = torch.empty((B, L, H, d) if save_q else (0,), dtype=torch.float8_e4m3fn, device=q.device)
    qs = torch.empty((B, L, H) if save_q else (0,), dtype=torch.float32, device=q.device)
    call("cin_indexer_scores_fp8_q", ptr(q), dtype_code(q), ptr(kc), ptr(k_scale.contiguous()),
         ptr(weights.contiguous()), B, L, S, H, d, softmax_scale, ptr(out), ptr(q8) if save_q else None,
         ptr(qs) if save_q else None, stream_of(q))
    return out, q8, qs


def _launch_wgrad(q8, q_scale, k8, k_scale, grad_scores, softmax_scale):
    B, L, H, d = q8.shape
    S = k8.shape[1]
    qc, kc = _codes_u8(q8).contiguous(), _codes_u8(k8).contiguous()
    g = grad_scores.float().contiguous()
    nws = max(1, _cdiv(S, 512) * B * L * H)  # one partial per 512-key range
    ws = torch.empty(nws, dtype=torch.float32, device=q8.device)
    dw = torch.empty((B, L, H), dtype=torch.float32, device=q8.device)
    call("cin_indexer_weights_grad", ptr(qc), ptr(q_scale.contiguous()), ptr(kc), ptr(k_scale.contiguous()),
         ptr(g), B, L, S, H, d, softmax_scale, ptr(ws), nws, ptr(dw), stream_of(qc))
    return dw


class _IndexerScoresQ(torch.autograd.Function):
    """kernels.indexer_scores_fp8 in eager mode: the launches of indexer_quantize_k and
    indexer_scores_fp8_q, and in backward indexer_weights_grad_fp8's, called directly."""

    @staticmethod
    def forward(ctx, q, k, w, softmax_scale, save_q):
        k8, ks = _launch_quant_k(k, q.shape[2])
        out, q8, qs = _launch_scores_q(q, k8, ks, w, softmax_scale, save_q)
        if save_q:
            ctx.save_for_backward(q8, qs, k8, ks)
        ctx.softmax_scale = softmax_scale
        return out

    @staticmethod
    def backward(ctx, grad):
        q8, qs, k8, ks = ctx.saved_tensors
        return None, None, _launch_wgrad(q8, qs, k8, ks, grad, ctx.softmax_scale), None, None


@custom_op("indexer_quantize_k", "(Tensor k, int H) -> (Tensor, Tensor)")
def _indexer_quant_k_op(k, H):
    """k's side of indexer_quantize alone: (codes [B, S, d], first scales [B, S])."""
    return _launch_quant_k(k, H)


@_indexer_quant_k_op.register_fake
def _(k, H):
    B, S, d = k.shape
    return k.new_empty((B, S, d), dtype=torch.float8_e4m3fn), k.new_empty((B, S), dtype=torch.float32)


@custom_op("indexer_scores_fp8_q", "(Tensor q, Tensor k8, Tensor k_scale, Tensor weights, float softmax_scale, "
           "bool save_q) -> (Tensor, Tensor, Tensor)")
def _indexer_q_op(q, k8, k_scale, weights, softmax_scale, save_q):
    """Scores from unquantized q (cin_indexer_scores_fp8_q): (scores [B, L, S], q codes
    [B, L, H, d], q first scales [B, L, H]), the last two empty unless save_q."""
    return _launch_scores_q(q, k8, k_scale, weights, softmax_scale, save_q)


@_indexer_q_op.register_fake
def _(q, k8, k_scale, weights, softmax_scale, save_q):
    B, L, H, d = q.shape
    return (q.new_empty((B, L, k8.shape[1]), dtype=torch.float32),
            q.new_empty((B, L, H, d) if save_q else (0,), dtype=torch.float8_e4m3fn),
            q.new_empty((B, L, H) if save_q else (0,), dtype=torch.float32))


def _indexer_q_setup(ctx, inputs, output):
    _q, k8, k_scale, _weights, softmax_scale, save_q = inputs
    _out, q8, q_scale = output
    ctx.mark_non_differentiable(q8, q_scale)
    ctx.save_q = save_q
    if save_q:
        ctx.save_for_backward(q8, q_scale, k8, k_scale)
    ctx.softmax_scale = softmax_scale


def _indexer_q_backward(ctx, grad, _grad_q8, _grad_qs):
    dw = None
    if ctx.needs_input_grad[3]:
        _require(ctx.save_q, "indexer_scores_fp8_q: the weights' gradient needs save_q=True")
        q8, q_scale, k8, k_scale = ctx.saved_tensors
        dw = _indexer_wgrad_op(q8, q_scale, k8, k_scale, grad, ctx.softmax_scale)
    return None, None, None, dw, None, None


_indexer_q_op.register_autograd(_indexer_q_backward, setup_context=_indexer_q_setup)


@custom_op("indexer_scores_fp8",
           "(Tensor q8, Tensor q_scale, Tensor k8, Tensor k_scale, Tensor weights, float softmax_scale) -> Tensor")
def _indexer_op(q8, q_scale, k8, k_scale, weights, softmax_scale):
    B, L, H, d = q8.shape
    S = k8.shape[1]
    qc, kc = _codes_u8(q8).contiguous(), _codes_u8(k8).contiguous()
    out = torch.empty((B, L, S), dtype=torch.float32, device=q8.device)
    call("cin_indexer_scores_fp8", ptr(qc), ptr(q_scale.contiguous()), ptr(kc), ptr(k_scale.contiguous()),
         ptr(weights.contiguous()), B, L, S, H, d, softmax_scale, ptr(out), stream_of(qc))
    return out


@_indexer_op.register_fake
def _(q8, q_scale, k8, k_scale, weights, softmax_scale):
    return q8.new_empty((q8.shape[0], q8.shape[1], k8.shape[1]), dtype=torch.float32)


@custom_op("indexer_weights_grad_fp8",
           "(Tensor q8, Tensor q_scale, Tensor k8, Tensor k_scale, Tensor grad_scores, float softmax_scale) -> Tensor")
def _indexer_wgrad_op(q8, q_scale, k8, k_scale, grad_scores, softmax_scale):
    return _launch_wgrad(q8, q_scale, k8, k_scale, grad_scores, softmax_scale)


@_indexer_wgrad_op.register_fake
def _(q8, q_scale, k8, k_scale, grad_scores, softmax_scale):
    return q8.new_empty(q8.shape[:3], dtype=torch.float32)


def _indexer_setup(ctx, inputs, output):
    q8, q_scale, k8, k_scale, _weights, softmax_scale = inputs
    ctx.save_for_backward(q8, q_scale, k8, k_scale)
    ctx.softmax_scale = softmax_scale


def _indexer_backward(ctx, grad):
    q8, q_scale, k8, k_scale = ctx.saved_tensors
    dw = None
    if ctx.needs_input_grad[4]:
        dw = _indexer_wgrad_op(q8, q_scale, k8, k_scale, grad, ctx.softmax_scale)
    return None, None, None, None, dw, None


_indexer_op.register_autograd(_indexer_backward, setup_context=_indexer_setup)


# ---------------------------------------------------------------------------
# Outside the FP8 path: torch restatements that keep the reference's names importable
# ---------------------------------------------------------------------------
def lightning_indexer_fused(q: torch.Tensor, k: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """I[b, i, j] = sum_h relu(q[b, i, h, :] . k[b, j, :]) * w[b, i, h] in fp32, fp16 out
    (reference src/kernels.py:392-432).  Plain torch."""
    _require(q.is_cuda and k.is_cuda, "Inputs must be on CUDA")
    B, Lq, H, D = q.shape
    s = torch.matmul(q.float().reshape(B, Lq * H, D), k.float().transpose(1, 2).contiguous())
    s = s.relu_().reshape(B, Lq, H, -1)
    return (s * w.float().unsqueeze(-1)).sum(dim=2).to(torch.float16)


def sparse_attention(q, k, v, idx, scale=None):
    """Attention of each query t over the keys idx[b, t, :] with idx <= t (reference
    src/kernels.py:1176-1320): returns (output [B, H, L, Dv] in q's dtype, attention
    probabilities [B, H, L, K] fp32, zero where masked).  Plain torch, autograd through the
    output; the probabilities are returned detached, as the reference's backward ignores
    their gradient."""
    if scale is None:
        scale = q.shape[-1] ** -0.5
    B, H, L, _ = q.shape
    valid = idx <= torch.arange(L, device=idx.device).view(1, L, 1)
    ic = idx.clamp(0, L - 1)
    bi = torch.arange(B, device=idx.device).view(B, 1, 1)
    kg = k.float().permute(0, 2, 1, 3)[bi, ic].permute(0, 3, 1, 2, 4)   # [B, H, L, K, D]
    vg = v.float().permute(0, 2, 1, 3)[bi, ic].permute(0, 3, 1, 2, 4)
    scores = (q.float().unsqueeze(3) * kg).sum(-1) * scale
    scores = scores.masked_fill(~valid.unsqueeze(1), float("-inf"))
    p = torch.softmax(scores, dim=-1).nan_to_num(0.0)
    out = (p.unsqueeze(-1) * vg).sum(3)
    return out.to(q.dtype), p.detach()
