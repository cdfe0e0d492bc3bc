"""ctypes binding of libcinnamon_fp8.so (the C ABI declared in include/cinnamon_fp8.h).

The library is loaded lazily, after ``import torch``, so it binds to the HIP
runtime torch has already mapped.  There is no fallback: if the library is
missing or fails to load, every call raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
DEFAULT_PATH = os.path.join(_HERE, "libcinnamon_fp8.so")

CIN_DT_BF16, CIN_DT_F32, CIN_DT_F16 = 0, 1, 2
CIN_OK, CIN_ERR_ARG, CIN_ERR_UNSUPPORTED, CIN_ERR_HIP = 0, -1, -2, -3

_DTYPE_CODE = {torch.bfloat16: CIN_DT_BF16, torch.float32: CIN_DT_F32, torch.float16: CIN_DT_F16}

_p, _i64, _i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int

# name -> argtypes (all return int)
SIGNATURES: dict[str, list] = {
    "cin_abi_version": [],
    "cin_quant_rowwise": [_p, _i32, _i64, _i64, _i64, _i64, _i64, _i32, _p, _i64, _p, _i64, _i64, _p],
    "cin_quant_blockwise": [_p, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _p, _i64, _p, _i64,
                            _p, _i64, _p],
    "cin_dequant": [_p, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _p, _i32, _i64, _p],
    "cin_quant_fwd": [_p, _i32, _i64, _i64, _i64, _i32, _p, _i64, _p, _i64, _i64, _p, _i32, _i64, _i64, _p,
                      _i64, _p, _i64, _p, _i64, _p],
    "cin_quant_dual": [_p, _i32, _i64, _i64, _i64, _i64, _i32, _p, _i64, _p, _i64, _i64, _p, _i64, _p,
                       _i64, _i64, _p],
    "cin_requant_row_to_block": [_p, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _p, _i64, _p, _i64, _p],
    "cin_quant_backward": [_p, _i32, _i64, _i64, _i64, _i32, _p, _i64, _p, _i64, _i64, _p, _i64, _p,
                           _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _p, _i64, _p],
    "cin_transpose_u8": [_p, _i64, _i64, _i64, _p, _i64, _p],
    "cin_gemm_fp8_bs": [_p, _i64, _p, _i64, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _i64, _p,
                        _i32, _i64, _p],
    "cin_grouped_gemm_fp8": [_p, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _i64, _p,
                             _p, _i64, _i64, _i64, _i64, _p, _i32, _i64, _p],
    "cin_quant_dual_grouped": [_p, _i32, _i64, _i64, _i64, _p, _p, _i64, _i32, _p, _i64, _p, _i64,
                               _i64, _p, _i64, _p, _i64, _i64, _p],
    "cin_requant_row_to_block_grouped": [_p, _i64, _i64, _i64, _p, _i64, _i64, _p, _p, _i64, _p,
                                         _i64, _p, _i64, _p],
    "cin_grouped_gemm_f16": [_p, _i32, _i64, _p, _i32, _i64, _i64, _p, _p, _i64, _i64, _i64, _i64,
                             _p, _i64, _p],
    "cin_grouped_gemm_fp8_wgrad": [_p, _i64, _p, _i64, _i64, _p, _i64, _p, _i64, _p, _p, _i64, _i64,
                                   _i64, _i64, _i64, _p, _i32, _i64, _i64, _p],
    "cin_silu_mul_quant_rowwise": [_p, _i32, _i64, _i64, _i64, _i32, _i32, _p, _i64, _p, _i64, _i64, _p],
    "cin_swiglu_backward": [_p, _i64, _p, _i32, _i64, _i64, _i64, _p, _i64, _p],
    "cin_swiglu_dual_grouped": [_p, _i64, _p, _i32, _i64, _i64, _i64, _p, _p, _i64, _i32, _p, _i64, _p,
                                _i64, _i64, _p, _i64, _p, _i64, _i64, _p],
    "cin_zero_rows_outside_ranges": [_p, _i64, _i64, _i64, _p, _p, _i64, _p],
    "cin_indexer_quantize": [_p, _i32, _p, _i32, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p],
    "cin_indexer_scores_fp8": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, _p,
                               _p],
    "cin_indexer_scores_fp8_q": [_p, _i32, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, _p,
                                 _p, _p, _p],
    "cin_indexer_weights_grad": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, _p,
                                 _i64, _p, _p],
    "cin_indexer_weights_grad_workspace": [_i64, _i64, _i64, _i64],
    "cin_moe_route": [_p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _i64, _p],
    "cin_moe_route_workspace": [_i64, _i64, _i64],
    "cin_moe_route_noalloc": [_p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p],
    "cin_moe_gather_quant_rowwise": [_p, _i32, _i64, _i64, _i64, _p, _i64, _i64, _i32, _p, _i64, _p,
                                     _i64, _i64, _p],
    "cin_moe_gather_sum": [_p, _i32, _i64, _p, _i64, _i64, _i64, _i64, _p, _i32, _i64, _p],
    "cin_moe_scatter_quant_rowwise": [_p, _i32, _i64, _i64, _i64, _p, _i64, _p, _i64, _i32, _p, _i64,
                                      _p, _i64, _i64, _p],
    "cin_moe_scatter_quant_rowwise_ws": [_p, _i32, _i64, _i64, _i64, _p, _i64, _p, _i64, _i32, _p, _i64,
                                         _p, _i64, _i64, _p, _p],
    "cin_moe_combine": [_p, _i32, _i64, _p, _i32, _i64, _p, _i64, _i64, _i64, _i64, _p, _i64, _p],
    "cin_moe_combine_backward": [_p, _i64, _p, _i32, _i64, _p, _i32, _i64, _p, _p, _i64, _i64, _i64,
                                 _i64, _p, _i32, _i64, _p, _p],
}

# entry points that return something other than an int status
RESTYPES = {"cin_indexer_weights_grad_workspace": ctypes.c_int64}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class CinnamonLibraryError(RuntimeError):
    """The native library is missing, failed to load, or reported an error."""


def library_path() -> str:
    return os.environ.get("CINNAMON_FP8_LIB", DEFAULT_PATH)


def load() -> ctypes.CDLL:
    """Load (once) and return the native library; raises if it is unavailable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not os.path.exists(path):
            raise CinnamonLibraryError(
                f"{path} not found: build it with `python -m cinnamon_amd._build` "
                "(or __graft_entry__.build())")
        try:
            lib = ctypes.CDLL(path)
        except OSError as e:  # pragma: no cover - depends on the host
            raise CinnamonLibraryError(f"failed to load {path}: {e}") from e
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = RESTYPES.get(name, ctypes.c_int)
        lib.cin_last_error.argtypes = []
        lib.cin_last_error.restype = ctypes.c_char_p
        _lib = lib
        return lib


def last_error() -> str:
    return load().cin_last_error().decode(errors="replace")


def call(name: str, *args) -> None:
    """Call an entry point; raise ValueError (bad argument) or RuntimeError on failure."""
    rc = getattr(load(), name)(*args)
    if rc != CIN_OK:
        msg = f"{name} failed ({rc}): {last_error()}"
        if rc == CIN_ERR_ARG:
            raise ValueError(msg)
        raise CinnamonLibraryError(msg)


def dtype_code(t) -> int:
    """CIN_DT_* code of a tensor's dtype (or of a torch.dtype)."""
    dt = t if isinstance(t, torch.dtype) else t.dtype
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise ValueError(f"unsupported dtype {dt}; expected bfloat16, float16 or float32") from None


def stream_of(t: torch.Tensor) -> ctypes.c_void_p:
    """torch's current HIP stream on the tensor's device (as a hipStream_t)."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())
