"""CPU checks of the C ABI: the library loads, exports every declared entry point, and
rejects invalid arguments before touching the GPU."""
import ctypes
import os
import re

import pytest

from cinnamon_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cinnamon_fp8.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(cin_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for name in ["cin_quant_rowwise", "cin_quant_blockwise", "cin_dequant", "cin_quant_dual",
                 "cin_requant_row_to_block", "cin_gemm_fp8_bs", "cin_grouped_gemm_fp8",
                 "cin_last_error", "cin_abi_version"]:
        assert name in syms


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    # and the ctypes binding covers every compute entry point
    assert set(declared_symbols()) - {"cin_last_error"} == set(_lib.SIGNATURES)


def test_abi_version():
    assert _lib.load().cin_abi_version() == 3


def test_no_rpath_to_a_second_hip_runtime():
    # the library must bind to the HIP runtime torch already mapped (by soname)
    out = os.popen(f"readelf -d {_lib.library_path()}").read()
    assert "libamdhip64.so.7" in out


@pytest.mark.parametrize("call", [
    ("cin_quant_rowwise", (None, 7, 4, 128, 128, 1, 128, 0, None, 128, None, 1, 1, None)),   # bad dtype
    ("cin_quant_rowwise", (None, 0, 4, 128, 128, 1, 0, 0, None, 128, None, 1, 1, None)),     # block 0
    ("cin_quant_rowwise", (None, 0, 4, 128, 128, 1, 128, 0, None, 128, None, 1, 1, None)),   # null ptr
    ("cin_quant_rowwise", (1, 0, 4, 256, 256, 1, 128, 0, 1, 256, 1, 2, 2, None)),            # scales overlap
    ("cin_quant_blockwise", (None, 0, 4, 4, 4, 1, 2048, 2048, 0, None, 4, None, 0, None, 1, None)),
    ("cin_gemm_fp8_bs", (None, 32, None, 1, 1, None, 32, None, 1, 1, 4, 4, 24, None, 0, 4, None)),
    ("cin_gemm_fp8_bs", (None, 32, None, 1, 1, None, 32, None, 1, 1, 4, 4, 32, None, 5, 4, None)),
    ("cin_dequant", (None, 4, 4, 4, 1, None, 1, 1, 1, 128, None, 2, 4, None)),            # fp16 out
    # quant_fwd: x, xdt, M, K, sxm, rs, xq, sxqm, xs, sxsm, sxsk, w, wdt, N, swm, wq, swqm, wqt, swqtm, ws,
    #            swsm, s
    ("cin_quant_fwd", (None, 9, 4, 256, 256, 0, None, 256, None, 2, 1, None, 0, 256, 256, None, 256, None, 0,
                       None, 2, None)),                                                     # bad x dtype
    ("cin_quant_fwd", (None, 0, 4, 256, 256, 0, None, 256, None, 2, 1, None, 0, 256, 256, None, 256, None, 0,
                       None, 2, None)),                                                     # null pointers
    ("cin_quant_fwd", (1, 0, 4, 256, 256, 0, 1, 128, 1, 2, 1, 1, 0, 256, 256, 1, 256, None, 0,
                       1, 2, None)),                                                        # xq stride < K
    ("cin_quant_fwd", (1, 0, 4, 256, 256, 0, 1, 256, 1, 2, 1, 1, 0, 256, 256, None, 256, None, 0,
                       1, 2, None)),                                                        # no weight output
    ("cin_quant_fwd", (1, 0, 4, 256, 256, 0, 1, 256, 1, 1, 3, 1, 0, 256, 256, 1, 256, None, 0,
                       1, 2, None)),                                                        # xs column stride < M
    # quant_backward: dy, dt, M, N, sdm, rs, q, sqm, s, ssm, ssk, qt, sqtm, st, sstm, sstk, xq, K, sxqm,
    #                 xs, sxsm, sxsk, xbt, sxbtm, sblk, ssbm, stream
    ("cin_quant_backward", (None, 9, 256, 256, 256, 0, None, 256, None, 2, 1, None, 256, None, 2, 1, None, 256,
                            256, None, 2, 1, None, 256, None, 2, None)),                    # bad dtype
    ("cin_quant_backward", (None, 0, 256, 256, 256, 0, None, 256, None, 2, 1, None, 256, None, 2, 1, None, 256,
                            256, None, 2, 1, None, 256, None, 2, None)),                    # null pointers
    ("cin_quant_backward", (1, 0, 256, 256, 256, 0, 1, 256, 1, 2, 1, 1, 256, 1, 2, 1, 8, 256, 128,
                            1, 2, 1, 8, 256, 1, 2, None)),                                  # X stride < K
    ("cin_quant_backward", (1, 0, 256, 256, 256, 0, 1, 256, 1, 1, 2, 1, 256, 1, 2, 1, 8, 256, 256,
                            1, 2, 1, 8, 256, 1, 2, None)),                                  # s column stride < M
    # swiglu_dual_grouped: dh, sdm, h12, dt, s12, T, H, starts, ends, E, rs, q, sqm, s, ssm, ssk, qt, sqtm,
    #                      st, sstm, sstk, stream
    ("cin_swiglu_dual_grouped", (1, 200, 1, 9, 400, 16, 200, 1, 1, 1, 0, 1, 400, 1, 1, 16, 1, 128, 1, 1, 1,
                                 None)),                                                     # bad h12 dtype
    ("cin_swiglu_dual_grouped", (1, 200, 1, 0, 400, 16, 200, 1, 1, 1, 0, 1, 400, 1, 1, 16, 1, 128, 1, 1, 1,
                                 None)),                                                     # H % 128
    ("cin_swiglu_dual_grouped", (None, 256, 1, 0, 512, 16, 256, 1, 1, 1, 0, 1, 512, 1, 1, 16, 1, 128, 1, 1, 1,
                                 None)),                                                     # null dh
    ("cin_moe_route", (None, 16, 2, 0, None, None, None, None, None, None, 0, None)),        # E = 0
    ("cin_moe_route", (None, 16, 2, 5000, None, None, None, None, None, None, 0, None)),     # E > 4096
    ("cin_moe_route", (None, 16, 2, 8, None, None, None, None, None, None, 0, None)),        # null ptrs
    ("cin_moe_gather_sum", (None, 1, 8, None, 4, 17, 68, 8, None, 1, 8, None)),              # k > 16
    ("cin_moe_combine", (None, 1, 8, None, 7, 2, None, 4, 2, 8, 8, None, 8, None)),          # bad score dtype
    ("cin_moe_combine", (None, 5, 8, None, 1, 2, None, 4, 2, 8, 8, None, 8, None)),          # bad y dtype
    ("cin_moe_gather_quant_rowwise", (None, 0, 4, 256, 256, None, 8, 0, 0, None, 256, None, 2, 1, None)),
    # scatter_quant_ws: x, dt, T, N, sxm, inv, k, perm, rows, rs, q, sqm, s, ssm, ssk, ws, stream
    ("cin_moe_scatter_quant_rowwise_ws", (1, 0, 4, 256, 256, 1, 2, 1, 8, 0, 1, 256, 1, 1, 8, None, None)),  # no ws
    ("cin_moe_scatter_quant_rowwise_ws", (1, 9, 4, 256, 256, 1, 2, 1, 8, 0, 1, 256, 1, 1, 8, 1, None)),     # dtype
    ("cin_moe_scatter_quant_rowwise_ws", (16, 0, 4, 256, 256, 8, 2, 8, 8, 0, 8, 256, 8, 1, 8, 4, None)),    # ws align
    ("cin_indexer_scores_fp8", (None, None, None, None, None, 1, 8, 8, 2, 48, 0.1, None, None)),   # d % 32
    ("cin_indexer_scores_fp8", (None, None, None, None, None, 1, 8, 8, 2, 288, 0.1, None, None)),  # d > 256
    ("cin_indexer_scores_fp8", (None, None, None, None, None, 1, 8, 8, 0, 64, 0.1, None, None)),   # H = 0
    ("cin_indexer_scores_fp8", (None, None, None, None, None, 1, 8, 8, 2, 64, 0.1, None, None)),   # null ptrs
    # scores_fp8_q: q, q_dtype, k8, k_scale, weights, B, L, S, H, d, softmax_scale, scores, q8, q_scale, stream
    ("cin_indexer_scores_fp8_q", (16, 9, None, None, None, 1, 8, 8, 2, 64, 0.1, None, None, None, None)),   # dtype
    ("cin_indexer_scores_fp8_q", (16, 0, None, None, None, 1, 8, 8, 5, 64, 0.1, None, None, None, None)),   # H > 4
    ("cin_indexer_scores_fp8_q", (16, 0, None, None, None, 1, 8, 8, 3, 192, 0.1, None, None, None, None)),  # H > 2
    ("cin_indexer_scores_fp8_q", (16, 0, None, None, None, 1, 8, 8, 2, 64, 0.1, None, 16, None, None)),     # q8 alone
    ("cin_indexer_scores_fp8_q", (None, 0, None, None, None, 1, 8, 8, 2, 64, 0.1, None, None, None, None)), # null q
    ("cin_indexer_scores_fp8_q", (8, 0, None, None, None, 1, 8, 8, 2, 64, 0.1, None, None, None, None)),    # q align
    ("cin_indexer_scores_fp8_q", (16, 0, None, None, None, 1, 8, 8, 2, 64, 0.1, None, None, None, None)),   # null k8
    ("cin_indexer_weights_grad", (None, None, None, None, None, 1, 8, 8, 2, 48, 0.1, None, 16, None, None)),
    ("cin_indexer_weights_grad", (None, None, None, None, None, 1, 8, 8, 2, 64, 0.1, None, 15, None, None)),
])
def test_invalid_arguments_rejected_without_gpu(call):
    name, args = call
    fn = getattr(_lib.load(), name)
    rc = fn(*[ctypes.c_void_p(0) if a is None else a for a in args])
    assert rc == _lib.CIN_ERR_ARG
    assert _lib.last_error()


def test_empty_shapes_are_noops():
    lib = _lib.load()
    # M == 0: nothing to do, no device touched
    assert lib.cin_quant_rowwise(None, 0, 0, 128, 128, 1, 128, 0, None, 128, None, 1, 1, None) == 0
    assert lib.cin_gemm_fp8_bs(None, 32, None, 1, 1, None, 32, None, 1, 1, 0, 4, 32, None, 0, 4, None) == 0
    assert lib.cin_moe_gather_sum(None, 1, 8, None, 0, 2, 0, 8, None, 1, 8, None) == 0
    assert lib.cin_moe_combine(None, 1, 8, None, 1, 2, None, 0, 2, 0, 8, None, 8, None) == 0
    assert lib.cin_indexer_scores_fp8(None, None, None, None, None, 1, 0, 8, 2, 64, 0.1, None, None) == 0
    assert lib.cin_indexer_scores_fp8_q(None, 0, None, None, None, 1, 0, 8, 2, 64, 0.1, None, None, None,
                                        None) == 0
    assert lib.cin_quant_fwd(None, 0, 0, 256, 256, 0, None, 256, None, 2, 1, None, 0, 0, 256, None, 256, None,
                             0, None, 2, None) == 0
    assert lib.cin_quant_backward(None, 0, 0, 256, 256, 0, None, 256, None, 2, 1, None, 0, None, 0, 1, None,
                                  256, 256, None, 2, 1, None, 0, None, 2, None) == 0


def test_indexer_weights_grad_workspace_size():
    lib = _lib.load()
    assert lib.cin_indexer_weights_grad_workspace(16, 1024, 1024, 4) == 2 * 16 * 1024 * 4  # 512-key ranges
    assert lib.cin_indexer_weights_grad_workspace(2, 100, 513, 3) == 2 * 2 * 100 * 3
    assert lib.cin_indexer_weights_grad_workspace(64, 32768, 32768, 64) == 64 * 64 * 32768 * 64  # > 2^31


def test_moe_route_workspace_size():
    lib = _lib.load()
    assert lib.cin_moe_route_workspace(16384, 8, 32) == 2 * 128 * 32   # 1024 assignments per block
    assert lib.cin_moe_route_workspace(1, 1, 4) == 8
    assert lib.cin_moe_route_workspace(0, 8, 4) == 0
