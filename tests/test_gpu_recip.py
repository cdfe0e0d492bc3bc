"""The SwiGLU backward's sigmoid reciprocal (recip_ge1 in cinnamon_amd/csrc/cin_common.h:
v_rcp_f32 and one Newton step for d in [1, 2^126), the division above) against the IEEE
division 1.0f / d on every fp32 d >= 1: all 2^30 finite values, infinity and the positive
NaNs, compared on the device by tests/gpu_checks/recip_check.hip (built by build())."""
import ctypes
import os

import pytest

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(__file__), "gpu_checks", "librecip_check.so")


def test_recip_ge1_equals_the_division_for_every_d_at_least_one(dev):
    assert os.path.exists(LIB), f"{LIB} is missing: run __graft_entry__.build()"
    lib = ctypes.CDLL(LIB)
    f = lib.cin_test_recip_ge1_mismatches
    f.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint32)]
    f.restype = ctypes.c_longlong
    first_bad = ctypes.c_uint32(0)
    n = f(0x3F800000, 0x7FFFFFFF, ctypes.byref(first_bad))  # 1.0 up to the largest positive NaN
    assert n >= 0, "HIP error in the check"
    assert n == 0, f"{n} mismatches, the first at bits {first_bad.value:#010x}"
