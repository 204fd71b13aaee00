"""CPU checks of the C ABI: the library loads, exports every symbol that
include/gphq.h declares, maps status codes to the reference's messages, and
rejects bad arguments before touching a device (so these run without a GPU).
"""
import ctypes
import os
import re

import pytest

from gophonic_amd import gphq

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = []
    for h in os.listdir(os.path.join(ROOT, "include")):
        if h.endswith(".h"):
            text = open(os.path.join(ROOT, "include", h)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names += re.findall(r"\b(gphq_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    lib = gphq.load()
    names = declared_functions()
    assert names, "no declarations found"
    for name in names:
        assert hasattr(lib, name), name
        assert name in gphq.SIGNATURES, f"{name} has no ctypes signature"


def test_error_strings_are_the_reference_messages():
    assert gphq.error_string(gphq.ERR_INVALID_DIMENSIONS) == "q8gemv: invalid dimensions"  # q8gemv.go:20
    assert gphq.error_string(gphq.ERR_INVALID_WEIGHT_LENGTH) == "q8gemv: invalid weight length"  # q8gemv.go:24,27
    assert gphq.error_string(gphq.ERR_DIMENSIONS) == "q8gemm: invalid dimensions or buffer length"  # packed.go:26
    assert gphq.error_string(gphq.ERR_NON_FINITE) == "q8gemm: non-finite row scale"  # packed.go:27
    assert gphq.error_string(gphq.OK) == ""


# q8gemv_test.go:91-117 shape cases: (x_len, q_len, s_len, dst_len, k, n) -> status.
SHAPE_CASES = [
    ("negative-k", 0, 0, 0, 0, -1, 0, gphq.ERR_INVALID_DIMENSIONS),
    ("negative-n", 0, 0, 0, 0, 0, -1, gphq.ERR_INVALID_DIMENSIONS),
    ("activation-length", 1, 0, 0, 0, 0, 0, gphq.ERR_INVALID_DIMENSIONS),
    ("scale-length", 0, 0, 1, 0, 0, 0, gphq.ERR_INVALID_DIMENSIONS),
    ("output-length", 0, 0, 0, 1, 0, 0, gphq.ERR_INVALID_DIMENSIONS),
    ("weights-length", 1, 1, 2, 2, 1, 2, gphq.ERR_INVALID_WEIGHT_LENGTH),
    ("k0-with-weights", 0, 3, 2, 2, 0, 2, gphq.ERR_INVALID_WEIGHT_LENGTH),
    ("ragged-weights", 4, 7, 2, 2, 4, 2, gphq.ERR_INVALID_WEIGHT_LENGTH),
]


@pytest.mark.parametrize("name,xl,ql,sl,dl,k,n,want", SHAPE_CASES, ids=[c[0] for c in SHAPE_CASES])
def test_q8gemv_shape_checks_before_any_device_work(name, xl, ql, sl, dl, k, n, want):
    lib = gphq.load()
    # Non-null dummy pointers: validation must fail before any dereference.
    p = ctypes.c_void_p(16)
    got = lib.gphq_q8gemv_mul_into(p, xl, p, ql, p, sl, p, dl, k, n, None)
    assert got == want


def test_q8gemv_empty_output_is_a_no_op():
    lib = gphq.load()
    assert lib.gphq_q8gemv_mul_into(None, 0, None, 0, None, 0, None, 0, 0, 0, None) == gphq.OK
    assert lib.gphq_q8gemv_mul_into(None, 5, None, 0, None, 0, None, 0, 5, 0, None) == gphq.OK


def test_gemv_rejects_bad_formats_and_shapes():
    lib = gphq.load()
    p = ctypes.c_void_p(256)
    assert lib.gphq_gemv(3, p, p, p, p, 64, 4, None) == gphq.ERR_UNSUPPORTED
    assert lib.gphq_gemv(gphq.FMT_Q8B, p, p, p, p, 48, 4, None) == gphq.ERR_DIMENSIONS  # K % 32
    assert lib.gphq_gemv(gphq.FMT_Q4, p, p, p, p, 40, 4, None) == gphq.ERR_DIMENSIONS
    assert lib.gphq_gemv(gphq.FMT_Q8B, p, p, p, p, -32, 4, None) == gphq.ERR_DIMENSIONS
    assert lib.gphq_gemv(gphq.FMT_Q8B, ctypes.c_void_p(8), p, p, p, 64, 4, None) == gphq.ERR_DIMENSIONS  # alignment
    assert lib.gphq_gemv(gphq.FMT_Q8B, p, p, p, p, 64, 0, None) == gphq.OK  # nothing to do
