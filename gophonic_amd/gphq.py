"""ctypes binding of libgphq's C ABI (include/gphq.h).

This is the same binding a Python caller would add; tests and bench.py call the
library only through it. Device buffers are torch tensors (torch is used for
HBM allocation and streams only); every call passes raw device pointers and
the current torch stream to the C ABI. There is no fallback: if libgphq.so is
missing or a call fails, an exception is raised.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgphq.so")

OK = 0
ERR_INVALID_DIMENSIONS = -1
ERR_INVALID_WEIGHT_LENGTH = -2
ERR_DIMENSIONS = -3
ERR_NON_FINITE = -4
ERR_HIP = -5
ERR_UNSUPPORTED = -6

FMT_Q4, FMT_Q8, FMT_Q8B, FMT_Q8B_F32 = 4, 8, 9, 10

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_vpp = ctypes.POINTER(ctypes.c_void_p)

# name -> (restype, argtypes); every symbol include/gphq.h declares.
SIGNATURES = {
    "gphq_error_string": (ctypes.c_char_p, [ctypes.c_int]),
    "gphq_last_hip_error": (ctypes.c_int, []),
    "gphq_version": (ctypes.c_char_p, []),
    "gphq_q8gemv_mul_into": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _vp]),
    "gphq_gemv": (ctypes.c_int, [ctypes.c_int, _vp, _vp, _vp, _vp, _i64, _i64, _vp]),
    "gphq_gemv_batch": (ctypes.c_int, [ctypes.c_int, _vpp, _vpp, _vpp, _vpp, ctypes.c_int, _i64, _i64, _vp]),
}

GEMV_MAX_BATCH = 32


class GphqError(RuntimeError):
    """A libgphq status other than GPHQ_OK; .status holds the code."""

    def __init__(self, status, message):
        super().__init__(message)
        self.status = status


_lib = None


def load():
    """Loads libgphq.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run `python -m gophonic_amd.build` first")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def error_string(status):
    return load().gphq_error_string(status).decode()


def check(status):
    if status != OK:
        msg = error_string(status)
        if status == ERR_HIP:
            msg += f" (hipError_t {load().gphq_last_hip_error()})"
        raise GphqError(status, msg)
    return status


def ptr(t):
    """Device address of a torch tensor (None -> NULL)."""
    return None if t is None else t.data_ptr()


def stream_handle(stream=None):
    import torch

    s = torch.cuda.current_stream() if stream is None else stream
    return s.cuda_stream


def q8gemv_mul_into(x, q, scales, dst, k, n, stream=None):
    """q8gemv.MulInto (q8gemv/q8gemv.go:18-30) on device tensors."""
    return check(
        load().gphq_q8gemv_mul_into(
            ptr(x), x.numel(), ptr(q), q.numel(), ptr(scales), scales.numel(), ptr(dst), dst.numel(), k, n,
            stream_handle(stream),
        )
    )


def gemv(fmt, codes, scales, x, y, k, n, stream=None):
    """qwen3lm gemv<PRO_PLAIN, EPI_STORE, fmt> (gpu.metal:68-162)."""
    return check(load().gphq_gemv(fmt, ptr(codes), ptr(scales), ptr(x), ptr(y), k, n, stream_handle(stream)))


def _ptr_array(ts):
    arr = (ctypes.c_void_p * max(1, len(ts)))()
    for i, t in enumerate(ts):
        arr[i] = ptr(t)
    return arr


def gemv_batch(fmt, codes, scales, xs, ys, k, n, stream=None):
    """Several qwen3lm gemv dispatches of one shape in one launch (gphq_gemv_batch)."""
    count = len(codes)
    if not (len(scales) == len(xs) == len(ys) == count):
        raise ValueError("gemv_batch: list lengths differ")
    return check(
        load().gphq_gemv_batch(
            fmt, _ptr_array(codes), _ptr_array(scales), _ptr_array(xs), _ptr_array(ys), count, k, n,
            stream_handle(stream),
        )
    )
