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
_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); every symbol include/gphq.h declares.
SIGNATURES = {
    "gphq_error_string": (ctypes.c_char_p, [ctypes.c_int]),
    "gphq_last_hip_error": (ctypes.c_int, []),
    "gphq_version": (ctypes.c_char_p, []),
    "gphq_q8gemv_mul_into": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _vp]),
    "gphq_gemv": (ctypes.c_int, [ctypes.c_int, _vp, _vp, _vp, _vp, _i64, _i64, _vp]),
    "gphq_gemv_batch": (ctypes.c_int, [ctypes.c_int, _vpp, _vpp, _vpp, _vpp, ctypes.c_int, _i64, _i64, _vp]),
    "gphq_gemv_vec_workspace_bytes": (_i64, [_i64, _i64]),
    "gphq_gemv_vec": (ctypes.c_int, [ctypes.c_int, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp]),
    "gphq_q8gemm_new_weights_i8": (ctypes.c_int, [_i64, _i64, _vpp]),
    "gphq_q8gemm_weights_i8_free": (None, [_vp]),
    "gphq_q8gemm_weights_i8_pack": (ctypes.c_int, [_vp, _vp, _i64, _vp, _i64]),
    "gphq_q8gemm_weights_i8_pack_rows": (ctypes.c_int, [_vp, _vp, _i64, _vp, _i64, _i64]),
    "gphq_q8gemm_weights_i8_dims": (ctypes.c_int, [_vp, _i64p, _i64p]),
    "gphq_q8gemm_weights_i8_panels": (_i64, [_vp]),
    "gphq_q8gemm_weights_i8_strips": (_i64, [_vp]),
    "gphq_q8gemm_weights_i8_bytes": (_i64, [_vp]),
    "gphq_q8gemm_new_workspace_i8": (ctypes.c_int, [_i64, _i64, _vpp]),
    "gphq_q8gemm_workspace_i8_free": (None, [_vp]),
    "gphq_q8gemm_workspace_i8_prepare": (ctypes.c_int, [_vp, _i64, _i64]),
    "gphq_q8gemm_workspace_i8_set_row_scale": (ctypes.c_int, [_vp, _i64, ctypes.c_float]),
    "gphq_q8gemm_workspace_i8_pack_range": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "gphq_q8gemm_workspace_i8_pack": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "gphq_q8gemm_workspace_i8_row_scales": (ctypes.c_int, [_vp, _vp, _vp, _vp]),
    "gphq_q8gemm_mul_panels_i8": (ctypes.c_int, [_vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp]),
    "gphq_q8gemm_mul_strips_i8": (ctypes.c_int, [_vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp]),
    "gphq_q8gemm_new_weights": (ctypes.c_int, [_i64, _i64, _vpp]),
    "gphq_q8gemm_new_weights_f16": (ctypes.c_int, [_i64, _i64, _vpp]),
    "gphq_q8gemm_weights_f16_bytes": (_i64, [_i64, _i64]),
    "gphq_q8gemm_new_weights_f16_buffer": (ctypes.c_int, [_i64, _i64, _vp, _i64, _vpp]),
    "gphq_q8gemm_weights_free": (None, [_vp]),
    "gphq_q8gemm_weights_pack": (ctypes.c_int, [_vp, _vp, _i64, _vp, _i64]),
    "gphq_q8gemm_weights_pack_bf16": (ctypes.c_int, [_vp, _vp, _i64, _i64p]),
    "gphq_q8gemm_weights_pack_bf16_rows": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i64p]),
    "gphq_q8gemm_weights_dims": (ctypes.c_int, [_vp, _i64p, _i64p]),
    "gphq_q8gemm_weights_panels": (_i64, [_vp]),
    "gphq_q8gemm_weights_bytes": (_i64, [_vp]),
    "gphq_q8gemm_weights_is_f16": (ctypes.c_int, [_vp]),
    "gphq_q8gemm_new_workspace": (ctypes.c_int, [_i64, _i64, _vpp]),
    "gphq_q8gemm_workspace_free": (None, [_vp]),
    "gphq_q8gemm_workspace_prepare": (ctypes.c_int, [_vp, _i64, _i64]),
    "gphq_q8gemm_workspace_prepare_row_f16": (ctypes.c_int, [_vp, _i64]),
    "gphq_q8gemm_workspace_prepare_rows_f16": (ctypes.c_int, [_vp, _i64, _i64]),
    "gphq_q8gemm_workspace_set_row_scale": (ctypes.c_int, [_vp, _i64, ctypes.c_float]),
    "gphq_q8gemm_workspace_pack_range": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "gphq_q8gemm_workspace_pack": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "gphq_q8gemm_workspace_row_scales": (ctypes.c_int, [_vp, _vp, _vp, _vp]),
    "gphq_q8gemm_workspace_activations": (ctypes.c_int, [_vp, _vp, _vp]),
    "gphq_q8gemm_mul_panels": (ctypes.c_int, [_vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp]),
    "gphq_q8gemm_mul_into": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i64, _vp, _vp, _vp]),
    "gphq_mm_workspace_bytes": (_i64, [_i64, _i64]),
    "gphq_mm": (ctypes.c_int, [ctypes.c_int, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _i64, _vp]),
}

FMT_GPTQ4_G128 = 12

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
        # torch ships its own libamdhip64.so.7 (same soname as /opt/rocm's).
        # The first one loaded serves the whole process, so load torch's before
        # libgphq: the binding hands torch streams and device pointers to the
        # library, and both sides must then talk to one HIP runtime.
        import torch  # noqa: F401

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


def _host(a, dtype):
    import numpy as np

    a = np.ascontiguousarray(a, dtype=dtype)
    return a, a.ctypes.data


class WeightsI8:
    """q8gemm.WeightsI8 (int8.go:13-77), device resident."""

    def __init__(self, k, n):
        h = ctypes.c_void_p()
        check(load().gphq_q8gemm_new_weights_i8(k, n, ctypes.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            load().gphq_q8gemm_weights_i8_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def pack(self, q, scales):
        import numpy as np

        q, qp = _host(q, np.int8)
        s, sp = _host(scales, np.float32)
        return check(load().gphq_q8gemm_weights_i8_pack(self.h, qp, q.size, sp, s.size))

    def pack_rows(self, q, scales, row0):
        import numpy as np

        q, qp = _host(q, np.int8)
        s, sp = _host(scales, np.float32)
        return check(load().gphq_q8gemm_weights_i8_pack_rows(self.h, qp, q.size, sp, s.size, row0))

    def dims(self):
        k, n = ctypes.c_int64(), ctypes.c_int64()
        load().gphq_q8gemm_weights_i8_dims(self.h, ctypes.byref(k), ctypes.byref(n))
        return k.value, n.value

    def panels(self):
        return load().gphq_q8gemm_weights_i8_panels(self.h)

    def strips(self):
        return load().gphq_q8gemm_weights_i8_strips(self.h)

    def bytes(self):
        return load().gphq_q8gemm_weights_i8_bytes(self.h)


class WorkspaceI8:
    """q8gemm.WorkspaceI8 (int8.go:79-168), device resident, up to max_rows rows."""

    def __init__(self, k, max_rows=16):
        h = ctypes.c_void_p()
        check(load().gphq_q8gemm_new_workspace_i8(k, max_rows, ctypes.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            load().gphq_q8gemm_workspace_i8_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def prepare(self, rows, k):
        return check(load().gphq_q8gemm_workspace_i8_prepare(self.h, rows, k))

    def set_row_scale(self, row, max_abs):
        return check(load().gphq_q8gemm_workspace_i8_set_row_scale(self.h, row, float(max_abs)))

    def pack_range(self, x, stride, k0, k1, stream=None):
        return check(
            load().gphq_q8gemm_workspace_i8_pack_range(self.h, ptr(x), x.numel(), stride, k0, k1, stream_handle(stream))
        )

    def pack(self, x, rows, k, stride=None, stream=None):
        stride = k if stride is None else stride
        return check(
            load().gphq_q8gemm_workspace_i8_pack(self.h, ptr(x), x.numel(), rows, k, stride, stream_handle(stream))
        )

    def row_scales(self, scale, inverse, stream=None):
        return check(load().gphq_q8gemm_workspace_i8_row_scales(self.h, ptr(scale), ptr(inverse), stream_handle(stream)))


def mul_panels_i8(dst, stride, ws, w, p0, p1, stream=None):
    """q8gemm.MulPanelsI8 (int8.go:174-197)."""
    return check(load().gphq_q8gemm_mul_panels_i8(ptr(dst), dst.numel(), stride, ws.h, w.h, p0, p1, stream_handle(stream)))


def mul_strips_i8(dst, stride, ws, w, s0, s1, stream=None):
    """q8gemm.MulStripsI8 (int8.go:224-241)."""
    return check(load().gphq_q8gemm_mul_strips_i8(ptr(dst), dst.numel(), stride, ws.h, w.h, s0, s1, stream_handle(stream)))


class Weights:
    """q8gemm.Weights (packed.go:35-239): int8 (f16=False) or FP16 storage, device resident.
    With `buffer` (a device tensor of weights_f16_bytes(k, n) bytes) it binds
    caller-owned storage like NewWeightsF16Buffer."""

    def __init__(self, k, n, f16=False, buffer=None):
        h = ctypes.c_void_p()
        self._buffer = buffer
        if buffer is not None:
            check(load().gphq_q8gemm_new_weights_f16_buffer(k, n, ptr(buffer), buffer.numel() * buffer.element_size(),
                                                             ctypes.byref(h)))
        elif f16:
            check(load().gphq_q8gemm_new_weights_f16(k, n, ctypes.byref(h)))
        else:
            check(load().gphq_q8gemm_new_weights(k, n, ctypes.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            load().gphq_q8gemm_weights_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def pack(self, q, scales):
        import numpy as np

        q, qp = _host(q, np.int8)
        s, sp = _host(scales, np.float32)
        return check(load().gphq_q8gemm_weights_pack(self.h, qp, q.size, sp, s.size))

    def pack_bf16(self, bf16):
        import numpy as np

        b, bp = _host(bf16, np.uint16)
        r = ctypes.c_int64()
        check(load().gphq_q8gemm_weights_pack_bf16(self.h, bp, b.size, ctypes.byref(r)))
        return r.value

    def pack_bf16_rows(self, bf16, row0):
        import numpy as np

        b, bp = _host(bf16, np.uint16)
        r = ctypes.c_int64()
        check(load().gphq_q8gemm_weights_pack_bf16_rows(self.h, bp, b.size, row0, ctypes.byref(r)))
        return r.value

    def dims(self):
        k, n = ctypes.c_int64(), ctypes.c_int64()
        load().gphq_q8gemm_weights_dims(self.h, ctypes.byref(k), ctypes.byref(n))
        return k.value, n.value

    def panels(self):
        return load().gphq_q8gemm_weights_panels(self.h)

    def bytes(self):
        return load().gphq_q8gemm_weights_bytes(self.h)

    def f16(self):
        return bool(load().gphq_q8gemm_weights_is_f16(self.h))


def weights_f16_bytes(k, n):
    return load().gphq_q8gemm_weights_f16_bytes(k, n)


class Workspace:
    """q8gemm.Workspace (gemm.go:20-226), device resident, up to max_rows rows."""

    def __init__(self, k, max_rows=16):
        h = ctypes.c_void_p()
        check(load().gphq_q8gemm_new_workspace(k, max_rows, ctypes.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            load().gphq_q8gemm_workspace_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def prepare(self, rows, k):
        return check(load().gphq_q8gemm_workspace_prepare(self.h, rows, k))

    def prepare_row_f16(self, k):
        return check(load().gphq_q8gemm_workspace_prepare_row_f16(self.h, k))

    def prepare_rows_f16(self, rows, k):
        return check(load().gphq_q8gemm_workspace_prepare_rows_f16(self.h, rows, k))

    def set_row_scale(self, row, max_abs):
        return check(load().gphq_q8gemm_workspace_set_row_scale(self.h, row, float(max_abs)))

    def pack_range(self, x, stride, k0, k1, stream=None):
        return check(
            load().gphq_q8gemm_workspace_pack_range(self.h, ptr(x), x.numel(), stride, k0, k1, stream_handle(stream))
        )

    def pack(self, x, rows, k, stride=None, stream=None):
        stride = k if stride is None else stride
        return check(load().gphq_q8gemm_workspace_pack(self.h, ptr(x), x.numel(), rows, k, stride, stream_handle(stream)))

    def row_scales(self, scale, inverse, stream=None):
        return check(load().gphq_q8gemm_workspace_row_scales(self.h, ptr(scale), ptr(inverse), stream_handle(stream)))

    def activations(self, out, stream=None):
        return check(load().gphq_q8gemm_workspace_activations(self.h, ptr(out), stream_handle(stream)))


def mul_panels(dst, stride, ws, w, p0, p1, stream=None):
    """q8gemm.MulPanels (gemm.go:228-272)."""
    return check(load().gphq_q8gemm_mul_panels(ptr(dst), dst.numel(), stride, ws.h, w.h, p0, p1, stream_handle(stream)))


def mul_into(dst, x, rows, w, ws, stream=None):
    """q8gemm.MulInto (gemm.go:274-286)."""
    return check(load().gphq_q8gemm_mul_into(ptr(dst), dst.numel(), ptr(x), x.numel(), rows, w.h, ws.h, stream_handle(stream)))


def mm_workspace_bytes(m, k):
    return load().gphq_mm_workspace_bytes(m, k)


def mm(fmt, codes, scales, x, y, m, k, n, work, zeros=None, stream=None):
    """qwen3lm mm<PRO_PLAIN, EPI_STORE, fmt> (gpu.metal:766-927) or the GPTQ4_G128 variant."""
    return check(
        load().gphq_mm(fmt, ptr(codes), ptr(scales), ptr(zeros), ptr(x), ptr(y), m, k, n, ptr(work),
                       work.numel() * work.element_size(), stream_handle(stream))
    )


GEMV_VEC_MAX_LANES = 32


def gemv_vec_workspace_bytes(lanes, k):
    return load().gphq_gemv_vec_workspace_bytes(lanes, k)


def gemv_vec(fmt, codes, scales, x, y, lanes, k, n, work, x_stride=None, y_stride=None, stream=None):
    """Multi-vector GEMV (qwen3lm gemvQ8BVector<V>, gpu.metal:239-314): x [lanes][k] -> y [lanes][n]."""
    x_stride = k if x_stride is None else x_stride
    y_stride = n if y_stride is None else y_stride
    return check(
        load().gphq_gemv_vec(fmt, ptr(codes), ptr(scales), ptr(x), x_stride, ptr(y), y_stride, lanes, k, n, ptr(work),
                             work.numel() * work.element_size(), stream_handle(stream))
    )
