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
ERR_GEOMETRY = -7
ERR_FOREIGN_WORKSPACE = -8
ERR_BATCH_SHAPE = -9
ERR_LANE_CAPACITY = -10
ERR_FOREIGN_PREFIX = -11
ERR_DUPLICATE_PREFIX = -12
ERR_PREFIX_FULL = -13
ERR_TOKEN_RANGE = -14
ERR_OVERLAP = -15
ERR_NON_FINITE_HIDDEN = -16
ERR_MODEL_INCOMPLETE = -17
ERR_WORKSPACE = -18
ERR_KEEP_RANGE = -19
ERR_PREFIX_CAPACITY = -20
ERR_EMPTY_SEQUENCE = -21
ERR_CONTEXT = -22
ERR_DEST_WIDTH = -23
ERR_TOKEN_VOCAB = -24
ERR_NON_FINITE_STATE = -25
ERR_NOT_POSITIVE_DEFINITE = -26
ERR_SEQUENCE_COUNT = -27
ERR_PASS_ROWS = -28
ERR_LOGITS_SHAPE = -29
ERR_SCRATCH_LIMIT = -30
ERR_TAIL_SHAPE = -31
ERR_REUSE = -32
ERR_EMBED_ROWS = -33
ERR_IO = -34
ERR_FORMAT = -35
ERR_TENSOR_MISSING = -36
ERR_TENSOR_SHAPE = -37
ERR_TENSOR_DTYPE = -38
ERR_TENSOR_NON_FINITE = -39
ERR_READ_RANGE = -40
ERR_GPTQ_WIDTH = -41
ERR_CALIBRATION_EMPTY = -42
ERR_CALIBRATION_SHAPE = -43
TAIL_MAX_ROWS = 256

FMT_Q4, FMT_Q8, FMT_Q8B, FMT_Q8B_F32 = 4, 8, 9, 10
PASS_FP16, PASS_INT8 = 0, 1  # gphq_prefill_set_arith

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_vpp = ctypes.POINTER(ctypes.c_void_p)
_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); every symbol include/gphq.h declares.
SIGNATURES = {
    "gphq_error_string": (ctypes.c_char_p, [ctypes.c_int]),
    "gphq_error_detail": (ctypes.c_char_p, []),
    "gphq_checkpoint_open": (ctypes.c_int, [ctypes.c_char_p, _vpp]),
    "gphq_checkpoint_close": (None, [_vp]),
    "gphq_checkpoint_has": (ctypes.c_int, [_vp, ctypes.c_char_p]),
    "gphq_checkpoint_info": (ctypes.c_int, [_vp, ctypes.c_char_p, _vp, _vp, _i64, _i64p]),
    "gphq_checkpoint_lookup": (ctypes.c_int, [_vp, ctypes.c_char_p, _vp, _i64, _vp]),
    "gphq_checkpoint_read_bits": (ctypes.c_int, [_vp, ctypes.c_char_p, _vp, _i64, _i64]),
    "gphq_checkpoint_bf16": (ctypes.c_int, [_vp, ctypes.c_char_p, _vp, _i64, _vp, _i64]),
    "gphq_checkpoint_bf16_device": (ctypes.c_int, [_vp, ctypes.c_char_p, _vp, _i64, _vp, _i64]),
    "gphq_checkpoint_float32": (ctypes.c_int, [_vp, ctypes.c_char_p, _vp, _i64, _vp, _i64]),
    "gphq_checkpoint_map_bf16": (ctypes.c_int, [_vp, ctypes.c_char_p, _vp, _i64, _vpp, _vpp]),
    "gphq_mapping_free": (None, [_vp]),
    "gphq_gptq_row_bytes": (ctypes.c_int, [ctypes.c_int, _i64, _i64p, _i64p]),
    "gphq_gptq_fingerprint": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64)]),
    "gphq_gptq_path": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, _i64]),
    "gphq_gptq_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, _vp, _vpp]),
    "gphq_gptq_close": (None, [_vp]),
    "gphq_gptq_bits": (ctypes.c_int, [_vp]),
    "gphq_gptq_projection": (ctypes.c_int, [_vp, ctypes.c_char_p, _i64p, _i64p]),
    "gphq_gptq_place": (ctypes.c_int, [_vp, ctypes.c_char_p, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _i64,
                                       ctypes.POINTER(ctypes.c_int)]),
    "gphq_gptq_create": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, _vpp]),
    "gphq_gptq_write": (ctypes.c_int, [_vp, _vp, _i64]),
    "gphq_gptq_write_device": (ctypes.c_int, [_vp, _vp, _i64]),
    "gphq_gptq_commit": (ctypes.c_int, [_vp]),
    "gphq_gptq_abort": (None, [_vp]),
    "gphq_wcache_round_up": (_i64, [_i64]),
    "gphq_wcache_key": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, _vp, _i64, ctypes.c_char_p, _i64]),
    "gphq_wcache_sha256": (ctypes.c_int, [_vp, _i64, _vp]),
    "gphq_wcache_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, _i64, _vpp]),
    "gphq_wcache_fresh": (ctypes.c_int, [_vp]),
    "gphq_wcache_payload": (_vp, [_vp, _i64p]),
    "gphq_wcache_done": (None, [_vp, _vp, _i64]),
    "gphq_wcache_commit": (None, [_vp]),
    "gphq_wcache_close": (ctypes.c_int, [_vp]),
    "gphq_last_hip_error": (ctypes.c_int, []),
    "gphq_version": (ctypes.c_char_p, []),
    "gphq_q8gemv_mul_into": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _vp]),
    "gphq_gemv": (ctypes.c_int, [ctypes.c_int, _vp, _vp, _vp, _vp, _i64, _i64, _vp]),
    "gphq_gemv_batch": (ctypes.c_int, [ctypes.c_int, _vpp, _vpp, _vpp, _vpp, ctypes.c_int, _i64, _i64, _vp]),
    "gphq_gemv_vec_workspace_bytes": (_i64, [_i64, _i64]),
    "gphq_gemv_vec": (ctypes.c_int, [ctypes.c_int, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp]),
    "gphq_gemv_vec_noalloc": (ctypes.c_int, [ctypes.c_int, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp]),
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
    "gphq_q8gemm_reference_f16_bytes": (_i64, [_i64, _i64]),
    "gphq_q8gemm_weights_f16_load_reference": (ctypes.c_int, [_vp, _vp, _i64]),
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
    "gphq_lm_layer_layout": (ctypes.c_int, [_vp, _vp, _i64p]),
    "gphq_lm_head_layout": (ctypes.c_int, [_vp, _i64p, _i64p, _i64p]),
    "gphq_lm_new": (ctypes.c_int, [_vp, _vpp]),
    "gphq_lm_free": (None, [_vp]),
    "gphq_lm_bind_layer": (ctypes.c_int, [_vp, _i64, _vp]),
    "gphq_lm_bind_embed": (ctypes.c_int, [_vp, _vp, _i64]),
    "gphq_lm_bind_head": (ctypes.c_int, [_vp, _vp, _i64, _vp]),
    "gphq_prefix_new": (ctypes.c_int, [_vp, _i64, _vpp]),
    "gphq_prefix_free": (None, [_vp]),
    "gphq_prefix_kv": (ctypes.c_int, [_vp, _vpp, _vpp, _i64p]),
    "gphq_prefix_copy": (ctypes.c_int, [_vp, _vp, _i64, _vp]),
    "gphq_decode_batch_new": (ctypes.c_int, [_vp, _i64, _vpp]),
    "gphq_decode_batch_free": (None, [_vp]),
    "gphq_decode_batch_set_vec_min_lanes": (ctypes.c_int, [_vp, _i64]),
    "gphq_decode_batch_into": (ctypes.c_int, [_vp, _vpp, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _vp]),
    "gphq_decode_batch_greedy_into": (ctypes.c_int, [_vp, _vpp, _i64, _vp, _vp, _vp, _i64, _vp, _vp]),
    "gphq_decode_greedy_run": (ctypes.c_int, [_vp, _vpp, _i64, _vp, _vp, _i64, _vp, _i64, _vp, _i64, _vp]),
    "gphq_decode_extend": (ctypes.c_int, [_vp, _vpp, _i64, _vp, _vp, _i64, _vp]),
    "gphq_decode_batch_check": (ctypes.c_int, [_vp, _vp]),
    "gphq_decode_batch_logits": (ctypes.c_int, [_vp, _vp, _i64, _vp, _i64, _vp]),
    "gphq_decode_batch_set_graph": (ctypes.c_int, [_vp, ctypes.c_int]),
    "gphq_prepare_work_bytes": (_i64, [_i64, _i64]),
    "gphq_prepare_projection": (ctypes.c_int, [_vp, _vp, _i64, _vp]),
    "gphq_prepare_layer_jobs": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _vp]),
    "gphq_prepare_head_chunk_rows": (_i64, [_vp]),
    "gphq_prepare_head_job": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp]),
    "gphq_prepare_lm_work_bytes": (_i64, [_vp]),
    "gphq_prepare_layer": (ctypes.c_int, [_vp, _vpp, _vp, _vp, _vp, _i64, _vp, _i64, _vp]),
    "gphq_prepare_head": (ctypes.c_int, [_vp, _vp, _vp, _i64, _vp, _i64, _vp]),
    "gphq_mm_split_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "gphq_prefill_new": (ctypes.c_int, [_vp, _i64, _vpp]),
    "gphq_prefill_free": (None, [_vp]),
    "gphq_prefill_rows": (ctypes.c_int, [_vp]),
    "gphq_prefill_extend": (ctypes.c_int, [_vp, _vp, _i64, _vp, _i64, _vp, _i64, _vp]),
    "gphq_prefill_extend_embed": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _vp]),
    "gphq_prefill_batch": (ctypes.c_int, [_vp, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _vp]),
    "gphq_q8b_quantize": (ctypes.c_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp]),
    "gphq_q8b_gemm": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "gphq_prefill_check": (ctypes.c_int, [_vp, _vp]),
    "gphq_prefill_set_arith": (ctypes.c_int, [_vp, ctypes.c_int]),
    "gphq_prefill_arith": (ctypes.c_int, [_vp]),
    "gphq_prefill_project": (ctypes.c_int, [_vp, _i64, ctypes.c_int, _vp, _i64, _vp, _vp]),
    "gphq_gptq_work_bytes": (_i64, [_i64]),
    "gphq_gptq_factor": (ctypes.c_int, [_vp, _i64, _i64, _vp, _vp, _vp, _i64, _vp]),
    "gphq_gptq_round_work_bytes": (_i64, [_i64, _i64]),
    "gphq_gptq_round": (ctypes.c_int, [_vp, _i64, _i64, _vp, _vp, ctypes.c_int, _vp, _vp, _vp, _i64, _vp]),
    "gphq_gptq_calibration_new": (ctypes.c_int, [_vp, _vp, _vp, _i64, _vp, _i64, _vpp, _vp]),
    "gphq_gptq_calibration_free": (None, [_vp]),
    "gphq_gptq_calibration_layer": (ctypes.c_int, [_vp, _vpp, _vp, _vp, _vp, _vp, ctypes.c_int, _vpp, _vpp, _vp]),
    "gphq_gptq_calibration_rows": (ctypes.c_int, [_vp, ctypes.c_int, _vp, _i64, _i64p, _i64p, _vp]),
    "gphq_gptq_calibration_sequences": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i64p]),
    "gphq_gptq_quantize": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, _vp, _vp, _vp, _i64, _vp, _vp, _vp]),
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

    def load_reference(self, ref_bytes):
        """Loads FP16 weights from the reference's own packed buffer bytes
        (panels [n/64][k/2][64][2] then n fp32 scales; a numpy uint8 array)."""
        import numpy as np

        b, bp = _host(np.asarray(ref_bytes).view(np.uint8).reshape(-1), np.uint8)
        return check(load().gphq_q8gemm_weights_f16_load_reference(self.h, bp, b.size))

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


def mm_split_workspace_bytes(m, k, n):
    return load().gphq_mm_split_workspace_bytes(m, k, n)


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


GEMV_VEC_NOALLOC_BYTES = 4 << 20


def gemv_vec_noalloc(fmt, codes, scales, x, y, lanes, k, n, x_stride=None, y_stride=None, stream=None):
    """gemv_vec with the library's static scratch (gphq_gemv_vec_noalloc): allocates nothing."""
    x_stride = k if x_stride is None else x_stride
    y_stride = n if y_stride is None else y_stride
    return check(
        load().gphq_gemv_vec_noalloc(fmt, ptr(codes), ptr(scales), ptr(x), x_stride, ptr(y), y_stride, lanes, k, n,
                                     stream_handle(stream))
    )


# ---- qwen3lm decode provider (gphq_lm_* / gphq_prefix_* / gphq_decode_*) ----

DECODE_MAX_LANES = 32


class LmConfig(ctypes.Structure):
    """gphq_lm_config: model geometry and the layer weight format."""

    _fields_ = [(n, ctypes.c_int64) for n in ("hidden", "layers", "heads", "kv_heads", "head_dim", "intermediate",
                                               "vocab", "max_positions")] + [
        ("eps", ctypes.c_double), ("rope_theta", ctypes.c_double), ("fmt", ctypes.c_int32),
        ("reserved", ctypes.c_int32)]


class LmLayer(ctypes.Structure):
    """gphq_lm_layer: one layer's device buffer, byte offsets and head norms."""

    _fields_ = [("buf_dev", ctypes.c_void_p), ("buf_bytes", ctypes.c_int64)] + [
        (n, ctypes.c_int64) for n in ("qkv", "qkv_scale", "o", "o_scale", "gu", "gu_scale", "d", "d_scale")] + [
        ("q_norm_host", ctypes.c_void_p), ("k_norm_host", ctypes.c_void_p)]


def lm_config(hidden, layers, heads, kv_heads, head_dim, intermediate, vocab, max_positions, fmt, eps=1e-6,
              rope_theta=1e6):
    return LmConfig(hidden, layers, heads, kv_heads, head_dim, intermediate, vocab, max_positions, eps, rope_theta,
                    fmt, 0)


def lm_layer_layout(cfg):
    """gpu_darwin.go place(): (LmLayer with offsets, total bytes)."""
    L, n = LmLayer(), ctypes.c_int64()
    check(load().gphq_lm_layer_layout(ctypes.byref(cfg), ctypes.byref(L), ctypes.byref(n)))
    return L, n.value


def lm_head_layout(cfg):
    """loadHead's buffer: (rows, scale_offset, bytes)."""
    r, so, n = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    check(load().gphq_lm_head_layout(ctypes.byref(cfg), ctypes.byref(r), ctypes.byref(so), ctypes.byref(n)))
    return r.value, so.value, n.value


class Lm:
    """gphq_lm: a device-resident qwen3lm model (gpuModel). Bound device
    buffers are kept alive by this object."""

    def __init__(self, cfg):
        h = ctypes.c_void_p()
        check(load().gphq_lm_new(ctypes.byref(cfg), ctypes.byref(h)))
        self.h, self.cfg, self._keep = h, cfg, []

    def close(self):
        if self.h:
            load().gphq_lm_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def bind_layer(self, layer, buf, desc, q_norm, k_norm):
        """buf: uint8 device tensor laid out as desc (from lm_layer_layout)."""
        import numpy as np

        qn, qp = _host(q_norm, np.float32)
        kn, kp = _host(k_norm, np.float32)
        d = LmLayer.from_buffer_copy(desc)
        d.buf_dev, d.buf_bytes = buf.data_ptr(), buf.numel() * buf.element_size()
        d.q_norm_host, d.k_norm_host = qp, kp
        check(load().gphq_lm_bind_layer(self.h, layer, ctypes.byref(d)))
        self._keep.append(buf)

    def bind_embed(self, embed):
        """embed: int16/uint16-bit BF16 device tensor [vocab][hidden]."""
        check(load().gphq_lm_bind_embed(self.h, embed.data_ptr(), embed.numel()))
        self._keep.append(embed)

    def bind_head(self, head, final_norm):
        import numpy as np

        fn, fp = _host(final_norm, np.float32)
        check(load().gphq_lm_bind_head(self.h, head.data_ptr(), head.numel() * head.element_size(), fp))
        self._keep.append(head)


class Prefix:
    """gphq_prefix: one lane's K/V cache (gpuPrefix)."""

    def __init__(self, lm, capacity):
        h = ctypes.c_void_p()
        check(load().gphq_prefix_new(lm.h, capacity, ctypes.byref(h)))
        self.h, self.lm, self.capacity = h, lm, capacity

    def close(self):
        if self.h:
            load().gphq_prefix_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def kv(self):
        """(kc, vc) device addresses and the capacity."""
        k, v, c = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_int64()
        check(load().gphq_prefix_kv(self.h, ctypes.byref(k), ctypes.byref(v), ctypes.byref(c)))
        return k.value, v.value, c.value

    def copy_from(self, src, n, stream=None):
        check(load().gphq_prefix_copy(self.h, src.h, n, stream_handle(stream)))


def _prefix_array(kvs):
    arr = (ctypes.c_void_p * len(kvs))()
    for i, p in enumerate(kvs):
        arr[i] = p.h.value if p is not None and p.h else None
    return arr


class DecodeBatch:
    """gphq_decode_batch: scratch for up to `capacity` lanes (gpuDecodeBatchWorkspace)."""

    def __init__(self, lm, capacity):
        h = ctypes.c_void_p()
        check(load().gphq_decode_batch_new(lm.h, capacity, ctypes.byref(h)))
        self.h, self.lm, self.capacity = h, lm, capacity

    def close(self):
        if self.h:
            load().gphq_decode_batch_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_vec_min_lanes(self, lanes):
        check(load().gphq_decode_batch_set_vec_min_lanes(self.h, lanes))

    def set_graph(self, on):
        check(load().gphq_decode_batch_set_graph(self.h, 1 if on else 0))

    @staticmethod
    def _args(positions, tokens):
        import numpy as np

        pos, pp = _host(positions, np.int64)
        tok, tp = _host(tokens, np.int32)
        return pos, pp, tok, tp

    def into(self, kvs, positions, tokens, hidden, logits, stream=None):
        """DecodeBatchInto: hidden [lanes][hidden], logits [lanes][vocab] device tensors."""
        pos, pp, tok, tp = self._args(positions, tokens)
        check(load().gphq_decode_batch_into(self.h, _prefix_array(kvs), len(kvs), pp, tp, ptr(hidden),
                                            0 if hidden is None else hidden.numel(), ptr(logits),
                                            0 if logits is None else logits.numel(), stream_handle(stream)))

    def greedy_into(self, kvs, positions, tokens, hidden, next_tokens, stream=None):
        """DecodeBatchGreedyInto: next_tokens int32 [lanes] device tensor."""
        pos, pp, tok, tp = self._args(positions, tokens)
        check(load().gphq_decode_batch_greedy_into(self.h, _prefix_array(kvs), len(kvs), pp, tp, ptr(hidden),
                                                   0 if hidden is None else hidden.numel(), ptr(next_tokens),
                                                   stream_handle(stream)))

    def greedy_run(self, kvs, positions, tokens, steps, tokens_out, hidden=None, stream=None):
        """`steps` chained greedy steps; tokens_out int32 [steps][lanes] device tensor."""
        pos, pp, tok, tp = self._args(positions, tokens)
        check(load().gphq_decode_greedy_run(self.h, _prefix_array(kvs), len(kvs), pp, tp, steps, ptr(tokens_out),
                                            tokens_out.numel(), ptr(hidden), 0 if hidden is None else hidden.numel(),
                                            stream_handle(stream)))

    def extend(self, kvs, positions, tokens, stream=None):
        """Teacher-forced steps; tokens [steps][lanes] host array."""
        import numpy as np

        pos, pp = _host(positions, np.int64)
        tok = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1, len(kvs))
        check(load().gphq_decode_extend(self.h, _prefix_array(kvs), len(kvs), pp, tok.ctypes.data, tok.shape[0],
                                        stream_handle(stream)))

    def logits(self, hidden, logits, stream=None):
        """LogitsRowsInto: hidden [k][hidden] post-final-norm states, logits [k][vocab] device tensors."""
        check(load().gphq_decode_batch_logits(self.h, ptr(hidden), 0 if hidden is None else hidden.numel(),
                                              ptr(logits), 0 if logits is None else logits.numel(),
                                              stream_handle(stream)))

    def check(self, stream=None):
        return check(load().gphq_decode_batch_check(self.h, stream_handle(stream)))


class Embeds(ctypes.Structure):
    """gphq_embeds: placeholder token and its replacement rows (evaluator.go:155-163)."""

    _fields_ = [("token", ctypes.c_int32), ("reserved", ctypes.c_int32), ("rows_dev", ctypes.c_void_p),
                ("rows_len", ctypes.c_int64)]


class Prefill:
    """gphq_prefill: the batched pass's scratch for up to `rows` tokens per pass
    (gpuWorkspace, gpu_darwin.go:895-960)."""

    def __init__(self, lm, rows):
        h = ctypes.c_void_p()
        check(load().gphq_prefill_new(lm.h, rows, ctypes.byref(h)))
        self.h, self.lm, self.rows = h, lm, rows

    def close(self):
        if self.h:
            load().gphq_prefill_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def extend(self, kv, keep, tokens, hidden, stream=None):
        """HiddenLastExtendInto (evaluator.go:146): tokens (host ints) continue
        the first `keep` rows of kv; hidden [hidden] device tensor receives the
        last token's post-final-norm state."""
        import numpy as np

        tok = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
        check(load().gphq_prefill_extend(self.h, kv.h if kv is not None else None, keep, tok.ctypes.data, tok.size,
                                         ptr(hidden), 0 if hidden is None else hidden.numel(), stream_handle(stream)))

    def extend_embed(self, kv, stored, keep, tokens, tail, embeds_token=0, embeds_rows=None, reuse=0, stream=None):
        """HiddenTailContinueEmbedInto (evaluator.go:293-310): tokens (host
        ints) continue the first `keep` of the `stored` tokens of kv;
        placeholders equal to embeds_token take the rows of embeds_rows (a
        float32 device tensor [occurrences][hidden]) when given; tail (a
        float32 device tensor [k][hidden], or [hidden] for k = 1) receives the
        post-final-norm states of the last k positions."""
        import numpy as np

        tok = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
        emb = None
        if embeds_rows is not None:
            emb = Embeds(int(embeds_token), 0, ptr(embeds_rows), embeds_rows.numel())
        check(load().gphq_prefill_extend_embed(self.h, kv.h if kv is not None else None, stored, keep, reuse,
                                               tok.ctypes.data if tok.size else None, tok.size,
                                               None if emb is None else ctypes.byref(emb), ptr(tail),
                                               0 if tail is None else tail.numel(), stream_handle(stream)))

    def batch(self, seqs, hidden, shared=None, past=0, stream=None):
        """HiddenLastBatchInto (evaluator.go:531), or HiddenLastSharedInto
        (evaluator.go:413) with `shared` (a Prefix holding `past` tokens, only
        read): seqs is a list of host token lists; hidden [len(seqs), hidden]
        device tensor receives each sequence's last-token state."""
        import numpy as np

        lens = np.array([len(q) for q in seqs], dtype=np.int64)
        flat = np.ascontiguousarray(np.concatenate([np.asarray(q, dtype=np.int64) for q in seqs])
                                    if len(seqs) else np.zeros(0), dtype=np.int32)
        check(load().gphq_prefill_batch(self.h, shared.h if shared is not None else None, past,
                                        flat.ctypes.data if flat.size else None, lens.ctypes.data if lens.size else None,
                                        len(seqs), ptr(hidden), 0 if hidden is None else hidden.numel(),
                                        stream_handle(stream)))

    def check(self, stream=None):
        return check(load().gphq_prefill_check(self.h, stream_handle(stream)))

    def set_arith(self, arith):
        """PASS_FP16 (the GPU provider's mm) or PASS_INT8 (the CPU provider's
        int8 route, Q8 layers only)."""
        check(load().gphq_prefill_set_arith(self.h, arith))

    @property
    def arith(self):
        return load().gphq_prefill_arith(self.h)

    def project(self, layer, proj, x, rows, y, stream=None):
        """One projection of a pass (0 QKV, 1 O add, 2 gate/up SwiGLU, 3 down
        add) on `rows` rows of device tensor x into device tensor y."""
        check(load().gphq_prefill_project(self.h, layer, proj, ptr(x), rows, ptr(y), stream_handle(stream)))


def lm_from_stored(geom_kwargs, fmt, layers, embed_bf16, final_norm, head, device="cuda"):
    """Builds a device model from stored (already quantized) host weights, as
    loadGPU uploads prepareGPU's buffers: per layer one buffer with the
    reference's placement. layers: objects with .qkv/.o/.gu/.down = (codes,
    scales) numpy arrays and .q_norm/.k_norm; head = (codes, scales) of the
    padded Q8B head."""
    import numpy as np
    import torch

    cfg = lm_config(fmt=fmt, **geom_kwargs)
    desc, nbytes = lm_layer_layout(cfg)
    lm = Lm(cfg)

    def put(buf, off, a):
        b = np.ascontiguousarray(a).view(np.uint8).reshape(-1)
        buf[off:off + b.size] = torch.from_numpy(b.copy())

    for i, L in enumerate(layers):
        host = torch.zeros(nbytes, dtype=torch.uint8)
        for (c, sc), (wo, so) in zip((L.qkv, L.o, L.gu, L.down), ((desc.qkv, desc.qkv_scale), (desc.o, desc.o_scale),
                                                                   (desc.gu, desc.gu_scale), (desc.d, desc.d_scale))):
            put(host, wo, c)
            put(host, so, sc)
        lm.bind_layer(i, host.to(device), desc, L.q_norm, L.k_norm)
    emb = torch.from_numpy(np.ascontiguousarray(embed_bf16).view(np.int16).reshape(cfg.vocab, cfg.hidden).copy())
    lm.bind_embed(emb.to(device))
    rows, so, hb = lm_head_layout(cfg)
    host = torch.zeros(hb, dtype=torch.uint8)
    put(host, 0, head[0])
    put(host, so, head[1])
    lm.bind_head(host.to(device), final_norm)
    return lm


def lm_random(geom_kwargs, fmt, seed, device="cuda", host=False):
    """A random-init Qwen3-shaped model in the qwen3lm GPU layout, generated on
    the device with a seeded torch generator (lmtest's distributions,
    lmtest/lmtest.go:34-80): int8 codes U[-127,127] (Q4: bytes U[0,255]),
    scales |N(0,1)|*0.02, norms 1 + N(0,0.02), BF16 embeddings N(0,1), and a
    Q8B head padded to 16 rows with zeros.

    Returns (lm, weight_bytes, stored): weight_bytes are the layer and head
    codes and scales one decode step reads; stored is None, or with host=True
    a dict of host copies (layers: list of dicts qkv/o/gu/down = (codes,
    scales) and q_norm/k_norm; embed (uint16 BF16 bits); final_norm; head =
    (codes, scales)) for a CPU check of the same model."""
    import numpy as np
    import torch

    cfg = lm_config(fmt=fmt, **geom_kwargs)
    desc, nbytes = lm_layer_layout(cfg)
    lm = Lm(cfg)
    gen = torch.Generator(device=device).manual_seed(seed)
    rng = np.random.default_rng(seed)
    H, I, hd = cfg.hidden, cfg.intermediate, cfg.head_dim
    qd, kvd = cfg.heads * hd, cfg.kv_heads * hd
    regions = [("qkv", desc.qkv, desc.qkv_scale, qd + 2 * kvd, H), ("o", desc.o, desc.o_scale, H, qd),
               ("gu", desc.gu, desc.gu_scale, 2 * I, H), ("down", desc.d, desc.d_scale, H, I)]

    def fill(buf, w, s, rows, k, f, pad_rows=0):
        """Random codes and scales of `rows` rows (then `pad_rows` zero rows) at
        byte offsets w and s of buf; returns (bytes, host codes, host scales)."""
        rk = rows * k
        if f == FMT_Q4:
            nc = rk // 2
            buf[w:w + nc].copy_(torch.randint(0, 256, (nc,), dtype=torch.uint8, device=device, generator=gen))
            codes = buf[w:w + nc]
        else:
            nc = rk
            codes = buf[w:w + nc].view(torch.int8)
            codes.copy_(torch.randint(-127, 128, (nc,), dtype=torch.int8, device=device, generator=gen))
        ns = rows if f == FMT_Q8 else rk // 32
        sc = torch.randn(ns, device=device, generator=gen).abs() * 0.02
        if f in (FMT_Q8, FMT_Q8B_F32):
            scales = buf[s:s + 4 * ns].view(torch.float32)
            scales.copy_(sc)
            sb = 4 * ns
        else:
            scales = buf[s:s + 2 * ns].view(torch.float16)
            scales.copy_(sc.half())
            sb = 2 * ns
        hc = hs = None
        if host:
            cpad = (rows + pad_rows) * k // (2 if f == FMT_Q4 else 1)
            spad = (rows + pad_rows) * (1 if f == FMT_Q8 else k // 32) * (sb // ns)
            hc = buf[w:w + cpad].cpu().numpy()
            hs = buf[s:s + spad].cpu().numpy()
            hc = hc.view(np.int8) if f != FMT_Q4 else hc
            hs = hs.view(np.float32) if f in (FMT_Q8, FMT_Q8B_F32) else hs.view(np.uint16)
        return nc + sb, hc, hs

    weight_bytes = 0
    stored = dict(layers=[]) if host else None
    for layer in range(cfg.layers):
        buf = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        mats = {}
        for name, w, s_, rows, k in regions:
            b, hc, hs = fill(buf, w, s_, rows, k, fmt)
            weight_bytes += b
            mats[name] = (hc, hs)
        qn = (1 + 0.02 * rng.standard_normal(hd)).astype(np.float32)
        kn = (1 + 0.02 * rng.standard_normal(hd)).astype(np.float32)
        lm.bind_layer(layer, buf, desc, qn, kn)
        if host:
            stored["layers"].append(dict(mats, q_norm=qn, k_norm=kn))
    emb = torch.randn((cfg.vocab, H), device=device, generator=gen).to(torch.bfloat16).view(torch.int16)
    lm.bind_embed(emb)
    rows, so, hb = lm_head_layout(cfg)
    head = torch.zeros(hb, dtype=torch.uint8, device=device)
    b, hc, hs = fill(head, 0, so, cfg.vocab, H, FMT_Q8B, pad_rows=rows - cfg.vocab)  # padding rows stay zero
    weight_bytes += b
    final_norm = (1 + 0.02 * rng.standard_normal(H)).astype(np.float32)
    lm.bind_head(head, final_norm)
    if host:
        stored.update(embed=emb.cpu().numpy().view(np.uint16), final_norm=final_norm, head=(hc, hs))
    torch.cuda.synchronize()
    return lm, weight_bytes, stored


# ---- weight preparation (gphq_prepare_projection) ----------------------------


class RotationSpec(ctypes.Structure):
    _fields_ = [("width", ctypes.c_int64), ("tile", ctypes.c_int64)]


class PrepareJob(ctypes.Structure):
    _fields_ = [("src_bf16_dev", ctypes.c_void_p), ("n", ctypes.c_int64), ("k", ctypes.c_int64),
                ("norm_host", ctypes.c_void_p), ("in_rot", RotationSpec), ("out_rot", RotationSpec),
                ("fmt", ctypes.c_int32), ("reserved", ctypes.c_int32), ("dst_dev", ctypes.c_void_p),
                ("dst_bytes", ctypes.c_int64), ("base", ctypes.c_int64), ("sc", ctypes.c_int64),
                ("step", ctypes.c_int64), ("row0", ctypes.c_int64), ("scale_mul", ctypes.c_float)]


def prepare_work_bytes(n, k):
    return load().gphq_prepare_work_bytes(n, k)


def prepare_projection(src_bf16, n, k, fmt, dst, base, sc, norm=None, in_rot=(0, 0), out_rot=(0, 0), step=1, row0=0,
                       scale_mul=1.0, work=None, stream=None):
    """One prepareGPU job: src_bf16 device int16 tensor [n][k] -> quantized rows in dst
    (a uint8 device tensor) at byte offsets base (codes) and sc (scales)."""
    import numpy as np
    import torch

    if work is None:
        work = torch.empty(prepare_work_bytes(n, k), dtype=torch.uint8, device=dst.device)
    nh = None
    if norm is not None:
        nh = np.ascontiguousarray(norm, dtype=np.float32)
    job = PrepareJob(src_bf16.data_ptr(), n, k, None if nh is None else nh.ctypes.data, RotationSpec(*in_rot),
                     RotationSpec(*out_rot), fmt, 0, dst.data_ptr(), dst.numel() * dst.element_size(), base, sc,
                     step, row0, scale_mul)
    check(load().gphq_prepare_projection(ctypes.byref(job), work.data_ptr(), work.numel() * work.element_size(),
                                         stream_handle(stream)))


def _bf16_device(bits, shape, device):
    """BF16 bits (numpy uint16/int16 or a device int16 tensor) as a contiguous device int16 tensor."""
    import numpy as np
    import torch

    if isinstance(bits, torch.Tensor):
        return bits.reshape(shape).contiguous().to(device)
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16).reshape(shape).copy()).to(device)


def _bf16_host_f32(bits):
    import numpy as np
    import torch

    if isinstance(bits, torch.Tensor):
        bits = bits.cpu().numpy()
    return (np.asarray(bits).view(np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(-1)


LAYER_PROJECTIONS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                     "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


def prepare_layer_jobs(cfg, input_norm, post_norm, dst=None):
    """gphq_prepare_layer_jobs: the seven PrepareJob of one layer (src unset)."""
    import numpy as np

    an, ap = _host(input_norm, np.float32)
    mn, mp = _host(post_norm, np.float32)
    jobs = (PrepareJob * 7)()
    check(load().gphq_prepare_layer_jobs(ctypes.byref(cfg), ap, mp, None if dst is None else dst.data_ptr(),
                                         0 if dst is None else dst.numel() * dst.element_size(), jobs))
    return list(jobs), (an, mn)


def prepare_lm(geom_kwargs, fmt, tensors, device="cuda", prefix="model.", head_name="lm_head.weight", stream=None):
    """prepareGPU (gpu_darwin.go:392-567) for a dense Qwen3 checkpoint, on the
    device, through the library's job list (gphq_prepare_layer /
    gphq_prepare_head): every projection of every layer quantized into its
    layer buffer (the placement of gphq_lm_layer_layout), the head into its
    own buffer (Q8B, in chunks of max(inter, 4096) rows), and the model bound.

    tensors maps checkpoint names (model.layers.N.self_attn.q_proj.weight, ...,
    model.embed_tokens.weight, model.norm.weight, lm_head.weight) to BF16 bits:
    numpy uint16/int16 arrays or device int16 tensors. Returns an Lm.
    """
    import torch

    cfg = lm_config(fmt=fmt, **geom_kwargs)
    desc, nbytes = lm_layer_layout(cfg)
    h = cfg.hidden
    lm = Lm(cfg)
    work = torch.empty(load().gphq_prepare_lm_work_bytes(ctypes.byref(cfg)), dtype=torch.uint8, device=device)
    for i in range(cfg.layers):
        p = f"{prefix}layers.{i}."
        an = _bf16_host_f32(tensors[p + "input_layernorm.weight"])
        mn = _bf16_host_f32(tensors[p + "post_attention_layernorm.weight"])
        jobs, (an, mn) = prepare_layer_jobs(cfg, an, mn)
        srcs = [_bf16_device(tensors[p + name + ".weight"], (j.n, j.k), device)
                for name, j in zip(LAYER_PROJECTIONS, jobs)]
        arr = (ctypes.c_void_p * 7)(*[t.data_ptr() for t in srcs])
        buf = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        check(load().gphq_prepare_layer(ctypes.byref(cfg), arr, an.ctypes.data, mn.ctypes.data, buf.data_ptr(),
                                        nbytes, work.data_ptr(), work.numel(), stream_handle(stream)))
        del srcs
        lm.bind_layer(i, buf, desc, _bf16_host_f32(tensors[p + "self_attn.q_norm.weight"]),
                      _bf16_host_f32(tensors[p + "self_attn.k_norm.weight"]))
    lm.bind_embed(_bf16_device(tensors[prefix + "embed_tokens.weight"], (cfg.vocab, h), device))
    rows, head_sc, head_bytes = lm_head_layout(cfg)
    head_buf = torch.zeros(head_bytes, dtype=torch.uint8, device=device)
    head_src = _bf16_device(tensors[head_name], (cfg.vocab, h), device)
    check(load().gphq_prepare_head(ctypes.byref(cfg), head_src.data_ptr(), head_buf.data_ptr(), head_bytes,
                                   work.data_ptr(), work.numel(), stream_handle(stream)))
    del head_src
    lm.bind_head(head_buf, _bf16_host_f32(tensors[prefix + "norm.weight"]))
    torch.cuda.synchronize()
    return lm


# ---- GPTQ producer (gphq_gptq_*) ----------------------------------------------


def q8b_quantize(x, rows, k, q, d, x_stride=None, stream=None):
    """Block-32 int8 activations (gphq_q8b_quantize): x [rows][k] fp32 device tensor ->
    q [rows][k] int8 and d [rows][k/32] fp32."""
    return check(load().gphq_q8b_quantize(ptr(x), rows, k, k if x_stride is None else x_stride, ptr(q), ptr(d),
                                          stream_handle(stream)))


def q8b_gemm(qa, da, qw, dw, y, m, k, n, stream=None):
    """Block-32 int8 GEMM (gphq_q8b_gemm): y [m][n] from codes and block scales."""
    return check(load().gphq_q8b_gemm(ptr(qa), ptr(da), ptr(qw), ptr(dw), ptr(y), m, k, n, stream_handle(stream)))


def gptq_factor(x, rows, k, u, dead, stream=None):
    """quantizeGroup's H = X^T X, damping and gptqInverseFactor: x [rows][k]
    fp32, u [k][k] fp32 and dead [k] uint8 device tensors. Synchronizes."""
    import torch

    work = torch.empty(load().gphq_gptq_work_bytes(k), dtype=torch.uint8, device=x.device)
    return check(load().gphq_gptq_factor(ptr(x), rows, k, ptr(u), ptr(dead), ptr(work), work.numel(),
                                         stream_handle(stream)))


def gptq_round(w, n, k, u, dead, bits, codes, scales, stream=None):
    """gptqRound of w [n][k] (fp32 device tensor, rounded in place)."""
    import torch

    work = torch.empty(load().gphq_gptq_round_work_bytes(n, k), dtype=torch.uint8, device=w.device)
    return check(load().gphq_gptq_round(ptr(w), n, k, ptr(u), ptr(dead), bits, ptr(codes), ptr(scales), ptr(work),
                                        work.numel(), stream_handle(stream)))


# ---- GPTQ calibration pass (gphq_gptq_calibration_* / gphq_gptq_quantize) ----

CAL_RESIDUAL, CAL_ATTN_INPUT, CAL_CONTEXT, CAL_MLP_INPUT, CAL_DOWN_INPUT = range(5)
GPTQ_MAX_SEQ, GPTQ_MAX_ROWS = 256, 4096  # gptqMaxSeq, gptqMaxRows (gptq.go:39-40)
GPTQ_PROGRESS = ctypes.CFUNCTYPE(None, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p)


def gptq_calibration_sequences(text_lens):
    """calibrationSequences' cut (gptq.go:275-287): the sequence lengths of
    tokenized texts of the given lengths."""
    import numpy as np

    lens = np.ascontiguousarray(text_lens, dtype=np.int64)
    n = ctypes.c_int64()
    check(load().gphq_gptq_calibration_sequences(lens.ctypes.data if lens.size else None, lens.size, None, 0,
                                                 ctypes.byref(n)))
    out = np.zeros(max(n.value, 1), np.int64)
    check(load().gphq_gptq_calibration_sequences(lens.ctypes.data if lens.size else None, lens.size, out.ctypes.data,
                                                 n.value, ctypes.byref(n)))
    return out[: n.value]


class GptqCalibration:
    """gphq_gptq_calibration: the calibration pass of QuantizeGPTQ
    (newCalibration / calibration.layer, qwen3lm/gptq.go:344-524) over token-id
    sequences, on the device. embed: BF16 bits [vocab][hidden] (int16 or
    uint16 device tensor), kept alive by this object."""

    def __init__(self, cfg, sequences, embed, stream=None):
        import numpy as np

        self.cfg = cfg
        lens = np.array([len(s) for s in sequences], np.int64)
        ids = np.concatenate([np.asarray(s, np.int32) for s in sequences]) if len(sequences) else np.zeros(0, np.int32)
        ids = np.ascontiguousarray(ids, np.int32)
        self.h = ctypes.c_void_p()
        self._embed = embed
        check(load().gphq_gptq_calibration_new(ctypes.byref(cfg), ids.ctypes.data if ids.size else None,
                                               lens.ctypes.data if lens.size else None, lens.size, ptr(embed),
                                               embed.numel(), ctypes.byref(self.h), stream_handle(stream)))

    def close(self):
        if self.h:
            load().gphq_gptq_calibration_free(self.h)
            self.h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def layer(self, srcs, input_norm, post_norm, q_norm, k_norm, bits, codes, scales, stream=None):
        """calibration.layer: srcs = the seven BF16 projections (device
        tensors, LAYER_PROJECTIONS order); norms float32 host arrays; codes /
        scales = seven uint8 device tensors sized by gptqRowBytes."""
        import numpy as np

        arr = lambda ts: (ctypes.c_void_p * 7)(*[t.data_ptr() for t in ts])
        norms = [np.ascontiguousarray(v, np.float32) for v in (input_norm, post_norm, q_norm, k_norm)]
        check(load().gphq_gptq_calibration_layer(self.h, arr(srcs), *[v.ctypes.data for v in norms], bits,
                                                 arr(codes), arr(scales), stream_handle(stream)))

    def rows(self, which, stream=None):
        """A copy of one set of rows [rows][width] as a float32 device tensor."""
        import torch

        r, w = ctypes.c_int64(), ctypes.c_int64()
        check(load().gphq_gptq_calibration_rows(self.h, which, None, 0, ctypes.byref(r), ctypes.byref(w), None))
        out = torch.empty((r.value, w.value), dtype=torch.float32, device="cuda")
        check(load().gphq_gptq_calibration_rows(self.h, which, out.data_ptr(), out.numel(), None, None,
                                                stream_handle(stream)))
        return out


def gptq_quantize(path, fmt, cfg, texts, progress=None, stream=None):
    """QuantizeGPTQ (qwen3lm/gptq.go:197-266) for tokenized calibration texts:
    writes gophonic-gptq-<fmt>.bin next to the checkpoint in path."""
    import numpy as np

    lens = np.array([len(t) for t in texts], np.int64)
    ids = np.ascontiguousarray(np.concatenate([np.asarray(t, np.int32) for t in texts]) if len(texts)
                               else np.zeros(0, np.int32), np.int32)
    cb = GPTQ_PROGRESS(lambda layer, layers, user: progress(layer, layers)) if progress else None
    st = load().gphq_gptq_quantize(str(path).encode(), fmt.encode(), ctypes.byref(cfg),
                                   ids.ctypes.data if ids.size else None, lens.ctypes.data if lens.size else None,
                                   lens.size, ctypes.cast(cb, ctypes.c_void_p) if cb else None, None,
                                   stream_handle(stream))
    if st != OK:
        detail = load().gphq_error_detail().decode()
        raise GphqError(st, detail or error_string(st))
