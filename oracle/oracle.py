"""numpy front end of the CPU oracle (liboracle.so, built from gphq_oracle.c).

TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the checker or the CPU
baseline. The product library (gophonic_amd / libgphq.so) never calls it.

Each wrapper names the reference function it restates; the C file carries the
file:line citations.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i8p = ctypes.POINTER(ctypes.c_int8)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p


def build():
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)


def _load():
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    sig = {
        "orc_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
        "orc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
        "orc_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
        "orc_max_abs": (ctypes.c_float, [_f32p, _i64]),
        "orc_q8gemv_mul_into": (None, [_f32p, _i8p, _f32p, _f32p, _i64, _i64]),
        "orc_q8gemv_mul_into_fma": (None, [_f32p, _i8p, _f32p, _f32p, _i64, _i64]),
        "orc_quantize_row_q8": (ctypes.c_float, [_f32p, _i64, _i8p]),
        "orc_quantize_row_q8b": (None, [_f32p, _i64, _i8p, _u16p, ctypes.c_float]),
        "orc_quantize_row_q4": (None, [_f32p, _i64, _u8p, _u16p, ctypes.c_float]),
        "orc_q4_group_scale": (ctypes.c_float, [_f32p, _i64]),
        "orc_gemv": (None, [ctypes.c_int, _vp, _vp, _f32p, _f32p, _i64, _i64]),
        "orc_gemv_f64": (None, [ctypes.c_int, _vp, _vp, _f32p, _f64p, _f64p, _i64, _i64]),
        "orc_f16_row_scale": (None, [ctypes.c_float, _f32p, _f32p]),
        "orc_f16_pack_rows": (None, [_f32p, _i64, _i64, _i64, _u16p, _f32p, _f32p]),
        "orc_pack_bf16_row": (_i64, [_u16p, _i64, _u16p, _f32p]),
        "orc_mul_panels": (None, [_f32p, _i64, _u16p, _f32p, _i64, _i8p, _u16p, _f32p, _i64, _i64, _i64, _i64]),
        "orc_pack_panels_u16": (None, [_u16p, _i64, _i64, _u16p]),
        "orc_pack_panels_i8": (None, [_i8p, _i64, _i64, _i8p]),
        "orc_i8_row_scale": (None, [ctypes.c_float, _f32p, _f32p]),
        "orc_i8_quantize": (ctypes.c_int8, [ctypes.c_float]),
        "orc_i8_pack_rows": (None, [_f32p, _i64, _i64, _i64, _i8p, _f32p, _f32p]),
        "orc_q8b_quantize": (None, [_f32p, _i64, _i64, _i64, _i8p, _f32p]),
        "orc_q8b_gemm": (None, [_i8p, _f32p, _i8p, _f32p, _f32p, _i64, _i64, _i64]),
        "orc_i8_mul_panels": (None, [_f32p, _i64, _i8p, _f32p, _i64, _i8p, _f32p, _i64, _i64, _i64, _i64]),
        "orc_i8_mul_panels_mt": (None, [_f32p, _i64, _i8p, _f32p, _i64, _i8p, _f32p, _i64, _i64, ctypes.c_int]),
        "orc_pack_panels_i8_quads": (None, [_i8p, _i64, _i64, _i8p]),
        "orc_f32_to_f16_array": (None, [_f32p, _u16p, _i64]),
        "orc_f16_to_f32_array": (None, [_u16p, _f32p, _i64]),
        "orc_i8_quantize_array": (None, [_f32p, _i8p, _i64]),
        "orc_mm_f64": (None, [ctypes.c_int, _vp, _vp, _u8p, _f32p, _f64p, _f64p, _i64, _i64, _i64]),
        "orc_splitmix64_next": (ctypes.c_uint64, [ctypes.POINTER(ctypes.c_uint64)]),
        "orc_rotation": (_i64, [_i64, _f32p, _f32p]),
        "orc_fwht": (None, [_f32p, _i64]),
        "orc_rotation_apply": (None, [_f32p, _i64, ctypes.c_float, _f32p, _i64]),
        "orc_rotation_unapply": (None, [_f32p, _i64, ctypes.c_float, _f32p, _i64]),
        "orc_rotation_apply_rows": (None, [_f32p, _i64, ctypes.c_float, _f32p, _i64, _i64]),
        "orc_prepare_projection": (None, [_u16p, _i64, _i64, _f32p, _f32p, _i64, ctypes.c_float, _f32p, _i64,
                                          ctypes.c_float, ctypes.c_int, _u8p, _i64, _i64, _i64, _i64,
                                          ctypes.c_float, _f32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _p(a, t):
    return a.ctypes.data_as(t)


def _c(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a


# Format tags shared with libgphq (include/gphq.h GPHQ_FMT_*).
FMT_Q8, FMT_Q8B, FMT_Q8B_F32, FMT_Q4 = 8, 9, 10, 4


def f32_to_f16(f):
    """q8gemm.f32ToF16 (gemm.go:297-327) elementwise -> uint16 bits."""
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.zeros(f.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_array(_p(f, _f32p), _p(out, _u16p), f.size)
    return out


def f16_to_f32(h):
    """q8gemm.f16ToF32 (gemm.go:329-341) elementwise."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.zeros(h.shape, dtype=np.float32)
    lib().orc_f16_to_f32_array(_p(h, _u16p), _p(out, _f32p), h.size)
    return out


def i8_quantize_array(v):
    """q8gemm quantize (int8.go:163-168) elementwise."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.zeros(v.shape, dtype=np.int8)
    lib().orc_i8_quantize_array(_p(v, _f32p), _p(out, _i8p), v.size)
    return out


def max_abs(x):
    x = _c(x, np.float32)
    return lib().orc_max_abs(_p(x, _f32p), x.size)


def q8gemv_mul_into(x, q, scales, k, n, fma=False):
    """q8gemv.scalarMulInto (scalar.go:8-17): returns dst[n]."""
    x, q, s = _c(x, np.float32), _c(q, np.int8), _c(scales, np.float32)
    dst = np.zeros(n, dtype=np.float32)
    fn = lib().orc_q8gemv_mul_into_fma if fma else lib().orc_q8gemv_mul_into
    fn(_p(x, _f32p), _p(q, _i8p), _p(s, _f32p), _p(dst, _f32p), k, n)
    return dst


def quantize_row_q8(row):
    """qwen3lm quantizeRow (gpu_darwin.go:582-594) -> (codes, scale)."""
    row = _c(row, np.float32)
    q = np.zeros(row.size, dtype=np.int8)
    s = lib().orc_quantize_row_q8(_p(row, _f32p), row.size, _p(q, _i8p))
    return q, np.float32(s)


def quantize_row_q8b(row, mul=1.0):
    """qwen3lm quantizeRowQ8B (gpu_darwin.go:599-614) -> (codes, f16 scales)."""
    row = _c(row, np.float32)
    q = np.zeros(row.size, dtype=np.int8)
    sc = np.zeros(row.size // 32, dtype=np.uint16)
    lib().orc_quantize_row_q8b(_p(row, _f32p), row.size, _p(q, _i8p), _p(sc, _u16p), mul)
    return q, sc


def quantize_row_q4(row, mul=1.0):
    """qwen3lm quantizeRowQ4 (gpu_darwin.go:616-658) -> (bytes, f16 scales)."""
    row = _c(row, np.float32)
    q = np.zeros(row.size // 2, dtype=np.uint8)
    sc = np.zeros(row.size // 32, dtype=np.uint16)
    lib().orc_quantize_row_q4(_p(row, _f32p), row.size, _p(q, _u8p), _p(sc, _u16p), mul)
    return q, sc


def q4_group_scale(v):
    """qwen3lm q4GroupScale (gptq.go:762-791)."""
    v = _c(v, np.float32)
    return np.float32(lib().orc_q4_group_scale(_p(v, _f32p), v.size))


def gemv(fmt, codes, scales, x, k, n):
    """qwen3lm gemv semantics (gpu.metal:68-162) as scalar loops -> y[n]."""
    codes = np.ascontiguousarray(codes)
    scales = np.ascontiguousarray(scales)
    x = _c(x, np.float32)
    y = np.zeros(n, dtype=np.float32)
    lib().orc_gemv(fmt, codes.ctypes.data, scales.ctypes.data, _p(x, _f32p), _p(y, _f32p), k, n)
    return y


def gemv_f64(fmt, codes, scales, x, k, n):
    """float64 dequantized product (gpu_darwin_test.go:44-56) -> (y, sum|w x|)."""
    codes = np.ascontiguousarray(codes)
    scales = np.ascontiguousarray(scales)
    x = _c(x, np.float32)
    y = np.zeros(n, dtype=np.float64)
    a = np.zeros(n, dtype=np.float64)
    lib().orc_gemv_f64(fmt, codes.ctypes.data, scales.ctypes.data, _p(x, _f32p), _p(y, _f64p), _p(a, _f64p), k, n)
    return y, a


def f16_row_scale(m):
    s, inv = ctypes.c_float(), ctypes.c_float()
    lib().orc_f16_row_scale(m, ctypes.byref(s), ctypes.byref(inv))
    return np.float32(s.value), np.float32(inv.value)


def f16_pack_rows(x, rows, k, stride=None):
    """q8gemm Workspace.Pack (gemm.go:65-77,127-135,155-226) -> (f16[rows,k], scale, inverse)."""
    stride = k if stride is None else stride
    x = _c(x, np.float32)
    out = np.zeros((rows, k), dtype=np.uint16)
    s = np.zeros(rows, dtype=np.float32)
    inv = np.zeros(rows, dtype=np.float32)
    lib().orc_f16_pack_rows(_p(x, _f32p), rows, k, stride, _p(out, _u16p), _p(s, _f32p), _p(inv, _f32p))
    return out, s, inv


def pack_bf16_rows(bf16, k, n):
    """q8gemm PackBF16 (packed.go:128-175) -> (f16[n,k], scales[n], rounded) or None."""
    bf16 = _c(bf16, np.uint16).reshape(n, k)
    out = np.zeros((n, k), dtype=np.uint16)
    sc = np.zeros(n, dtype=np.float32)
    rounded = 0
    for r in range(n):
        s = ctypes.c_float()
        got = lib().orc_pack_bf16_row(_p(bf16[r], _u16p), k, _p(out[r], _u16p), ctypes.byref(s))
        if got < 0:
            return None
        rounded += got
        sc[r] = s.value
    return out, sc, rounded


def mul_panels(act_f16, row_inverse, w, scales, k, n, p0=0, p1=None, stride=None, dst=None):
    """q8gemm scalarMulPanels (scalar.go:9-20). w: int8 [n,k] or uint16 FP16 bits [n,k]."""
    rows = act_f16.shape[0]
    p1 = (n + 63) // 64 if p1 is None else p1
    stride = n if stride is None else stride
    act = _c(act_f16, np.uint16)
    inv = _c(row_inverse, np.float32)
    s = _c(scales, np.float32)
    if dst is None:
        dst = np.zeros(max(0, (rows - 1) * stride + n), dtype=np.float32)
    w = np.ascontiguousarray(w)
    if w.dtype == np.uint16:
        wi8, wf16 = None, _p(w, _u16p)
    else:
        wi8, wf16 = _p(w.astype(np.int8, copy=False), _i8p), None
    lib().orc_mul_panels(_p(dst, _f32p), stride, _p(act, _u16p), _p(inv, _f32p), rows, wi8, wf16, _p(s, _f32p), k, n, p0, p1)
    return dst


def i8_row_scale(m):
    s, inv = ctypes.c_float(), ctypes.c_float()
    lib().orc_i8_row_scale(m, ctypes.byref(s), ctypes.byref(inv))
    return np.float32(s.value), np.float32(inv.value)


def i8_quantize(v):
    return lib().orc_i8_quantize(float(np.float32(v)))


def i8_pack_rows(x, rows, k, stride=None):
    """q8gemm WorkspaceI8 Prepare/SetRowScale/PackRange (int8.go:100-163) -> (q[rows,k], scale, inverse)."""
    stride = k if stride is None else stride
    x = _c(x, np.float32)
    out = np.zeros((rows, k), dtype=np.int8)
    s = np.zeros(rows, dtype=np.float32)
    inv = np.zeros(rows, dtype=np.float32)
    lib().orc_i8_pack_rows(_p(x, _f32p), rows, k, stride, _p(out, _i8p), _p(s, _f32p), _p(inv, _f32p))
    return out, s, inv


def q8b_quantize(x, rows, k, stride=None):
    """Block-32 variant of the int8 activation quantizer: each 32-value block
    takes WorkspaceI8's per-row rule (int8.go:106-168) -> (q [rows,k], d [rows,k/32])."""
    stride = k if stride is None else stride
    x = _c(x, np.float32)
    q = np.zeros((rows, k), dtype=np.int8)
    d = np.zeros((rows, k // 32), dtype=np.float32)
    lib().orc_q8b_quantize(_p(x, _f32p), rows, k, stride, _p(q, _i8p), _p(d, _f32p))
    return q, d


def q8b_gemm(qa, da, qw, dw, m, k, n):
    """Block-32 int8 GEMM: exact int32 per block, then acc = fmaf(dot, da*dw, acc) in block order."""
    y = np.zeros((m, n), dtype=np.float32)
    lib().orc_q8b_gemm(_p(_c(qa, np.int8), _i8p), _p(_c(da, np.float32), _f32p), _p(_c(qw, np.int8), _i8p),
                       _p(_c(dw, np.float32), _f32p), _p(y, _f32p), m, k, n)
    return y


def i8_mul_panels(act, row_scale, w, scales, k, n, p0=0, p1=None, stride=None, dst=None, threads=0):
    """q8gemm scalarMulPanelsI8 (int8.go:200-211)."""
    rows = act.shape[0]
    p1 = (n + 63) // 64 if p1 is None else p1
    stride = n if stride is None else stride
    act = _c(act, np.int8)
    rs = _c(row_scale, np.float32)
    w = _c(w, np.int8)
    s = _c(scales, np.float32)
    if dst is None:
        dst = np.zeros(max(0, (rows - 1) * stride + n), dtype=np.float32)
    if threads:
        lib().orc_i8_mul_panels_mt(_p(dst, _f32p), stride, _p(act, _i8p), _p(rs, _f32p), rows, _p(w, _i8p), _p(s, _f32p), k, n, threads)
    else:
        lib().orc_i8_mul_panels(_p(dst, _f32p), stride, _p(act, _i8p), _p(rs, _f32p), rows, _p(w, _i8p), _p(s, _f32p), k, n, p0, p1)
    return dst


def pack_panels(src, k, n):
    """q8gemm Weights panel layout [panel][K/2][64][2] (packed.go:183-204, 233-239)."""
    src = np.ascontiguousarray(src)
    panels, pairs = (n + 63) // 64, (k + 1) // 2
    if src.dtype == np.uint16:
        out = np.zeros(panels * pairs * 128, dtype=np.uint16)
        lib().orc_pack_panels_u16(_p(src, _u16p), k, n, _p(out, _u16p))
    else:
        src = src.astype(np.int8, copy=False)
        out = np.zeros(panels * pairs * 128, dtype=np.int8)
        lib().orc_pack_panels_i8(_p(src, _i8p), k, n, _p(out, _i8p))
    return out


def pack_panels_quads(src, k, n):
    """q8gemm WeightsI8 layout [panel][K/4][64][4] (int8.go:53-77)."""
    src = _c(src, np.int8)
    panels, quads = (n + 63) // 64, (k + 3) // 4
    out = np.zeros(panels * quads * 256, dtype=np.int8)
    lib().orc_pack_panels_i8_quads(_p(src, _i8p), k, n, _p(out, _i8p))
    return out


FMT_GPTQ4_G128 = 12


def mm_f64(fmt, codes, scales, x, m, k, n, zeros=None):
    """qwen3lm mm semantics (gpu.metal:766-927) in float64 -> (y[m,n], sum|a w|[m,n])."""
    codes = np.ascontiguousarray(codes)
    scales = np.ascontiguousarray(scales)
    x = _c(x, np.float32)
    z = None if zeros is None else _c(zeros, np.uint8)
    y = np.zeros((m, n), dtype=np.float64)
    a = np.zeros((m, n), dtype=np.float64)
    lib().orc_mm_f64(fmt, codes.ctypes.data, scales.ctypes.data, None if z is None else _p(z, _u8p), _p(x, _f32p),
                     _p(y, _f64p), _p(a, _f64p), m, k, n)
    return y, a


def splitmix64_outputs(seed, count):
    """The first `count` outputs of splitmix64 from state `seed`."""
    st = ctypes.c_uint64(seed)
    return [lib().orc_splitmix64_next(ctypes.byref(st)) for _ in range(count)]


def rotation_apply_f32(x, rot):
    """hadamard.go:51-58 rotation.apply in float32 (rot = (signs, block, scale))."""
    signs, block, scale = rot
    v = _c(x, np.float32).copy()
    lib().orc_rotation_apply(_p(_c(signs, np.float32), _f32p), block, scale, _p(v, _f32p), len(v))
    return v


def rotation_unapply_f32(x, rot):
    """hadamard.go:80-86 rotation.unapply in float32."""
    signs, block, scale = rot
    v = _c(x, np.float32).copy()
    lib().orc_rotation_unapply(_p(_c(signs, np.float32), _f32p), block, scale, _p(v, _f32p), len(v))
    return v


def rotation_apply_rows_f32(a, rot):
    """hadamard.go:88-104 rotation.applyRows in float32 on an n x k array (rot = (signs, block, scale))."""
    signs, block, scale = rot
    m = np.array(a, dtype=np.float32, copy=True, order="C")
    n, k = m.shape
    lib().orc_rotation_apply_rows(_p(_c(signs[:n], np.float32), _f32p), block, scale, _p(m, _f32p), n, k)
    return m


def prepare_projection(bf16, n, k, fmt, dst, base, sc, norm=None, in_rot=None, out_rot=None, step=1, row0=0,
                       scale_mul=1.0):
    """One prepareGPU job (gpu_darwin.go:511-567) on the CPU, writing into the uint8 array dst.
    in_rot / out_rot: (signs, block, scale) or None."""
    src = _c(bf16, np.uint16)
    work = np.empty(n * k, np.float32)
    nrm = None if norm is None else _c(norm, np.float32)
    ins = None if in_rot is None else _c(in_rot[0][:k], np.float32)
    outs = None if out_rot is None else _c(out_rot[0][:n], np.float32)
    lib().orc_prepare_projection(
        _p(src, _u16p), n, k, None if nrm is None else _p(nrm, _f32p),
        None if ins is None else _p(ins, _f32p), 0 if in_rot is None else in_rot[1],
        0.0 if in_rot is None else in_rot[2], None if outs is None else _p(outs, _f32p),
        0 if out_rot is None else out_rot[1], 0.0 if out_rot is None else out_rot[2], fmt, _p(dst, _u8p), base, sc,
        step, row0, scale_mul, _p(work, _f32p))
