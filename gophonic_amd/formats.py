"""ctypes binding of libgphq's file formats: safetensors checkpoints
(internal/safetensors), the GPTQ weight file "GPHQ0001" (qwen3lm/gptq.go) and
the prepared-weight cache "GPHWCACH" (internal/wcache), plus a loader that
combines them with the device preparation the way the reference's loadGPU
does (qwen3lm/gpu_darwin.go:161-338).
"""
import ctypes

from . import gphq
from .gphq import load

_FILE_ERRORS = {gphq.ERR_IO, gphq.ERR_FORMAT, gphq.ERR_TENSOR_MISSING, gphq.ERR_TENSOR_SHAPE, gphq.ERR_TENSOR_DTYPE,
                gphq.ERR_TENSOR_NON_FINITE, gphq.ERR_READ_RANGE, gphq.ERR_UNSUPPORTED, gphq.ERR_DIMENSIONS}


def check(status):
    """Raises GphqError with the reference's formatted message (the thread's
    error detail) for a file-format failure."""
    if status != gphq.OK:
        detail = load().gphq_error_detail().decode() if status in _FILE_ERRORS else ""
        raise gphq.GphqError(status, detail or gphq.error_string(status))
    return status


def _shape(shape):
    arr = (ctypes.c_int64 * max(len(shape), 1))(*shape)
    return arr, len(shape)


# ---- safetensors --------------------------------------------------------------

DTYPES = {gphq_code: name for gphq_code, name in ((1, "BF16"), (2, "F16"), (3, "F32"))}


class Checkpoint:
    """An open safetensors checkpoint directory (safetensors.Checkpoint)."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        check(load().gphq_checkpoint_open(str(path).encode(), ctypes.byref(h)))
        self.h, self.dir = h, str(path)

    def close(self):
        if self.h:
            load().gphq_checkpoint_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def has(self, name):
        return bool(load().gphq_checkpoint_has(self.h, name.encode()))

    def info(self, name):
        """(dtype name or None, shape tuple)."""
        dt, nd = ctypes.c_int32(), ctypes.c_int64()
        dims = (ctypes.c_int64 * 16)()
        check(load().gphq_checkpoint_info(self.h, name.encode(), ctypes.byref(dt), dims, 16, ctypes.byref(nd)))
        return DTYPES.get(dt.value), tuple(dims[i] for i in range(min(nd.value, 16)))

    def lookup(self, name, *shape):
        arr, nd = _shape(shape)
        dt = ctypes.c_int32()
        check(load().gphq_checkpoint_lookup(self.h, name.encode(), arr, nd, ctypes.byref(dt)))
        return DTYPES.get(dt.value)

    def read_bits(self, name, count, offset=0):
        import numpy as np

        out = np.zeros(count, np.uint16)
        check(load().gphq_checkpoint_read_bits(self.h, name.encode(), out.ctypes.data if count else None, count,
                                               offset))
        return out

    def bf16(self, name, *shape):
        import numpy as np

        arr, nd = _shape(shape)
        out = np.zeros(int(np.prod(shape)) if shape else 1, np.uint16)
        check(load().gphq_checkpoint_bf16(self.h, name.encode(), arr, nd, out.ctypes.data, out.size))
        return out.reshape(shape)

    def bf16_device(self, name, shape, device="cuda"):
        """BF16 bits into a new device int16 tensor of `shape`."""
        import torch

        arr, nd = _shape(shape)
        n = 1
        for d in shape:
            n *= d
        out = torch.empty(max(n, 1), dtype=torch.int16, device=device)
        check(load().gphq_checkpoint_bf16_device(self.h, name.encode(), arr, nd, out.data_ptr(), out.numel()))
        return out[:n].reshape(shape)

    def float32(self, name, *shape):
        import numpy as np

        arr, nd = _shape(shape)
        out = np.zeros(int(np.prod(shape)) if shape else 1, np.float32)
        check(load().gphq_checkpoint_float32(self.h, name.encode(), arr, nd, out.ctypes.data, out.size))
        return out.reshape(shape)

    def map_bf16(self, name, *shape):
        """(numpy uint16 view of the mapped bits, release function)."""
        import numpy as np

        arr, nd = _shape(shape)
        m, bits = ctypes.c_void_p(), ctypes.c_void_p()
        check(load().gphq_checkpoint_map_bf16(self.h, name.encode(), arr, nd, ctypes.byref(m), ctypes.byref(bits)))
        n = int(np.prod(shape)) if shape else 1
        view = np.ctypeslib.as_array(ctypes.cast(bits.value, ctypes.POINTER(ctypes.c_uint16)), shape=(n,)) \
            if n else np.zeros(0, np.uint16)
        return view.reshape(shape), (lambda: load().gphq_mapping_free(m))


# ---- GPTQ file ----------------------------------------------------------------

def gptq_row_bytes(bits, k):
    c, s = ctypes.c_int64(), ctypes.c_int64()
    check(load().gphq_gptq_row_bytes(bits, k, ctypes.byref(c), ctypes.byref(s)))
    return c.value, s.value


def gptq_fingerprint(path):
    v = ctypes.c_uint64()
    check(load().gphq_gptq_fingerprint(str(path).encode(), ctypes.byref(v)))
    return v.value


def gptq_path(path, fmt):
    buf = ctypes.create_string_buffer(4096)
    check(load().gphq_gptq_path(str(path).encode(), fmt.encode(), buf, 4096))
    return buf.value.decode()


class GptqFile:
    """An opened GPTQ weight file (gptqFile); open() returns None when there is
    none for this format and checkpoint."""

    def __init__(self, h, cfg):
        self.h, self.cfg = h, cfg

    @classmethod
    def open(cls, path, fmt, cfg):
        h = ctypes.c_void_p()
        check(load().gphq_gptq_open(str(path).encode(), fmt.encode(), ctypes.byref(cfg), ctypes.byref(h)))
        return cls(h, cfg) if h.value else None

    def close(self):
        if self.h:
            load().gphq_gptq_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def bits(self):
        return load().gphq_gptq_bits(self.h)

    def projection(self, name):
        """(codes offset, scales offset) or None."""
        c, s = ctypes.c_int64(), ctypes.c_int64()
        if not load().gphq_gptq_projection(self.h, name.encode(), ctypes.byref(c), ctypes.byref(s)):
            return None
        return c.value, s.value

    def place(self, name, n, k, buf, base, sc, row0=0, step=1):
        """Copies a projection into the device layer buffer `buf` (uint8 tensor); False if not held."""
        placed = ctypes.c_int()
        check(load().gphq_gptq_place(self.h, name.encode(), n, k, buf.data_ptr(), buf.numel(), base, sc, row0, step,
                                     ctypes.byref(placed)))
        return bool(placed.value)


class GptqWriter:
    """QuantizeGPTQ's output file, written through a temporary and renamed on commit."""

    def __init__(self, path, fmt):
        h = ctypes.c_void_p()
        check(load().gphq_gptq_create(str(path).encode(), fmt.encode(), ctypes.byref(h)))
        self.h = h

    def write(self, data):
        import numpy as np

        b = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        check(load().gphq_gptq_write(self.h, b.ctypes.data if b.size else None, b.size))

    def write_device(self, t):
        check(load().gphq_gptq_write_device(self.h, t.data_ptr(), t.numel() * t.element_size()))

    def commit(self):
        h, self.h = self.h, None
        check(load().gphq_gptq_commit(h))

    def abort(self):
        if self.h:
            load().gphq_gptq_abort(self.h)
            self.h = None

    def __del__(self):
        try:
            self.abort()
        except Exception:
            pass


# ---- weight cache ---------------------------------------------------------------

WCACHE_ALIGN = 16 << 10


def wcache_round_up(n):
    return load().gphq_wcache_round_up(n)


def wcache_key(path, kind, *parts):
    enc = [p.encode() for p in parts]
    arr = (ctypes.c_char_p * max(len(enc), 1))(*enc)
    buf = ctypes.create_string_buffer(4096)
    check(load().gphq_wcache_key(str(path).encode(), kind.encode(), arr, len(enc), buf, 4096))
    return buf.value.decode()


def sha256(data):
    import numpy as np

    b = np.frombuffer(bytes(data), np.uint8)
    out = (ctypes.c_uint8 * 32)()
    check(load().gphq_wcache_sha256(b.ctypes.data if b.size else None, b.size, out))
    return bytes(out)


class WcacheFile:
    """One mapped cache entry (wcache.File). cache_dir None: the default
    directory; "": anonymous memory."""

    def __init__(self, cache_dir, key, size):
        h = ctypes.c_void_p()
        d = None if cache_dir is None else str(cache_dir).encode()
        check(load().gphq_wcache_open(d, key.encode(), size, ctypes.byref(h)))
        self.h = h

    @property
    def fresh(self):
        return bool(load().gphq_wcache_fresh(self.h))

    def payload(self):
        """The payload as a numpy uint8 array over the mapping (writable while fresh)."""
        import numpy as np

        n = ctypes.c_int64()
        p = load().gphq_wcache_payload(self.h, ctypes.byref(n))
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_uint8)), shape=(n.value,))

    def done(self, offset, length):
        n = ctypes.c_int64()
        p = load().gphq_wcache_payload(self.h, ctypes.byref(n))
        load().gphq_wcache_done(self.h, p + offset, length)

    def commit(self):
        load().gphq_wcache_commit(self.h)

    def close(self):
        if self.h:
            h, self.h = self.h, None
            check(load().gphq_wcache_close(h))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Layout:
    """wcache.Layout: cuts a payload into aligned regions; take(n) returns
    the region's (offset, length)."""

    def __init__(self):
        self.off = 0

    def take(self, n):
        start = self.off
        self.off += wcache_round_up(n)
        return start, self.off - start

    @property
    def size(self):
        return self.off


# ---- loader: safetensors -> (GPTQ file | device preparation) -> cache -> model ----

# The weight formats' names (qwen3lm/weights.go:32-45; Q8B_F32 is this
# library's own) and their GPTQ files (gpu_darwin.go:440).
FORMAT_NAMES = {gphq.FMT_Q8: "gpu", gphq.FMT_Q8B: "gpu-q8", gphq.FMT_Q4: "gpu-q4", gphq.FMT_Q8B_F32: "gpu-q8-f32"}
GPTQ_FORMATS = {gphq.FMT_Q8: "gpu", gphq.FMT_Q4: "gpu-q4"}
CACHE_VERSION = "gphq-1"  # bumped when the prepared bytes change


def load_lm(path, geom_kwargs, fmt, cache_dir=None, device="cuda", prefix="model.", head_name="lm_head.weight"):
    """loadGPU + loadHead (qwen3lm/gpu_darwin.go:161-373) for a dense Qwen3
    safetensors checkpoint in `path`: the layer buffers are regions of one
    cache entry and the head has an entry of its own (wcache). A fresh entry
    is filled on the device -- each projection from the GPTQ file when one
    matches this checkpoint (gptq.go:113-190), else prepareGPU's job from the
    BF16 tensor -- copied into the entry and committed; a committed entry is
    uploaded as it is. Returns (Lm, stats) with stats = {"layers_fresh",
    "head_fresh", "gptq_placed"}."""
    import numpy as np
    import torch

    cfg = gphq.lm_config(fmt=fmt, **geom_kwargs)
    desc, nbytes = gphq.lm_layer_layout(cfg)
    kind = FORMAT_NAMES[fmt]
    ck = Checkpoint(path)
    lm = gphq.Lm(cfg)
    stats = {"layers_fresh": False, "head_fresh": False, "gptq_placed": 0}
    h = cfg.hidden

    def f32(name, *shape):
        return ck.float32(name, *shape).reshape(-1)

    # Layers: one entry, a region per layer.
    lay = Layout()
    regions = [lay.take(nbytes) for _ in range(cfg.layers)]
    entry = WcacheFile(cache_dir, wcache_key(path, kind, CACHE_VERSION, prefix, ""), lay.size)
    bufs = []
    if entry.fresh:
        stats["layers_fresh"] = True
        pre = GptqFile.open(path, GPTQ_FORMATS[fmt], cfg) if fmt in GPTQ_FORMATS else None
        work = torch.empty(load().gphq_prepare_lm_work_bytes(ctypes.byref(cfg)), dtype=torch.uint8, device=device)
        payload = entry.payload()
        for i, (off, _) in enumerate(regions):
            p = f"{prefix}layers.{i}."
            jobs, keep = gphq.prepare_layer_jobs(cfg, f32(p + "input_layernorm.weight", h),
                                                 f32(p + "post_attention_layernorm.weight", h))
            buf = torch.zeros(nbytes, dtype=torch.uint8, device=device)
            for name, j in zip(gphq.LAYER_PROJECTIONS, jobs):
                tensor = f"layers.{i}.{name}.weight"
                if pre is not None and pre.place(tensor, j.n, j.k, buf, j.base, j.sc, j.row0, j.step):
                    stats["gptq_placed"] += 1
                    continue
                src = ck.bf16_device(prefix + tensor, (j.n, j.k), device)
                j.src_bf16_dev, j.dst_dev, j.dst_bytes = src.data_ptr(), buf.data_ptr(), nbytes
                gphq.check(load().gphq_prepare_projection(ctypes.byref(j), work.data_ptr(), work.numel(), None))
            payload[off:off + nbytes] = buf.cpu().numpy()
            entry.done(off, nbytes)
            bufs.append(buf)
        if pre is not None:
            pre.close()
        entry.commit()
    else:
        payload = entry.payload()
        for off, _ in regions:
            bufs.append(torch.from_numpy(np.array(payload[off:off + nbytes])).to(device))
    for i, buf in enumerate(bufs):
        p = f"{prefix}layers.{i}."
        lm.bind_layer(i, buf, desc, f32(p + "self_attn.q_norm.weight", cfg.head_dim),
                      f32(p + "self_attn.k_norm.weight", cfg.head_dim))
    entry.close()
    lm.bind_embed(ck.bf16_device(prefix + "embed_tokens.weight", (cfg.vocab, h), device))
    # Head: an entry of its own ("<kind>-lm").
    rows, head_sc, head_bytes = gphq.lm_head_layout(cfg)
    hl = Layout()
    hl.take(head_bytes)
    hentry = WcacheFile(cache_dir, wcache_key(path, kind + "-lm", CACHE_VERSION, prefix, head_name), hl.size)
    if hentry.fresh:
        stats["head_fresh"] = True
        work = torch.empty(load().gphq_prepare_lm_work_bytes(ctypes.byref(cfg)), dtype=torch.uint8, device=device)
        head = torch.zeros(head_bytes, dtype=torch.uint8, device=device)
        src = ck.bf16_device(head_name, (cfg.vocab, h), device)
        gphq.check(load().gphq_prepare_head(ctypes.byref(cfg), src.data_ptr(), head.data_ptr(), head_bytes,
                                            work.data_ptr(), work.numel(), None))
        del src
        hentry.payload()[:head_bytes] = head.cpu().numpy()
        hentry.commit()
    else:
        head = torch.from_numpy(np.array(hentry.payload()[:head_bytes])).to(device)
    hentry.close()
    lm.bind_head(head, f32(prefix + "norm.weight", h))
    ck.close()
    torch.cuda.synchronize()
    return lm, stats
