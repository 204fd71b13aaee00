// Hugging Face safetensors checkpoints, single file or sharded
// (internal/safetensors/safetensors.go): the loader's source of BF16
// projections for gphq_prepare_layer. Tensors are read on demand into caller
// storage (host, or device through a host copy), or mapped read-only.
//
// A file is an 8-byte little-endian header length, a JSON header (padded
// with spaces) mapping each tensor name to {dtype, shape, data_offsets}, then
// the data; data_offsets are relative to the end of the header. A sharded
// checkpoint lists its files in model.safetensors.index.json's weight_map.
#include <errno.h>
#include <fcntl.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "common.h"
#include "host_io.h"

using namespace gphq;

namespace {

// ---- a small JSON reader: the header and the index are plain JSON ---------

struct JVal {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool integral = false;
    int64_t i = 0;
    double d = 0;
    std::string s;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;
    const JVal *get(const std::string &key) const {
        for (const auto &kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

struct JParser {
    const char *p, *end;
    int depth = 0;
    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    bool lit(const char *w) {
        const size_t n = strlen(w);
        if ((size_t)(end - p) < n || memcmp(p, w, n) != 0) return false;
        p += n;
        return true;
    }
    static void utf8(std::string &out, uint32_t c) {
        if (c < 0x80) {
            out += (char)c;
        } else if (c < 0x800) {
            out += (char)(0xC0 | (c >> 6));
            out += (char)(0x80 | (c & 0x3F));
        } else if (c < 0x10000) {
            out += (char)(0xE0 | (c >> 12));
            out += (char)(0x80 | ((c >> 6) & 0x3F));
            out += (char)(0x80 | (c & 0x3F));
        } else {
            out += (char)(0xF0 | (c >> 18));
            out += (char)(0x80 | ((c >> 12) & 0x3F));
            out += (char)(0x80 | ((c >> 6) & 0x3F));
            out += (char)(0x80 | (c & 0x3F));
        }
    }
    bool hex4(uint32_t &v) {
        if (end - p < 4) return false;
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool str(std::string &out) {
        if (p >= end || *p != '"') return false;
        ++p;
        out.clear();
        while (p < end && *p != '"') {
            const unsigned char c = (unsigned char)*p++;
            if (c < 0x20) return false;
            if (c != '\\') {
                out += (char)c;
                continue;
            }
            if (p >= end) return false;
            const char e = *p++;
            switch (e) {
            case '"': out += '"'; break;
            case '\\': out += '\\'; break;
            case '/': out += '/'; break;
            case 'b': out += '\b'; break;
            case 'f': out += '\f'; break;
            case 'n': out += '\n'; break;
            case 'r': out += '\r'; break;
            case 't': out += '\t'; break;
            case 'u': {
                uint32_t u;
                if (!hex4(u)) return false;
                if (u >= 0xD800 && u < 0xDC00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
                    p += 2;
                    uint32_t lo;
                    if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return false;
                    u = 0x10000 + ((u - 0xD800) << 10) + (lo - 0xDC00);
                }
                utf8(out, u);
                break;
            }
            default: return false;
            }
        }
        if (p >= end) return false;
        ++p;
        return true;
    }
    bool num(JVal &v) {
        const char *s = p;
        if (p < end && *p == '-') ++p;
        bool frac = false;
        while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '+' || *p == '-')) {
            frac |= *p == '.' || *p == 'e' || *p == 'E';
            ++p;
        }
        if (p == s) return false;
        const std::string t(s, p);
        v.kind = JVal::NUM;
        char *ep = nullptr;
        if (!frac) {
            errno = 0;
            v.i = strtoll(t.c_str(), &ep, 10);
            if (*ep || errno) return false;
            v.integral = true;
            v.d = (double)v.i;
        } else {
            v.d = strtod(t.c_str(), &ep);
            if (*ep) return false;
        }
        return true;
    }
    bool value(JVal &v) {
        if (++depth > 64) return false;
        ws();
        bool ok = false;
        if (p >= end) {
            ok = false;
        } else if (*p == '{') {
            ++p;
            v.kind = JVal::OBJ;
            ws();
            if (p < end && *p == '}') {
                ++p;
                ok = true;
            } else {
                while (true) {
                    ws();
                    std::string key;
                    if (!str(key)) break;
                    ws();
                    if (p >= end || *p != ':') break;
                    ++p;
                    JVal child;
                    if (!value(child)) break;
                    v.obj.emplace_back(std::move(key), std::move(child));
                    ws();
                    if (p < end && *p == ',') {
                        ++p;
                        continue;
                    }
                    if (p < end && *p == '}') {
                        ++p;
                        ok = true;
                    }
                    break;
                }
            }
        } else if (*p == '[') {
            ++p;
            v.kind = JVal::ARR;
            ws();
            if (p < end && *p == ']') {
                ++p;
                ok = true;
            } else {
                while (true) {
                    JVal child;
                    if (!value(child)) break;
                    v.arr.push_back(std::move(child));
                    ws();
                    if (p < end && *p == ',') {
                        ++p;
                        continue;
                    }
                    if (p < end && *p == ']') {
                        ++p;
                        ok = true;
                    }
                    break;
                }
            }
        } else if (*p == '"') {
            v.kind = JVal::STR;
            ok = str(v.s);
        } else if (lit("true")) {
            v.kind = JVal::BOOL;
            ok = true;
        } else if (lit("false")) {
            v.kind = JVal::BOOL;
            ok = true;
        } else if (lit("null")) {
            v.kind = JVal::NUL;
            ok = true;
        } else {
            ok = num(v);
        }
        --depth;
        return ok;
    }
};

bool parse_json(const char *data, size_t len, JVal &out) {
    JParser ps{data, data + len};
    if (!ps.value(out)) return false;
    ps.ws();
    return ps.p == ps.end;
}

int dtype_code(const std::string &s) {
    if (s == "BF16") return GPHQ_DTYPE_BF16;
    if (s == "F16") return GPHQ_DTYPE_F16;
    if (s == "F32") return GPHQ_DTYPE_F32;
    return 0;
}

std::string shape_str(const int64_t *shape, int64_t ndim) {
    std::string s = "[";
    for (int64_t i = 0; i < ndim; ++i) s += (i ? " " : "") + std::to_string(shape[i]);
    return s + "]";
}

// safetensors.go:273-280 F16ToF32, exactly.
float f16_to_f32(uint16_t h) {
    const float sign = (h & 0x8000) ? -1.0f : 1.0f;
    const int exp = (h >> 10) & 0x1f;
    const double mant = (double)(h & 0x3ff);
    if (exp == 0) return sign * (float)ldexp(mant, -24);
    if (exp == 31) return mant != 0 ? NAN : sign * INFINITY;
    return sign * (float)ldexp(1.0 + mant / 1024.0, exp - 15);
}

}  // namespace

struct gphq_checkpoint {
    struct Tensor {
        int file = -1;
        std::string dtype;
        std::vector<int64_t> shape;
        int64_t offset = 0, size = 0;
    };
    std::string dir;
    std::vector<int> files;
    std::unordered_map<std::string, Tensor> tensors;
};

struct gphq_mapping {
    void *base = nullptr;
    size_t len = 0;
    std::vector<uint16_t> copy;  // when the tensor could not be mapped
};

namespace {

// safetensors.go:85-127 readHeader.
int read_header(gphq_checkpoint *c, int fd, const std::string &name) {
    struct stat st;
    if (fstat(fd, &st) != 0) return fail(GPHQ_ERR_IO, strf("safetensors: %s: stat failed", name.c_str()));
    uint8_t lenBuf[8];
    if (!pread_full(fd, lenBuf, 8, 0))
        return fail(GPHQ_ERR_IO, strf("safetensors: %s: read header length", name.c_str()));
    uint64_t n = 0;
    for (int i = 7; i >= 0; --i) n = (n << 8) | lenBuf[i];
    if (n == 0 || n > (100u << 20) || (int64_t)n + 8 > (int64_t)st.st_size)
        return fail(GPHQ_ERR_FORMAT, strf("safetensors: %s: invalid safetensors header length", name.c_str()));
    std::string header((size_t)n, '\0');
    if (!pread_full(fd, &header[0], (size_t)n, 8))
        return fail(GPHQ_ERR_IO, strf("safetensors: %s: read header", name.c_str()));
    while (!header.empty() && header.back() == ' ') header.pop_back();  // safetensors pads with spaces
    JVal root;
    if (!parse_json(header.data(), header.size(), root) || root.kind != JVal::OBJ)
        return fail(GPHQ_ERR_FORMAT, strf("safetensors: %s: parse header", name.c_str()));
    const int64_t base = 8 + (int64_t)n;
    for (const auto &kv : root.obj) {
        if (kv.first == "__metadata__") continue;
        const JVal &e = kv.second;
        gphq_checkpoint::Tensor t;
        t.file = fd;
        const JVal *dt = e.kind == JVal::OBJ ? e.get("dtype") : nullptr;
        const JVal *sh = e.kind == JVal::OBJ ? e.get("shape") : nullptr;
        const JVal *off = e.kind == JVal::OBJ ? e.get("data_offsets") : nullptr;
        if (dt && dt->kind == JVal::STR) t.dtype = dt->s;
        if (sh && sh->kind == JVal::ARR)
            for (const JVal &d : sh->arr) t.shape.push_back(d.kind == JVal::NUM && d.integral ? d.i : -1);
        const bool offsOk = off && off->kind == JVal::ARR && off->arr.size() == 2 && off->arr[0].integral &&
                            off->arr[1].integral;
        const int64_t o0 = offsOk ? off->arr[0].i : -1, o1 = offsOk ? off->arr[1].i : -1;
        if (!offsOk || o0 < 0 || o1 < o0 || base + o1 > (int64_t)st.st_size)
            return fail(GPHQ_ERR_FORMAT,
                        strf("safetensors: %s: tensor %s has invalid data offsets", name.c_str(), kv.first.c_str()));
        t.offset = base + o0;
        t.size = o1 - o0;
        c->tensors[kv.first] = t;
    }
    return GPHQ_OK;
}

// safetensors.go:140-162 Lookup.
int lookup(const gphq_checkpoint *c, const char *name, const int64_t *shape, int64_t ndim,
           const gphq_checkpoint::Tensor **out) {
    if (!c || !name || ndim < 0 || (ndim > 0 && !shape)) return fail(GPHQ_ERR_DIMENSIONS, "safetensors: bad arguments");
    auto it = c->tensors.find(name);
    if (it == c->tensors.end()) return fail(GPHQ_ERR_TENSOR_MISSING, strf("checkpoint is missing %s", name));
    const gphq_checkpoint::Tensor &t = it->second;
    int64_t count = 1;
    for (int64_t i = 0; i < ndim; ++i) count *= shape[i];
    bool same = (int64_t)t.shape.size() == ndim;
    for (int64_t i = 0; same && i < ndim; ++i) same = t.shape[(size_t)i] == shape[i];
    if (!same)
        return fail(GPHQ_ERR_TENSOR_SHAPE,
                    strf("%s has shape %s, want %s", name, shape_str(t.shape.data(), (int64_t)t.shape.size()).c_str(),
                         shape_str(shape, ndim).c_str()));
    const int code = dtype_code(t.dtype);
    const int64_t width = code == GPHQ_DTYPE_F32 ? 4 : code ? 2 : 0;
    if (width == 0 || t.size != count * width)
        return fail(GPHQ_ERR_TENSOR_DTYPE, strf("%s has dtype %s and %lld bytes for shape %s", name, t.dtype.c_str(),
                                                (long long)t.size, shape_str(shape, ndim).c_str()));
    *out = &t;
    return GPHQ_OK;
}

int need_bf16(const gphq_checkpoint::Tensor &t, const char *name) {
    if (t.dtype != "BF16")
        return fail(GPHQ_ERR_TENSOR_DTYPE,
                    strf("%s is %s; the loader expects the official BF16 checkpoint", name, t.dtype.c_str()));
    return GPHQ_OK;
}

// safetensors.go:203-213 ReadBits.
int read_bits(const gphq_checkpoint::Tensor &t, uint16_t *dst, int64_t count, int64_t offset) {
    if (offset < 0 || count < 0 || 2 * (offset + count) > t.size) return fail(GPHQ_ERR_READ_RANGE, "read outside the tensor");
    if (count && !pread_full(t.file, dst, (size_t)count * 2, t.offset + 2 * offset))
        return fail(GPHQ_ERR_IO, "read tensor: short read");
    return GPHQ_OK;
}

}  // namespace

extern "C" {

int gphq_checkpoint_open(const char *dir, gphq_checkpoint **out) {
    // safetensors.go:39-82 Open.
    clear_detail();
    if (!out || !dir) return fail(GPHQ_ERR_DIMENSIONS, "safetensors: bad arguments");
    *out = nullptr;
    const uint16_t probe = 1;
    if (*(const uint8_t *)&probe != 1) return fail(GPHQ_ERR_FORMAT, "safetensors: loading requires a little-endian CPU");
    std::vector<std::string> names{"model.safetensors"};
    const std::string index = join_path(dir, "model.safetensors.index.json");
    const int ifd = open(index.c_str(), O_RDONLY | O_CLOEXEC);
    if (ifd >= 0) {
        struct stat st;
        std::string raw;
        bool ok = fstat(ifd, &st) == 0;
        if (ok) {
            raw.resize((size_t)st.st_size);
            ok = st.st_size == 0 || pread_full(ifd, &raw[0], raw.size(), 0);
        }
        close(ifd);
        JVal root;
        if (!ok || !parse_json(raw.data(), raw.size(), root) || root.kind != JVal::OBJ)
            return fail(GPHQ_ERR_FORMAT, "safetensors: parse index");
        names.clear();
        const JVal *wm = root.get("weight_map");
        if (wm && wm->kind == JVal::OBJ)
            for (const auto &kv : wm->obj) {
                if (kv.second.kind != JVal::STR) return fail(GPHQ_ERR_FORMAT, "safetensors: parse index");
                bool seen = false;
                for (const std::string &n : names) seen |= n == kv.second.s;
                if (!seen) names.push_back(kv.second.s);
            }
    }
    gphq_checkpoint *c = new gphq_checkpoint();
    c->dir = dir;
    for (const std::string &name : names) {
        if (name.find('/') != std::string::npos || name.empty() || name == "." || name == "..") {
            gphq_checkpoint_close(c);
            return fail(GPHQ_ERR_FORMAT, strf("safetensors: shard \"%s\" is not a plain file name", name.c_str()));
        }
        const int fd = open(join_path(dir, name).c_str(), O_RDONLY | O_CLOEXEC);
        if (fd < 0) {
            gphq_checkpoint_close(c);
            return fail(GPHQ_ERR_IO, strf("safetensors: open weights: %s: %s", name.c_str(), strerror(errno)));
        }
        c->files.push_back(fd);
        const int st = read_header(c, fd, name);
        if (st != GPHQ_OK) {
            gphq_checkpoint_close(c);
            return st;
        }
    }
    *out = c;
    return GPHQ_OK;
}

void gphq_checkpoint_close(gphq_checkpoint *c) {
    if (!c) return;
    for (int fd : c->files) close(fd);
    delete c;
}

int gphq_checkpoint_has(const gphq_checkpoint *c, const char *name) {
    return c && name && c->tensors.count(name) ? 1 : 0;
}

int gphq_checkpoint_info(const gphq_checkpoint *c, const char *name, int32_t *dtype, int64_t *shape, int64_t max_ndim,
                         int64_t *ndim) {
    // A tensor's Tensor.DType and Tensor.Shape (safetensors.go:25-31); dtype
    // is 0 for a type other than BF16, F16, F32.
    clear_detail();
    if (!c || !name || !ndim) return fail(GPHQ_ERR_DIMENSIONS, "safetensors: bad arguments");
    auto it = c->tensors.find(name);
    if (it == c->tensors.end()) return fail(GPHQ_ERR_TENSOR_MISSING, strf("checkpoint is missing %s", name));
    const gphq_checkpoint::Tensor &t = it->second;
    if (dtype) *dtype = dtype_code(t.dtype);
    *ndim = (int64_t)t.shape.size();
    for (int64_t i = 0; shape && i < std::min<int64_t>(max_ndim, *ndim); ++i) shape[i] = t.shape[(size_t)i];
    return GPHQ_OK;
}

int gphq_checkpoint_lookup(const gphq_checkpoint *c, const char *name, const int64_t *shape, int64_t ndim,
                           int32_t *dtype) {
    clear_detail();
    const gphq_checkpoint::Tensor *t = nullptr;
    GPHQ_TRY(lookup(c, name, shape, ndim, &t));
    if (dtype) *dtype = dtype_code(t->dtype);
    return GPHQ_OK;
}

int gphq_checkpoint_read_bits(const gphq_checkpoint *c, const char *name, uint16_t *dst, int64_t count,
                              int64_t offset) {
    clear_detail();
    if (!c || !name || (count && !dst)) return fail(GPHQ_ERR_DIMENSIONS, "safetensors: bad arguments");
    auto it = c->tensors.find(name);
    if (it == c->tensors.end()) return fail(GPHQ_ERR_TENSOR_MISSING, strf("checkpoint is missing %s", name));
    return read_bits(it->second, dst, count, offset);
}

int gphq_checkpoint_bf16(const gphq_checkpoint *c, const char *name, const int64_t *shape, int64_t ndim, uint16_t *dst,
                         int64_t dst_len) {
    // safetensors.go:165-176 BF16, into caller storage.
    clear_detail();
    const gphq_checkpoint::Tensor *t = nullptr;
    GPHQ_TRY(lookup(c, name, shape, ndim, &t));
    GPHQ_TRY(need_bf16(*t, name));
    if (dst_len < t->size / 2 || (t->size && !dst)) return fail(GPHQ_ERR_DIMENSIONS, "safetensors: destination too short");
    return read_bits(*t, dst, t->size / 2, 0);
}

int gphq_checkpoint_bf16_device(const gphq_checkpoint *c, const char *name, const int64_t *shape, int64_t ndim,
                                uint16_t *dst_dev, int64_t dst_len) {
    // BF16 into device storage (through a host copy), for the loader.
    clear_detail();
    const gphq_checkpoint::Tensor *t = nullptr;
    GPHQ_TRY(lookup(c, name, shape, ndim, &t));
    GPHQ_TRY(need_bf16(*t, name));
    if (dst_len < t->size / 2 || (t->size && !dst_dev)) return fail(GPHQ_ERR_DIMENSIONS, "safetensors: destination too short");
    std::vector<uint16_t> host((size_t)(t->size / 2));
    GPHQ_TRY(read_bits(*t, host.data(), t->size / 2, 0));
    if (host.empty()) return GPHQ_OK;
    return hip_status(hipMemcpy(dst_dev, host.data(), host.size() * 2, hipMemcpyHostToDevice));
}

int gphq_checkpoint_float32(const gphq_checkpoint *c, const char *name, const int64_t *shape, int64_t ndim, float *dst,
                            int64_t dst_len) {
    // safetensors.go:217-251 Float32: BF16, F16 or F32 widened; non-finite rejected.
    clear_detail();
    const gphq_checkpoint::Tensor *t = nullptr;
    GPHQ_TRY(lookup(c, name, shape, ndim, &t));
    int64_t n = 1;
    for (int64_t i = 0; i < ndim; ++i) n *= shape[i];
    if (dst_len < n || (n && !dst)) return fail(GPHQ_ERR_DIMENSIONS, "safetensors: destination too short");
    if (t->dtype == "F32") {
        if (n && !pread_full(t->file, dst, (size_t)n * 4, t->offset))
            return fail(GPHQ_ERR_IO, strf("read %s: short read", name));
    } else {
        std::vector<uint16_t> raw((size_t)n);
        GPHQ_TRY(read_bits(*t, raw.data(), n, 0));
        const bool bf = t->dtype == "BF16";
        for (int64_t i = 0; i < n; ++i) {
            if (bf) {
                const uint32_t u = (uint32_t)raw[(size_t)i] << 16;
                memcpy(&dst[i], &u, 4);
            } else {
                dst[i] = f16_to_f32(raw[(size_t)i]);
            }
        }
    }
    for (int64_t i = 0; i < n; ++i)
        if (!isfinite(dst[i])) return fail(GPHQ_ERR_TENSOR_NON_FINITE, strf("%s has a non-finite value", name));
    return GPHQ_OK;
}

int gphq_checkpoint_map_bf16(const gphq_checkpoint *c, const char *name, const int64_t *shape, int64_t ndim,
                             gphq_mapping **out, const uint16_t **bits) {
    // safetensors.go:178-200 MapBF16: a read-only mapping of the tensor's
    // pages, or a copy where the offset is odd. gphq_mapping_free releases it.
    clear_detail();
    if (!out || !bits) return fail(GPHQ_ERR_DIMENSIONS, "safetensors: bad arguments");
    *out = nullptr;
    *bits = nullptr;
    const gphq_checkpoint::Tensor *t = nullptr;
    GPHQ_TRY(lookup(c, name, shape, ndim, &t));
    GPHQ_TRY(need_bf16(*t, name));
    gphq_mapping *m = new gphq_mapping();
    const int64_t page = sysconf(_SC_PAGESIZE);
    const int64_t start = t->offset & ~(page - 1);
    if (t->offset % 2 == 0 && t->size > 0) {
        const size_t len = (size_t)(t->offset + t->size - start);
        void *p = mmap(nullptr, len, PROT_READ, MAP_SHARED, t->file, (off_t)start);
        if (p != MAP_FAILED) {
            m->base = p;
            m->len = len;
            *bits = (const uint16_t *)((const char *)p + (t->offset - start));
            *out = m;
            return GPHQ_OK;
        }
    }
    m->copy.resize((size_t)(t->size / 2));
    const int st = read_bits(*t, m->copy.data(), t->size / 2, 0);
    if (st != GPHQ_OK) {
        delete m;
        return st;
    }
    *bits = m->copy.data();
    *out = m;
    return GPHQ_OK;
}

void gphq_mapping_free(gphq_mapping *m) {
    if (!m) return;
    if (m->base) munmap(m->base, m->len);
    delete m;
}

}  // extern "C"
