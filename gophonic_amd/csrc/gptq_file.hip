// The GPTQ weight file cmd/qwen3-gptq writes next to a checkpoint and the GPU
// loader reads (qwen3lm/gptq.go:36-196, writer 227-270): "GPHQ0001", the
// bits (u64 LE), the checkpoint snapshot's fingerprint (u64 LE), then per
// layer and per projection in file order (q, k, v, o, gate, up, down) the
// codes of every row followed by the scales of every row, in the GPU formats:
// 8 bits = GPHQ_FMT_Q8 rows (int8 codes, one fp32 scale per row), 4 bits =
// GPHQ_FMT_Q4 rows (split nibbles, one FP16 scale per 32 values). The reader
// places a projection into a device layer buffer at prepareGPU's offsets,
// the writer takes the codes and scales gphq_gptq_round leaves on the device.
#include <errno.h>
#include <fcntl.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <vector>

#include "common.h"
#include "host_io.h"

using namespace gphq;

namespace {

const char kMagic[8] = {'G', 'P', 'H', 'Q', '0', '0', '0', '1'};
const char *const kProjections[GPHQ_LAYER_PROJECTIONS] = {
    "self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
    "mlp.gate_proj",    "mlp.up_proj",      "mlp.down_proj"};

void put_u64(uint8_t *p, uint64_t v) {
    for (int i = 0; i < 8; ++i) p[i] = (uint8_t)(v >> (8 * i));
}
uint64_t get_u64(const uint8_t *p) {
    uint64_t v = 0;
    for (int i = 7; i >= 0; --i) v = (v << 8) | p[i];
    return v;
}

// gptq.go:82-95 projectionShape.
void projection_shape(const gphq_lm_config &c, int p, int64_t *n, int64_t *k) {
    const int64_t qdim = c.heads * c.head_dim, kvd = c.kv_heads * c.head_dim;
    switch (p) {
    case 0: *n = qdim, *k = c.hidden; return;
    case 1: case 2: *n = kvd, *k = c.hidden; return;
    case 3: *n = c.hidden, *k = qdim; return;
    case 4: case 5: *n = c.intermediate, *k = c.hidden; return;
    }
    *n = c.hidden, *k = c.intermediate;
}

int format_bits(const char *format, int *bits) {
    // gptq.go:197-206: "gpu" is 8 bits, "gpu-q4" 4.
    if (format && !strcmp(format, "gpu")) *bits = 8;
    else if (format && !strcmp(format, "gpu-q4")) *bits = 4;
    else
        return fail(GPHQ_ERR_UNSUPPORTED, strf("qwen3: GPTQ supports \"gpu\" and \"gpu-q4\", not \"%s\"",
                                               format ? format : ""));
    return GPHQ_OK;
}

std::string path_for(const char *dir, const char *format) {
    return join_path(dir, strf("gophonic-gptq-%s.bin", format));  // gptq.go:42, 52-54
}

}  // namespace

namespace gphq {

// The GPTQ format's bits ("gpu" 8, "gpu-q4" 4), or GPHQ_ERR_UNSUPPORTED with
// the reference's message (gptq.go:197-206).
int gptq_format_bits(const char *format, int *bits) { return format_bits(format, bits); }

}  // namespace gphq

struct gphq_gptq_file {
    int fd = -1;
    int bits = 0;
    gphq_lm_config cfg{};
    std::vector<int64_t> offsets;  // per layer and projection
};

struct gphq_gptq_writer {
    int fd = -1;
    std::string tmp, path;
};

// The projection a tensor name after the decoder prefix names
// ("layers.3.mlp.up_proj.weight", gptq.go:145-165): 1 with its code and scale
// offsets and its shape (rows, input width) from the file's configuration, or
// 0 if the file does not hold it.
static int find_projection(const gphq_gptq_file *g, const char *name, int64_t *codes_off, int64_t *scales_off, int64_t *n,
                    int64_t *k) {
    if (!g || !name) return 0;
    if (strncmp(name, "layers.", 7) != 0) return 0;
    char *end = nullptr;
    errno = 0;
    const long long layer = strtoll(name + 7, &end, 10);
    if (end == name + 7 || errno || *end != '.' || layer < 0 || layer >= g->cfg.layers) return 0;
    std::string rest = end + 1;
    if (rest.size() >= 7 && rest.compare(rest.size() - 7, 7, ".weight") == 0) rest.resize(rest.size() - 7);
    for (int p = 0; p < GPHQ_LAYER_PROJECTIONS; ++p)
        if (rest == kProjections[p]) {
            int64_t cb, sb;
            projection_shape(g->cfg, p, n, k);
            gphq_gptq_row_bytes(g->bits, *k, &cb, &sb);
            const int64_t off = g->offsets[(size_t)(layer * GPHQ_LAYER_PROJECTIONS + p)];
            if (codes_off) *codes_off = off;
            if (scales_off) *scales_off = off + *n * cb;
            return 1;
        }
    return 0;
}

extern "C" {

int gphq_gptq_row_bytes(int bits, int64_t k, int64_t *codes, int64_t *scales) {
    // gptq.go:97-103 gptqRowBytes.
    if (!codes || !scales || k < 0 || (bits != 4 && bits != 8)) return GPHQ_ERR_DIMENSIONS;
    if (bits == 4) {
        *codes = k / 2;
        *scales = 2 * (k / 32);
    } else {
        *codes = k;
        *scales = 4;
    }
    return GPHQ_OK;
}

int gphq_gptq_fingerprint(const char *dir, uint64_t *out) {
    // gptq.go:56-80 snapshotFingerprint: FNV-1a 64 over "name size mtime_ns\n"
    // of the sorted *.safetensors and config.json files.
    clear_detail();
    if (!dir || !out) return fail(GPHQ_ERR_DIMENSIONS, "gptq: bad arguments");
    std::vector<DirEntry> entries;
    if (!list_dir(dir, entries)) return fail(GPHQ_ERR_IO, strf("gptq: read directory %s", dir));
    uint64_t h = 0xcbf29ce484222325ull;  // FNV-1a 64 offset basis
    for (const DirEntry &e : entries) {
        const size_t L = e.name.size();
        const bool st = L >= 12 && e.name.compare(L - 12, 12, ".safetensors") == 0;
        if (!st && e.name != "config.json") continue;
        struct stat s;
        if (stat(join_path(dir, e.name).c_str(), &s) != 0)
            return fail(GPHQ_ERR_IO, strf("gptq: stat %s", e.name.c_str()));
        const long long mtime = (long long)s.st_mtim.tv_sec * 1000000000LL + s.st_mtim.tv_nsec;
        const std::string line = strf("%s %lld %lld\n", e.name.c_str(), (long long)s.st_size, mtime);
        for (unsigned char ch : line) {
            h ^= ch;
            h *= 0x100000001b3ull;  // FNV-1a 64 prime
        }
    }
    *out = h;
    return GPHQ_OK;
}

int gphq_gptq_path(const char *dir, const char *format, char *out, int64_t out_len) {
    clear_detail();
    if (!dir || !format || !out) return fail(GPHQ_ERR_DIMENSIONS, "gptq: bad arguments");
    const std::string p = path_for(dir, format);
    if ((int64_t)p.size() + 1 > out_len) return fail(GPHQ_ERR_DIMENSIONS, "gptq: path buffer too short");
    memcpy(out, p.c_str(), p.size() + 1);
    return GPHQ_OK;
}

int gphq_gptq_open(const char *dir, const char *format, const gphq_lm_config *cfg, gphq_gptq_file **out) {
    // gptq.go:113-140 openGPTQ: *out stays NULL (and the status is GPHQ_OK)
    // when there is no file, or it was made for other bits or from other
    // checkpoint files, or its size is not the model's.
    clear_detail();
    if (!out || !dir || !cfg) return fail(GPHQ_ERR_DIMENSIONS, "gptq: bad arguments");
    *out = nullptr;
    int bits = 0;
    GPHQ_TRY(format_bits(format, &bits));
    const int fd = open(path_for(dir, format).c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return GPHQ_OK;
    uint8_t head[24];
    uint64_t fp = 0;
    const bool fpOk = gphq_gptq_fingerprint(dir, &fp) == GPHQ_OK;
    clear_detail();
    if (!pread_full(fd, head, 24, 0) || !fpOk || memcmp(head, kMagic, 8) != 0 || get_u64(head + 8) != (uint64_t)bits ||
        get_u64(head + 16) != fp) {
        close(fd);
        return GPHQ_OK;
    }
    gphq_gptq_file *g = new gphq_gptq_file();
    g->fd = fd;
    g->bits = bits;
    g->cfg = *cfg;
    int64_t off = 24;
    for (int64_t layer = 0; layer < cfg->layers; ++layer)
        for (int p = 0; p < GPHQ_LAYER_PROJECTIONS; ++p) {
            g->offsets.push_back(off);
            int64_t n, k, cb, sb;
            projection_shape(*cfg, p, &n, &k);
            gphq_gptq_row_bytes(bits, k, &cb, &sb);
            off += n * (cb + sb);
        }
    struct stat st;
    if (fstat(fd, &st) != 0 || (int64_t)st.st_size != off) {
        gphq_gptq_close(g);
        return GPHQ_OK;
    }
    *out = g;
    return GPHQ_OK;
}

void gphq_gptq_close(gphq_gptq_file *g) {
    if (!g) return;
    if (g->fd >= 0) close(g->fd);
    delete g;
}

int gphq_gptq_bits(const gphq_gptq_file *g) { return g ? g->bits : 0; }

int gphq_gptq_projection(const gphq_gptq_file *g, const char *name, int64_t *codes_off, int64_t *scales_off) {
    // gptq.go:145-165 projection: the offsets of a tensor named after the
    // decoder prefix ("layers.3.mlp.up_proj.weight"); 1 if the file holds it.
    int64_t n, k;
    return find_projection(g, name, codes_off, scales_off, &n, &k);
}

int gphq_gptq_place(const gphq_gptq_file *g, const char *name, int64_t n, int64_t k, void *buf_dev, int64_t buf_bytes,
                    int64_t base, int64_t sc, int64_t row0, int64_t step, int *placed) {
    // gptq.go:170-190 place: source row r lands at row row0 + r*step of the
    // codes at byte offset base and of the scales at sc of a device layer
    // buffer. *placed = 0 when the file does not hold the projection.
    clear_detail();
    if (!g || !name || !placed || !buf_dev || n < 0 || k < 0 || row0 < 0 || step < 1 || base < 0 || sc < 0)
        return fail(GPHQ_ERR_DIMENSIONS, "gptq: bad arguments");
    *placed = 0;
    int64_t codesAt = 0, scalesAt = 0, fn = 0, fk = 0;
    if (!find_projection(g, name, &codesAt, &scalesAt, &fn, &fk)) return GPHQ_OK;
    // The file's own layout bounds what is read: a caller's n or k that is
    // not the projection's shape would read into the next projection.
    if (n != fn || k != fk)
        return fail(GPHQ_ERR_DIMENSIONS, strf("gptq: %s is %lldx%lld in the file, not %lldx%lld", name, (long long)fn,
                                              (long long)fk, (long long)n, (long long)k));
    int64_t cb, sb;
    GPHQ_TRY(gphq_gptq_row_bytes(g->bits, k, &cb, &sb));
    if (n == 0) {
        *placed = 1;
        return GPHQ_OK;
    }
    const int64_t last = row0 + (n - 1) * step;
    if (base + (last + 1) * cb > buf_bytes || sc + (last + 1) * sb > buf_bytes)
        return fail(GPHQ_ERR_DIMENSIONS, "gptq: projection does not fit the layer buffer");
    std::vector<uint8_t> codes((size_t)(n * cb)), scales((size_t)(n * sb));
    if (!pread_full(g->fd, codes.data(), codes.size(), codesAt) ||
        !pread_full(g->fd, scales.data(), scales.size(), scalesAt))
        return fail(GPHQ_ERR_IO, strf("gptq: read %s", name));
    uint8_t *dst = (uint8_t *)buf_dev;
    GPHQ_TRY(hip_status(hipMemcpy2D(dst + base + row0 * cb, (size_t)(step * cb), codes.data(), (size_t)cb, (size_t)cb,
                                    (size_t)n, hipMemcpyHostToDevice)));
    GPHQ_TRY(hip_status(hipMemcpy2D(dst + sc + row0 * sb, (size_t)(step * sb), scales.data(), (size_t)sb, (size_t)sb,
                                    (size_t)n, hipMemcpyHostToDevice)));
    *placed = 1;
    return GPHQ_OK;
}

int gphq_gptq_create(const char *dir, const char *format, gphq_gptq_writer **out) {
    // QuantizeGPTQ's file (gptq.go:227-240): a temporary file next to the
    // checkpoint, the 24-byte header written first.
    clear_detail();
    if (!out || !dir) return fail(GPHQ_ERR_DIMENSIONS, "gptq: bad arguments");
    *out = nullptr;
    int bits = 0;
    GPHQ_TRY(format_bits(format, &bits));
    uint64_t fp = 0;
    GPHQ_TRY(gphq_gptq_fingerprint(dir, &fp));
    gphq_gptq_writer *w = new gphq_gptq_writer();
    w->path = path_for(dir, format);
    w->tmp = w->path + ".tmp";
    w->fd = open(w->tmp.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
    if (w->fd < 0) {
        const int e = errno;
        delete w;
        return fail(GPHQ_ERR_IO, strf("gptq: create %s.tmp: %s", path_for(dir, format).c_str(), strerror(e)));
    }
    uint8_t head[24];
    memcpy(head, kMagic, 8);
    put_u64(head + 8, (uint64_t)bits);
    put_u64(head + 16, fp);
    if (!write_full(w->fd, head, 24)) {
        gphq_gptq_abort(w);
        return fail(GPHQ_ERR_IO, "gptq: write header");
    }
    *out = w;
    return GPHQ_OK;
}

int gphq_gptq_write(gphq_gptq_writer *w, const void *data, int64_t len) {
    clear_detail();
    if (!w || len < 0 || (len && !data)) return fail(GPHQ_ERR_DIMENSIONS, "gptq: bad arguments");
    if (!write_full(w->fd, data, (size_t)len)) return fail(GPHQ_ERR_IO, "gptq: write");
    return GPHQ_OK;
}

int gphq_gptq_write_device(gphq_gptq_writer *w, const void *data_dev, int64_t len) {
    // Codes or scales from device memory (gphq_gptq_round's outputs).
    clear_detail();
    if (!w || len < 0 || (len && !data_dev)) return fail(GPHQ_ERR_DIMENSIONS, "gptq: bad arguments");
    std::vector<uint8_t> host((size_t)len);
    if (len) GPHQ_TRY(hip_status(hipMemcpy(host.data(), data_dev, (size_t)len, hipMemcpyDeviceToHost)));
    return gphq_gptq_write(w, host.data(), len);
}

int gphq_gptq_commit(gphq_gptq_writer *w) {
    // gptq.go:258-270: flush, close, then rename into place.
    clear_detail();
    if (!w) return fail(GPHQ_ERR_DIMENSIONS, "gptq: bad arguments");
    int st = GPHQ_OK;
    if (fsync(w->fd) != 0 || close(w->fd) != 0) st = fail(GPHQ_ERR_IO, "gptq: close");
    w->fd = -1;
    if (st == GPHQ_OK && rename(w->tmp.c_str(), w->path.c_str()) != 0) st = fail(GPHQ_ERR_IO, "gptq: rename");
    if (st != GPHQ_OK) unlink(w->tmp.c_str());
    delete w;
    return st;
}

void gphq_gptq_abort(gphq_gptq_writer *w) {
    if (!w) return;
    if (w->fd >= 0) close(w->fd);
    unlink(w->tmp.c_str());
    delete w;
}

}  // extern "C"
