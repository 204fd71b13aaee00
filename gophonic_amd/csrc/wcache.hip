// Prepared-weight cache files (internal/wcache/wcache.go): a checkpoint is
// prepared once, into a memory-mapped entry; later loads map the committed
// entry and, on this discrete GPU, upload from the mapping (the reference
// hands the mapped pages to a unified-memory GPU without a copy).
//
// An entry is a 16 KiB header ("GPHWCACH", total size u64 LE, complete flag
// u64 LE) followed by a payload of 16 KiB-aligned regions. A fresh entry is
// a temporary file that the caller fills and commits: the payload reaches
// the disk before the complete flag, the file is renamed into place, and the
// entries it replaces (same checkpoint and kind, other hash) are removed. An
// advisory lock makes one process prepare an entry while others wait to map
// it. Without a cache directory an entry lives in anonymous memory.
#include <errno.h>
#include <fcntl.h>
#include <glob.h>
#include <limits.h>
#include <stdlib.h>
#include <string.h>
#include <sys/file.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <time.h>
#include <unistd.h>

#include <string>
#include <vector>

#include "common.h"
#include "host_io.h"

using namespace gphq;

namespace {

constexpr int64_t kAlign = GPHQ_WCACHE_ALIGN;
constexpr int64_t kHeader = kAlign;
constexpr uint64_t kComplete = 1;
const char kMagic[8] = {'G', 'P', 'H', 'W', 'C', 'A', 'C', 'H'};

int64_t round_up(int64_t n) { return (n + kAlign - 1) & ~(kAlign - 1); }

void put_u64(uint8_t *p, uint64_t v) {
    for (int i = 0; i < 8; ++i) p[i] = (uint8_t)(v >> (8 * i));
}
uint64_t get_u64(const uint8_t *p) {
    uint64_t v = 0;
    for (int i = 7; i >= 0; --i) v = (v << 8) | p[i];
    return v;
}

// SHA-256 (FIPS 180-4), for entry keys.
struct Sha256 {
    uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a, 0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    uint8_t buf[64];
    size_t used = 0;
    uint64_t bits = 0;
    static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
    void block(const uint8_t *p) {
        static const uint32_t K[64] = {
            0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
            0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
            0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
            0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
            0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
            0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
            0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
            0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};
        uint32_t w[64];
        for (int i = 0; i < 16; ++i)
            w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 | (uint32_t)p[4 * i + 2] << 8 | p[4 * i + 3];
        for (int i = 16; i < 64; ++i) {
            const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], k = h[7];
        for (int i = 0; i < 64; ++i) {
            const uint32_t t1 = k + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + K[i] + w[i];
            const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
            k = g, g = f, f = e, e = d + t1, d = c, c = b, b = a, a = t1 + t2;
        }
        h[0] += a, h[1] += b, h[2] += c, h[3] += d, h[4] += e, h[5] += f, h[6] += g, h[7] += k;
    }
    void add(const void *data, size_t n) {
        const uint8_t *p = (const uint8_t *)data;
        bits += (uint64_t)n * 8;
        while (n > 0) {
            const size_t take = std::min(n, 64 - used);
            memcpy(buf + used, p, take);
            used += take, p += take, n -= take;
            if (used == 64) block(buf), used = 0;
        }
    }
    void add(const std::string &s) { add(s.data(), s.size()); }
    void sum(uint8_t out[32]) {
        const uint64_t total = bits;
        const uint8_t one = 0x80, zero = 0;
        add(&one, 1);
        while (used != 56) add(&zero, 1);
        uint8_t len[8];
        for (int i = 0; i < 8; ++i) len[i] = (uint8_t)(total >> (56 - 8 * i));
        add(len, 8);
        for (int i = 0; i < 8; ++i)
            for (int j = 0; j < 4; ++j) out[4 * i + j] = (uint8_t)(h[i] >> (24 - 8 * j));
    }
};

std::string hex(const uint8_t *p, size_t n) {
    static const char *d = "0123456789abcdef";
    std::string s;
    for (size_t i = 0; i < n; ++i) s += d[p[i] >> 4], s += d[p[i] & 15];
    return s;
}

// wcache.go:88-96 sanitize: per Unicode code point, letters, digits, '-'
// and '_' stay, anything else becomes '_'.
std::string sanitize(const std::string &s) {
    std::string out;
    for (size_t i = 0; i < s.size();) {
        const unsigned char c = (unsigned char)s[i];
        size_t len = 1;
        if (c >= 0xF0) len = 4;
        else if (c >= 0xE0) len = 3;
        else if (c >= 0xC0) len = 2;
        const bool keep = len == 1 && ((c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z') || (c >= '0' && c <= '9') ||
                                       c == '-' || c == '_');
        out += keep ? (char)c : '_';
        i += std::min(len, s.size() - i);
    }
    return out;
}

// filepath.Abs + Clean: a lexical absolute path (no symlink resolution).
std::string abs_clean(const std::string &p) {
    std::string full = p;
    if (p.empty() || p[0] != '/') {
        char cwd[PATH_MAX];
        if (!getcwd(cwd, sizeof cwd)) return "";
        full = std::string(cwd) + "/" + p;
    }
    std::vector<std::string> parts;
    size_t i = 0;
    while (i <= full.size()) {
        size_t j = full.find('/', i);
        if (j == std::string::npos) j = full.size();
        const std::string seg = full.substr(i, j - i);
        if (seg == "..") {
            if (!parts.empty()) parts.pop_back();
        } else if (!seg.empty() && seg != ".") {
            parts.push_back(seg);
        }
        i = j + 1;
    }
    std::string out;
    for (const std::string &s : parts) out += "/" + s;
    return out.empty() ? "/" : out;
}

std::string base_name(const std::string &p) {
    const size_t k = p.find_last_of('/');
    return k == std::string::npos ? p : p.substr(k + 1);
}

std::string default_dir() {
    // wcache.go:49-57: $GOPHONIC_CACHE, else the user cache directory
    // ($XDG_CACHE_HOME or ~/.cache) / gophonic.
    if (const char *d = getenv("GOPHONIC_CACHE")) return d;
    if (const char *x = getenv("XDG_CACHE_HOME"); x && x[0] == '/') return join_path(x, "gophonic");
    const char *home = getenv("HOME");
    if (!home || !home[0]) return "";
    return join_path(join_path(home, ".cache"), "gophonic");
}

// wcache.go:11-31 lock_unix.go lock: an exclusive advisory lock on path.
int lock_file(const std::string &path) {
    const int fd = open(path.c_str(), O_CREAT | O_RDWR | O_CLOEXEC, 0644);
    if (fd < 0) return -1;
    int r;
    do r = flock(fd, LOCK_EX);
    while (r != 0 && errno == EINTR);
    if (r != 0) {
        close(fd);
        return -1;
    }
    return fd;
}

}  // namespace

struct gphq_wcache_file {
    uint8_t *data = nullptr;  // the whole mapping: header, then the payload
    size_t len = 0;
    int fd = -1;              // the temporary file of a fresh entry
    int lock = -1;            // held while a fresh entry is prepared
    std::string path, tmp;
    bool fresh = false;
    bool anon = false;
};

namespace {

// wcache.go:142-162 openComplete.
gphq_wcache_file *open_complete(const std::string &path, int64_t total) {
    const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return nullptr;
    struct stat st;
    if (fstat(fd, &st) != 0 || (int64_t)st.st_size != total) {
        close(fd);
        return nullptr;
    }
    void *p = mmap(nullptr, (size_t)total, PROT_READ, MAP_SHARED, fd, 0);
    close(fd);
    if (p == MAP_FAILED) return nullptr;
    const uint8_t *d = (const uint8_t *)p;
    if (memcmp(d, kMagic, 8) != 0 || get_u64(d + 8) != (uint64_t)total || get_u64(d + 16) != kComplete) {
        munmap(p, (size_t)total);
        return nullptr;
    }
    gphq_wcache_file *f = new gphq_wcache_file();
    f->data = (uint8_t *)p;
    f->len = (size_t)total;
    f->path = path;
    return f;
}

// wcache.go:164-186 create.
gphq_wcache_file *create_entry(const std::string &path, int64_t total) {
    std::string tmpl = path + ".XXXXXX.tmp";
    std::vector<char> name(tmpl.begin(), tmpl.end());
    name.push_back('\0');
    const int fd = mkstemps(name.data(), 4);
    if (fd < 0) return nullptr;
    const std::string tmp(name.data());
    void *p = MAP_FAILED;
    if (ftruncate(fd, (off_t)total) == 0) p = mmap(nullptr, (size_t)total, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
    if (p == MAP_FAILED) {
        close(fd);
        unlink(tmp.c_str());
        return nullptr;
    }
    uint8_t *d = (uint8_t *)p;
    memcpy(d, kMagic, 8);
    put_u64(d + 8, (uint64_t)total);
    gphq_wcache_file *f = new gphq_wcache_file();
    f->data = d;
    f->len = (size_t)total;
    f->fd = fd;
    f->path = path;
    f->tmp = tmp;
    f->fresh = true;
    return f;
}

gphq_wcache_file *anonymous(int64_t total) {
    void *p = mmap(nullptr, (size_t)total, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
    if (p == MAP_FAILED) return nullptr;
    gphq_wcache_file *f = new gphq_wcache_file();
    f->data = (uint8_t *)p;
    f->len = (size_t)total;
    f->fresh = true;
    f->anon = true;
    return f;
}

// wcache.go:233-258 publish.
bool publish(gphq_wcache_file *f) {
    if (msync(f->data, f->len, MS_SYNC) != 0 || fsync(f->fd) != 0) return false;
    put_u64(f->data + 16, kComplete);  // the payload is on disk before the mark
    if (msync(f->data, kHeader, MS_SYNC) != 0 || fsync(f->fd) != 0) return false;
    if (rename(f->tmp.c_str(), f->path.c_str()) != 0) return false;
    // Remove the entries this one replaces: same checkpoint and kind
    // ("<name>-<where>.<kind>."), another hash.
    const std::string name = base_name(f->path);
    const std::string stem = name.size() > 4 ? name.substr(0, name.size() - 4) : name;  // without ".bin"
    const std::string prefix = stem.substr(0, stem.find_last_of('.') + 1);
    const std::string dir = f->path.substr(0, f->path.size() - name.size());
    std::vector<DirEntry> entries;
    if (list_dir(dir.empty() ? "." : dir, entries)) {
        const time_t now = time(nullptr);
        for (const DirEntry &e : entries) {
            if (e.name.compare(0, prefix.size(), prefix) != 0) continue;
            const std::string full = join_path(dir.empty() ? "." : dir, e.name);
            const size_t L = e.name.size();
            if (L >= 4 && e.name.compare(L - 4, 4, ".bin") == 0) {
                const std::string rest = e.name.substr(prefix.size(), L - 4 - prefix.size());
                if (full != f->path && e.name != name && rest.find('.') == std::string::npos) unlink(full.c_str());
            } else if (L >= 4 && e.name.compare(L - 4, 4, ".tmp") == 0) {
                // Temporary files an hour old were left by processes that died.
                if (now - (time_t)(e.mtime_ns / 1000000000LL) > 3600) unlink(full.c_str());
            }
        }
    }
    return true;
}

}  // namespace

extern "C" {

int64_t gphq_wcache_round_up(int64_t n) {
    // wcache.go:312 roundUp, of max(n, 1) as Layout.Take rounds (wcache.go:299-306).
    return n < 0 ? GPHQ_ERR_DIMENSIONS : round_up(std::max<int64_t>(n, 1));
}

int gphq_wcache_key(const char *dir, const char *kind, const char *const *parts, int64_t nparts, char *out,
                    int64_t out_len) {
    // wcache.go:63-86 Key: "<name>-<where>.<kind>.<hash>", where hashes the
    // absolute checkpoint path and hash covers the parts and every regular
    // file's name, size and modification time.
    clear_detail();
    if (!dir || !kind || !out || nparts < 0 || (nparts && !parts)) return fail(GPHQ_ERR_DIMENSIONS, "wcache: bad arguments");
    const std::string abs = abs_clean(dir);
    if (abs.empty()) return fail(GPHQ_ERR_IO, "wcache: no working directory");
    std::vector<DirEntry> entries;
    if (!list_dir(abs, entries)) return fail(GPHQ_ERR_IO, strf("wcache: read directory %s", abs.c_str()));
    Sha256 h;
    for (int64_t i = 0; i < nparts; ++i) {
        h.add(parts[i] ? parts[i] : "", parts[i] ? strlen(parts[i]) : 0);
        h.add("\0", 1);
    }
    for (const DirEntry &e : entries) {
        if (!e.regular) continue;
        h.add(e.name);
        h.add("\0", 1);
        h.add(std::to_string(e.size));
        h.add("\0", 1);
        h.add(std::to_string(e.mtime_ns));
        h.add("\0", 1);
    }
    uint8_t digest[32], where[32];
    h.sum(digest);
    Sha256 w;
    w.add(abs);
    w.sum(where);
    const std::string key = sanitize(base_name(abs)) + "-" + hex(where, 4) + "." + sanitize(kind) + "." + hex(digest, 12);
    if ((int64_t)key.size() + 1 > out_len) return fail(GPHQ_ERR_DIMENSIONS, "wcache: key buffer too short");
    memcpy(out, key.c_str(), key.size() + 1);
    return GPHQ_OK;
}

int gphq_wcache_sha256(const void *data, int64_t len, uint8_t *out32) {
    // The key's hash function, exposed for its known-answer tests.
    if (len < 0 || (len && !data) || !out32) return GPHQ_ERR_DIMENSIONS;
    Sha256 h;
    h.add(data, (size_t)len);
    h.sum(out32);
    return GPHQ_OK;
}

int gphq_wcache_open(const char *cache_dir, const char *key, int64_t size, gphq_wcache_file **out) {
    // wcache.go:109-140 Open. cache_dir NULL: the default directory; "":
    // no directory (anonymous memory).
    clear_detail();
    if (!out || !key) return fail(GPHQ_ERR_DIMENSIONS, "wcache: bad arguments");
    *out = nullptr;
    if (size < 0) return fail(GPHQ_ERR_DIMENSIONS, "wcache: negative size");
    const int64_t total = kHeader + round_up(std::max<int64_t>(size, 1));
    const std::string dir = cache_dir ? std::string(cache_dir) : default_dir();
    if (!dir.empty()) {
        const std::string path = join_path(dir, std::string(key) + ".bin");
        if (gphq_wcache_file *f = open_complete(path, total)) {
            *out = f;
            return GPHQ_OK;
        }
        // One loader prepares an entry; others wait for it and map it.
        mkdir(dir.c_str(), 0755);
        const std::string k(key);
        const int lk = lock_file(join_path(dir, k.substr(0, k.find_last_of('.') + 1) + "lock"));
        if (gphq_wcache_file *f = open_complete(path, total)) {
            if (lk >= 0) close(lk);
            *out = f;
            return GPHQ_OK;
        }
        if (gphq_wcache_file *f = create_entry(path, total)) {
            f->lock = lk;
            *out = f;
            return GPHQ_OK;
        }
        if (lk >= 0) close(lk);
    }
    gphq_wcache_file *f = anonymous(total);
    if (!f) return fail(GPHQ_ERR_IO, "wcache: anonymous mapping failed");
    *out = f;
    return GPHQ_OK;
}

int gphq_wcache_fresh(const gphq_wcache_file *f) { return f && f->fresh ? 1 : 0; }

void *gphq_wcache_payload(gphq_wcache_file *f, int64_t *len) {
    // wcache.go:193-196 Payload: the bytes after the header.
    if (!f || !f->data) {
        if (len) *len = 0;
        return nullptr;
    }
    if (len) *len = (int64_t)(f->len - kHeader);
    return f->data + kHeader;
}

void gphq_wcache_done(gphq_wcache_file *f, const void *region, int64_t len) {
    // wcache.go:198-205 Done: start writing a filled region back.
    if (!f || !f->fresh || f->fd < 0 || !region || len <= 0) return;
    const uintptr_t page = (uintptr_t)sysconf(_SC_PAGESIZE);
    const uintptr_t a = (uintptr_t)region & ~(page - 1);
    msync((void *)a, (size_t)((uintptr_t)region + (uintptr_t)len - a), MS_ASYNC);
}

void gphq_wcache_commit(gphq_wcache_file *f) {
    // wcache.go:207-231 Commit.
    if (!f || !f->fresh) return;
    f->fresh = false;
    if (f->anon) return;  // anonymous memory: nothing to publish
    const bool ok = publish(f);
    close(f->fd);
    f->fd = -1;
    if (f->lock >= 0) close(f->lock);
    f->lock = -1;
    if (!ok) {
        unlink(f->tmp.c_str());
        void *mem = mmap(nullptr, f->len, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
        if (mem != MAP_FAILED) {
            memcpy(mem, f->data, f->len);
            munmap(f->data, f->len);
            f->data = (uint8_t *)mem;
            f->anon = true;
        }
        return;
    }
    gphq_wcache_file *done = open_complete(f->path, (int64_t)f->len);
    if (!done) return;  // keep the writable mapping of the published file
    munmap(f->data, f->len);
    f->data = done->data;
    done->data = nullptr;
    delete done;
}

int gphq_wcache_close(gphq_wcache_file *f) {
    // wcache.go:262-277 Close: discards a still-fresh entry.
    if (!f) return GPHQ_OK;
    if (f->fresh && f->fd >= 0) {
        close(f->fd);
        unlink(f->tmp.c_str());
        if (f->lock >= 0) close(f->lock);
    }
    const int r = f->data ? munmap(f->data, f->len) : 0;
    delete f;
    return r == 0 ? GPHQ_OK : GPHQ_ERR_IO;
}

}  // extern "C"
