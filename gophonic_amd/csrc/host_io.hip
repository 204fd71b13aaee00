// Host-side helpers of the file formats: the thread's error detail, full
// reads and writes, and sorted directory listings.
#include "host_io.h"

#include <dirent.h>
#include <errno.h>
#include <stdarg.h>
#include <stdio.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>

#include "common.h"

namespace gphq {

static thread_local std::string g_detail;

int fail(int status, const std::string &detail) {
    g_detail = detail;
    return status;
}

void clear_detail() { g_detail.clear(); }

std::string strf(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    va_list ap2;
    va_copy(ap2, ap);
    const int n = vsnprintf(nullptr, 0, fmt, ap);
    va_end(ap);
    std::string out(n > 0 ? (size_t)n : 0, '\0');
    if (n > 0) vsnprintf(&out[0], (size_t)n + 1, fmt, ap2);
    va_end(ap2);
    return out;
}

bool pread_full(int fd, void *dst, size_t len, int64_t offset) {
    char *p = (char *)dst;
    while (len > 0) {
        const ssize_t r = pread(fd, p, len, (off_t)offset);
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return false;
        p += r;
        len -= (size_t)r;
        offset += r;
    }
    return true;
}

bool write_full(int fd, const void *src, size_t len) {
    const char *p = (const char *)src;
    while (len > 0) {
        const ssize_t r = write(fd, p, len);
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return false;
        p += r;
        len -= (size_t)r;
    }
    return true;
}

bool list_dir(const std::string &dir, std::vector<DirEntry> &out) {
    out.clear();
    DIR *d = opendir(dir.c_str());
    if (!d) return false;
    while (struct dirent *e = readdir(d)) {
        const std::string name = e->d_name;
        if (name == "." || name == "..") continue;
        DirEntry de;
        de.name = name;
        struct stat st;
        if (lstat(join_path(dir, name).c_str(), &st) == 0) {
            de.size = (int64_t)st.st_size;
            de.mtime_ns = (int64_t)st.st_mtim.tv_sec * 1000000000LL + st.st_mtim.tv_nsec;
            de.regular = S_ISREG(st.st_mode);
        }
        out.push_back(de);
    }
    closedir(d);
    std::sort(out.begin(), out.end(), [](const DirEntry &a, const DirEntry &b) { return a.name < b.name; });
    return true;
}

std::string join_path(const std::string &dir, const std::string &name) {
    if (dir.empty()) return name;
    return dir.back() == '/' ? dir + name : dir + "/" + name;
}

}  // namespace gphq

extern "C" const char *gphq_error_detail(void) { return gphq::g_detail.c_str(); }
