// Host-side helpers shared by the file formats (safetensors.hip,
// gptq_file.hip, wcache.hip): the thread's last error detail, whole-file and
// positional reads, and directory listings.
#pragma once
#include <stdint.h>

#include <string>
#include <vector>

namespace gphq {

// Sets the calling thread's formatted error detail (gphq_error_detail) and
// returns status, so a check can `return fail(code, "...")`.
int fail(int status, const std::string &detail);
// Clears the detail (a call that succeeds leaves no stale message).
void clear_detail();

// printf-style formatting into a std::string.
std::string strf(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

// Reads exactly len bytes at offset of fd; false on a short read or error.
bool pread_full(int fd, void *dst, size_t len, int64_t offset);
// Writes exactly len bytes; false on error.
bool write_full(int fd, const void *src, size_t len);

// One directory entry: name, size, modification time (ns), whether it is a
// regular file (lstat: a symbolic link is not).
struct DirEntry {
    std::string name;
    int64_t size = 0, mtime_ns = 0;
    bool regular = false;
};
// The entries of dir sorted by name ("." and ".." left out); false if dir
// cannot be read.
bool list_dir(const std::string &dir, std::vector<DirEntry> &out);

// Joins a directory and a file name with one '/'.
std::string join_path(const std::string &dir, const std::string &name);

}  // namespace gphq
