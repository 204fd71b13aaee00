// gphq_gemv_vec_noalloc: the multi-vector GEMV (gphq_gemv_vec) for callers
// that cannot allocate device memory -- code under HIP graph capture, serving
// loops that forbid allocation. Its scratch (the FP16 activation fragments
// and per-block scales the preparation kernel writes) lives in a file-scope
// device array instead of a caller workspace. Each GPU the library runs on
// holds its own copy of the array until the process ends.
//
// Host code never passes the array's name to a kernel: the name is a
// host-side stand-in, not a device address. The device address is resolved
// once per device, with that device current, by hipGetSymbolAddress, and kept
// per device; kernels take that address as their workspace argument.
//
// Every call on one GPU shares that GPU's array and leaves its contents for
// the next call. Nothing has to start at zero (the preparation kernel writes
// every value the GEMV kernels read), but calls that overlap on one GPU (on
// streams not ordered with each other) race on the array.
#include <mutex>

#include "common.h"

namespace gphq {
size_t gemv_vec_workspace_bytes(int V, int K);
int gemv_vec_launch(int fmt, const void *codes, const void *scales, const float *x, long xstride, float *y,
                    long ystride, int V, int K, int N, void *work, hipStream_t stream);
}  // namespace gphq

using namespace gphq;

namespace {

static __device__ __align__(256) uint8_t scratch[GPHQ_GEMV_VEC_NOALLOC_BYTES];

constexpr int kMaxDevices = 64;
std::once_flag g_once[kMaxDevices];
void *g_ptr[kMaxDevices];
hipError_t g_err[kMaxDevices];

// The device address of this device's scratch array (resolved on the first
// call with the device current), or GPHQ_ERR_HIP.
int scratch_for(int dev, void **out) {
    std::call_once(g_once[dev], [dev] {
        void *p = nullptr;
        g_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_ptr[dev] = g_err[dev] == hipSuccess ? p : nullptr;
    });
    if (g_err[dev] != hipSuccess) return hip_status(g_err[dev]);
    *out = g_ptr[dev];
    return GPHQ_OK;
}

}  // namespace

extern "C" {

int gphq_gemv_vec_noalloc(int fmt, const void *codes, const void *scales, const float *x, int64_t x_stride, float *y,
                          int64_t y_stride, int64_t lanes, int64_t k, int64_t n, void *stream) {
    // gphq_gemv_vec's checks in its order, the workspace ones replaced by the
    // scratch limit.
    if (fmt != GPHQ_FMT_Q8 && fmt != GPHQ_FMT_Q8B && fmt != GPHQ_FMT_Q8B_F32 && fmt != GPHQ_FMT_Q4)
        return GPHQ_ERR_UNSUPPORTED;
    if (lanes < 0 || lanes > GPHQ_GEMV_VEC_MAX_LANES || k < 0 || n < 0 || k > INT32_MAX || n > INT32_MAX)
        return GPHQ_ERR_DIMENSIONS;
    if (k % 32 != 0 || x_stride < k || y_stride < n || x_stride % 4 != 0) return GPHQ_ERR_DIMENSIONS;
    if (lanes == 0 || n == 0) return GPHQ_OK;
    if (k && (uintptr_t)x % 16 != 0) return GPHQ_ERR_DIMENSIONS;
    if (gemv_vec_workspace_bytes((int)lanes, (int)k) > (size_t)GPHQ_GEMV_VEC_NOALLOC_BYTES)
        return GPHQ_ERR_SCRATCH_LIMIT;
    if (!y || !scales) return GPHQ_ERR_DIMENSIONS;
    if (k && (!codes || !x || (uintptr_t)codes % 16 != 0)) return GPHQ_ERR_DIMENSIONS;
    // The scratch of the device the launch runs on: the current device, which
    // must own the stream.
    int dev = 0;
    GPHQ_TRY(hip_status(hipGetDevice(&dev)));
    if (dev < 0 || dev >= kMaxDevices) return GPHQ_ERR_UNSUPPORTED;
    if (stream) {
        hipDevice_t sdev = 0;
        GPHQ_TRY(hip_status(hipStreamGetDevice((hipStream_t)stream, &sdev)));
        if ((int)sdev != dev) return GPHQ_ERR_UNSUPPORTED;
    }
    void *work = nullptr;
    GPHQ_TRY(scratch_for(dev, &work));
    return gemv_vec_launch(fmt, codes, scales, x, (long)x_stride, y, (long)y_stride, (int)lanes, (int)k, (int)n, work,
                           (hipStream_t)stream);
}

}  // extern "C"
