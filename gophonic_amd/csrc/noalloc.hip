// gphq_gemv_vec_noalloc: the multi-vector GEMV (gphq_gemv_vec) for callers
// that cannot allocate device memory -- code under HIP graph capture, serving
// loops that forbid allocation. Its scratch (the FP16 activation fragments
// and per-block scales the preparation kernel writes) lives in a file-scope
// device array instead of a caller workspace. Each GPU the library runs on
// holds its own copy of the array until the process ends.
//
// Host code never passes the array's name to a kernel: the name is a
// host-side stand-in, not a device address. The device address is resolved
// per device, with that device current, by hipGetSymbolAddress on the first
// call that succeeds, and kept per device; kernels take that address as
// their workspace argument.
//
// Every call on one GPU shares that GPU's array and leaves its contents for
// the next call. Nothing has to start at zero (the preparation kernel writes
// every value the GEMV kernels read), but calls that overlap on one GPU (on
// streams not ordered with each other) race on the array.
#include <atomic>
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
std::mutex g_mu[kMaxDevices];
std::atomic<void *> g_ptr[kMaxDevices];

// The device address of this device's scratch array, resolved with the device
// current on the first call that succeeds (a failed lookup is not kept, so a
// later call tries again), or GPHQ_ERR_HIP. The lookup may run while the
// caller's stream is being captured: this thread's capture mode is relaxed
// around it, which lets a call that is not a stream operation run without
// invalidating the capture.
int scratch_for(int dev, void **out) {
    void *p = g_ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_mu[dev]);
        p = g_ptr[dev].load(std::memory_order_relaxed);
        if (!p) {
            hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
            GPHQ_TRY(hip_status(hipThreadExchangeStreamCaptureMode(&mode)));
            const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            GPHQ_TRY(hip_status(hipThreadExchangeStreamCaptureMode(&mode)));
            if (e != hipSuccess || !p) return hip_status(e != hipSuccess ? e : hipErrorInvalidSymbol);
            g_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
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
