// Small device utilities shared by the entry points. Zero fills use a kernel,
// never hipMemsetAsync, so callers may capture them in a HIP graph.
#include "common.h"

namespace gphq {

__global__ void fill_columns_kernel(float *dst, long stride, int rows, int c0, int c1, float v) {
    const int cols = c1 - c0;
    const size_t total = (size_t)rows * cols;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(i / cols), c = (int)(i % cols);
        dst[(size_t)r * stride + c0 + c] = v;
    }
}

// dst[r*stride + c] = +0.0f for r < rows, c in [c0, c1) (the reference's
// clear() of a K = 0 product, q8gemm/int8.go:187-191, gemm.go:250-255).
int fill_zero_columns(float *dst, long stride, int rows, int c0, int c1, hipStream_t stream) {
    if (rows <= 0 || c1 <= c0) return GPHQ_OK;
    const size_t total = (size_t)rows * (c1 - c0);
    const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, 4096);
    hipLaunchKernelGGL(fill_columns_kernel, dim3(blocks), dim3(256), 0, stream, dst, stride, rows, c0, c1, 0.0f);
    return launch_status();
}

// n floats of dst set to v.
int fill_f32(float *dst, size_t n, float v, hipStream_t stream) {
    if (n == 0) return GPHQ_OK;
    const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(fill_columns_kernel, dim3(blocks), dim3(256), 0, stream, dst, (long)n, 1, 0, (int)n, v);
    return launch_status();
}

}  // namespace gphq
