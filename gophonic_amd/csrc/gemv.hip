// GEMV over quantized weight rows: y = dequant(W) . x, fp32 activations.
//
// Design (gfx950): a 64-lane wavefront owns R consecutive output rows. Lane l
// streams bytes [16l, 16l+16) of each 1024-byte K step of every owned row with
// one 128-bit load (one wavefront instruction covers 1 KiB of a row,
// contiguous), so a row is read exactly once and the weight stream is fully
// coalesced. B K-steps of all R rows are issued before any arithmetic, which
// puts R*B 128-bit loads per lane in flight; the int8 codes are widened to
// fp32 in registers and multiplied by the fp32 activations, which are read
// through the L1/L2 (every wavefront of the chip reads the same x). Lane
// partial sums are reduced with DPP row permutes plus four readlanes, so no
// LDS and no barrier sits on the path.
//
// Block formats scale each 16-value chunk's partial sum once
// (acc = fma(d, t, acc)), which is the qwen3lm Metal arithmetic
// (gpu.metal:88-100); Q8 adds chunk sums and applies the row scale after the
// reduction (gpu.metal:98-129, q8gemv/scalar.go:13-15). Q4 consumes one
// 32-value block per lane step: acc = fma(d, sum(nib*x) - 8*sum(x), acc)
// (gpu.metal:102-123).
#include "common.h"

namespace gphq {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct GemvArgs {
    const void *codes;
    const void *scales;
    const float *x;
    float *y;
    int K;
    int N;
};

__device__ __forceinline__ float sext_byte_f(uint32_t v, int i) {
    return (float)((int32_t)(v << (24 - 8 * i)) >> 24);
}

// Dot product of 16 int8 codes (one 128-bit load) with 16 fp32 activations,
// as four 4-wide dot products summed, in the order of gpu.metal:91-92.
__device__ __forceinline__ float dot16(const u32x4 w, const float4 x0, const float4 x1, const float4 x2,
                                       const float4 x3) {
    float d0 = sext_byte_f(w.x, 0) * x0.x + sext_byte_f(w.x, 1) * x0.y + sext_byte_f(w.x, 2) * x0.z +
               sext_byte_f(w.x, 3) * x0.w;
    float d1 = sext_byte_f(w.y, 0) * x1.x + sext_byte_f(w.y, 1) * x1.y + sext_byte_f(w.y, 2) * x1.z +
               sext_byte_f(w.y, 3) * x1.w;
    float d2 = sext_byte_f(w.z, 0) * x2.x + sext_byte_f(w.z, 1) * x2.y + sext_byte_f(w.z, 2) * x2.z +
               sext_byte_f(w.z, 3) * x2.w;
    float d3 = sext_byte_f(w.w, 0) * x3.x + sext_byte_f(w.w, 1) * x3.y + sext_byte_f(w.w, 2) * x3.z +
               sext_byte_f(w.w, 3) * x3.w;
    return d0 + d1 + d2 + d3;
}

template <int FMT>
__device__ __forceinline__ float block_scale(const void *scales, size_t idx) {
    if constexpr (FMT == GPHQ_FMT_Q8B || FMT == GPHQ_FMT_Q4) {
        return half_bits_to_float(__builtin_nontemporal_load((const uint16_t *)scales + idx));
    } else {
        return __builtin_nontemporal_load((const float *)scales + idx);
    }
}

// 8-bit codes (Q8, Q8B, Q8B_F32); requires K % 16 == 0 and 16-byte aligned
// codes, so every row starts 16-byte aligned.
template <int FMT, int R, int B>
__global__ __launch_bounds__(256) void gemv8_kernel(GemvArgs a) {
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int row0 = wave * R;
    if (row0 >= a.N) return;
    const int K = a.K;
    const int8_t *W = (const int8_t *)a.codes;
    const size_t kb = (size_t)(K >> 5);
    int rows[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rows[r] = min(row0 + r, a.N - 1);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    for (int base = 0; base < K; base += 1024 * B) {
        u32x4 w[B][R];
        float d[B][R];
#pragma unroll
        for (int j = 0; j < B; ++j) {
            const int k0 = base + j * 1024 + lane * 16;
            const bool ok = k0 < K;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                w[j][r] = ok ? __builtin_nontemporal_load((const u32x4 *)(W + (size_t)rows[r] * K + k0))
                             : u32x4{0, 0, 0, 0};
                if constexpr (FMT != GPHQ_FMT_Q8)
                    d[j][r] = ok ? block_scale<FMT>(a.scales, (size_t)rows[r] * kb + (k0 >> 5)) : 0.0f;
            }
        }
#pragma unroll
        for (int j = 0; j < B; ++j) {
            const int k0 = base + j * 1024 + lane * 16;
            if (k0 < K) {
                const float4 *xv = (const float4 *)(a.x + k0);
                const float4 x0 = xv[0], x1 = xv[1], x2 = xv[2], x3 = xv[3];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float t = dot16(w[j][r], x0, x1, x2, x3);
                    if constexpr (FMT == GPHQ_FMT_Q8)
                        acc[r] += t;
                    else
                        acc[r] = fmaf(d[j][r], t, acc[r]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float s = wave_sum(acc[r]);
        if constexpr (FMT == GPHQ_FMT_Q8) s = s * ((const float *)a.scales)[rows[r]];
        if (lane == r && row0 + r < a.N) a.y[row0 + r] = s;
    }
}

// 4-bit split-nibble codes; requires K % 32 == 0. Lane l takes block
// (step*64 + l): 16 code bytes and 32 activations.
template <int R, int B>
__global__ __launch_bounds__(256) void gemv4_kernel(GemvArgs a) {
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int row0 = wave * R;
    if (row0 >= a.N) return;
    const int K = a.K;
    const uint8_t *W = (const uint8_t *)a.codes;
    const size_t kb = (size_t)(K >> 5);
    const size_t rowBytes = (size_t)(K >> 1);
    int rows[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rows[r] = min(row0 + r, a.N - 1);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    for (int base = 0; base < K; base += 2048 * B) {
        u32x4 w[B][R];
        float d[B][R];
#pragma unroll
        for (int j = 0; j < B; ++j) {
            const int k0 = base + j * 2048 + lane * 32;
            const bool ok = k0 < K;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                w[j][r] = ok ? __builtin_nontemporal_load((const u32x4 *)(W + (size_t)rows[r] * rowBytes + (k0 >> 1)))
                             : u32x4{0, 0, 0, 0};
                d[j][r] = ok ? block_scale<GPHQ_FMT_Q4>(a.scales, (size_t)rows[r] * kb + (k0 >> 5)) : 0.0f;
            }
        }
#pragma unroll
        for (int j = 0; j < B; ++j) {
            const int k0 = base + j * 2048 + lane * 32;
            if (k0 < K) {
                const float4 *xv = (const float4 *)(a.x + k0);
                float4 xs[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) xs[i] = xv[i];
                float4 s4 = xs[0] + xs[1] + xs[2] + xs[3] + xs[4] + xs[5] + xs[6] + xs[7];
                const float sx = (s4.x + s4.y + s4.z + s4.w) * 8.0f;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const uint32_t ww[4] = {w[j][r].x, w[j][r].y, w[j][r].z, w[j][r].w};
                    float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            const uint32_t q = (ww[c] >> (4 * h)) & 0x0F0F0F0Fu;
                            const float4 xv4 = xs[4 * h + c];
                            t.x = fmaf((float)(q & 0xff), xv4.x, t.x);
                            t.y = fmaf((float)((q >> 8) & 0xff), xv4.y, t.y);
                            t.z = fmaf((float)((q >> 16) & 0xff), xv4.z, t.z);
                            t.w = fmaf((float)(q >> 24), xv4.w, t.w);
                        }
                    }
                    acc[r] = fmaf(d[j][r], (t.x + t.y + t.z + t.w) - sx, acc[r]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float s = wave_sum(acc[r]);
        if (lane == r && row0 + r < a.N) a.y[row0 + r] = s;
    }
}

// Any K, any alignment (Q8 only): one wavefront per row, lanes stride through
// the row one code at a time. Used for shapes the vector path cannot take.
__global__ __launch_bounds__(256) void gemv8_generic_kernel(GemvArgs a) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= a.N) return;
    const int8_t *w = (const int8_t *)a.codes + (size_t)row * a.K;
    float acc = 0.0f;
    for (int k = lane; k < a.K; k += 64) acc = fmaf(a.x[k], (float)w[k], acc);
    const float s = wave_sum(acc) * ((const float *)a.scales)[row];
    if (lane == 0) a.y[row] = s;
}

template <typename Kern>
static int launch_rows(Kern kern, const GemvArgs &a, int rowsPerWave, hipStream_t stream) {
    const int wavesPerBlock = 4;
    const long waves = ((long)a.N + rowsPerWave - 1) / rowsPerWave;
    const long blocks = (waves + wavesPerBlock - 1) / wavesPerBlock;
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(64 * wavesPerBlock), 0, stream, a);
    return launch_status();
}

// Chooses a kernel for (fmt, K, N). All arguments were validated by the caller.
int gemv_launch(int fmt, const void *codes, const void *scales, const float *x, float *y, int K, int N,
                hipStream_t stream) {
    if (N == 0) return GPHQ_OK;
    GemvArgs a{codes, scales, x, y, K, N};
    constexpr int R = 2, B = 4;
    switch (fmt) {
    case GPHQ_FMT_Q8: {
        const bool vec = (K % 16 == 0) && ((uintptr_t)codes % 16 == 0) && ((uintptr_t)x % 16 == 0);
        if (!vec) return launch_rows(gemv8_generic_kernel, a, 1, stream);
        return launch_rows(gemv8_kernel<GPHQ_FMT_Q8, R, B>, a, R, stream);
    }
    case GPHQ_FMT_Q8B:
        return launch_rows(gemv8_kernel<GPHQ_FMT_Q8B, R, B>, a, R, stream);
    case GPHQ_FMT_Q8B_F32:
        return launch_rows(gemv8_kernel<GPHQ_FMT_Q8B_F32, R, B>, a, R, stream);
    case GPHQ_FMT_Q4:
        return launch_rows(gemv4_kernel<R, 2>, a, R, stream);
    }
    return GPHQ_ERR_UNSUPPORTED;
}

}  // namespace gphq
