// GEMV over quantized weight rows: y = dequant(W) . x, fp32 activations.
//
// Design (gfx950, measured on MI355X): a block of WPB wavefronts is SK K-slices
// x (WPB/SK) row groups of RW rows. Lane l of a wavefront streams bytes
// [16l, 16l+16) of each 1024-value K step of its RW rows with one 128-bit
// non-temporal load (one wavefront instruction = 1 KiB of one row,
// contiguous; every weight byte is read once). The wavefront's slice of x is
// loaded first, into registers, and reused for all RW rows, so x crosses the
// vector memory pipe once per row group rather than once per row; x and the
// block scales are requested before the weights because one wavefront's
// loads return in issue order. Codes are widened to fp32 in registers
// (v_cvt_f32_i32 with SDWA byte select) and multiplied by fp32 x. Lane
// partials are reduced with DPP row permutes plus four readlanes; the SK
// slice totals of a row meet in LDS and are added in slice order, so results
// are deterministic.
//
// One launch can run up to kMaxBatch independent GEMVs of the same shape
// (grid.y = GEMV), the equivalent of encoding several projections into one
// command buffer in the reference's projection stream
// (qwen3lm/gpu_projection_stream_darwin_test.go:75-90).
//
// Arithmetic per format follows qwen3lm/gpu.metal:85-129: block formats scale
// each 16-value chunk's partial sum once (acc = fma(d, t, acc)); Q8 adds chunk
// sums and applies the row scale after the reduction (also q8gemv/scalar.go);
// Q4 takes one 32-value block per lane step and computes
// acc = fma(d, sum(nib*x) - 8*sum(x), acc).
#include "common.h"

namespace gphq {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxBatch = 32;

struct GemvSet {
    const void *codes;
    const void *scales;
    const float *x;
    float *y;
};

template <int MAXB>
struct GemvBatch {
    GemvSet set[MAXB];
    int K;
    int N;
    float eps;  // PRO_NORM only
};

// Prologue and epilogue of the decode-step GEMVs (qwen3lm/gpu.metal:63-64,
// 72-80, 131-161). PRO_NORM scales the result by 1/sqrt(mean(x^2) + eps),
// the RMSNorm of the input whose weight is folded into the rows; the sum of
// squares comes from the x values the block already holds in registers.
// EPI_ADD adds the result into y (the residual stream). EPI_SWIGLU takes
// rows 2i (gate) and 2i+1 (up) and stores g/(1+exp(-g))*u at y[i].
enum { PRO_PLAIN = 0, PRO_NORM = 1 };
enum { EPI_STORE = 0, EPI_ADD = 1, EPI_SWIGLU = 2 };

__device__ __forceinline__ float sext_byte_f(uint32_t v, int i) {
    return (float)((int32_t)(v << (24 - 8 * i)) >> 24);
}

// Dot product of 16 int8 codes (one 128-bit load) with 16 fp32 activations,
// as four 4-wide dot products summed (gpu.metal:91-92).
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

// Adds the SK slice totals of each row (in slice order), applies the
// prologue's norm factor, the Q8 row scale and the epilogue. pss holds the SK
// slice sums of x^2 (PRO_NORM).
template <int FMT, int PRO, int EPI, int ROWS, int SK>
__device__ __forceinline__ void finish_rows(float (*part)[SK], const float *pss, const GemvSet &s, int rowBlock,
                                            int N, int K, float eps) {
    __syncthreads();
    float inv = 1.0f;
    if constexpr (PRO == PRO_NORM) {
        float ss = pss[0];
#pragma unroll
        for (int i = 1; i < SK; ++i) ss += pss[i];
        inv = 1.0f / sqrtf(ss / (float)K + eps);
    }
    auto total = [&](int r, int row) {
        float t = part[r][0];
#pragma unroll
        for (int i = 1; i < SK; ++i) t += part[r][i];
        t = t * inv;
        if constexpr (FMT == GPHQ_FMT_Q8) t = t * ((const float *)s.scales)[row];
        return t;
    };
    if constexpr (EPI == EPI_SWIGLU) {
        const int r = 2 * (int)threadIdx.x;
        if (r < ROWS) {
            const int row = rowBlock + r;
            if (row + 1 < N) {
                const float g = total(r, row), u = total(r + 1, row + 1);
                s.y[row >> 1] = g / (1.0f + expf(-g)) * u;
            }
        }
    } else if ((int)threadIdx.x < ROWS) {
        const int row = rowBlock + threadIdx.x;
        if (row < N) {
            const float t = total(threadIdx.x, row);
            if constexpr (EPI == EPI_ADD)
                s.y[row] += t;
            else
                s.y[row] = t;
        }
    }
}

// 8-bit codes (Q8, Q8B, Q8B_F32). Requires K % 16 == 0, 16-byte aligned codes
// and x (every row then starts 16-byte aligned).
// U > 1 issues the loads of U consecutive K steps before using any of them
// (more bytes in flight per wavefront for short, latency-bound GEMVs).
template <int FMT, int RW, int SK, int WPB, int MAXB, int PRO = PRO_PLAIN, int EPI = EPI_STORE, int U = 1>
__global__ __launch_bounds__(64 * WPB) void gemv8_kernel(const GemvBatch<MAXB> b) {
    constexpr int RG = WPB / SK;
    __shared__ float part[RG * RW][SK];
    __shared__ float pss[SK];
    const GemvSet s = b.set[blockIdx.y];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int rg = wv / SK, ks = wv % SK;
    const int rowBlock = blockIdx.x * (RG * RW);
    const int row0 = rowBlock + rg * RW;
    const int K = b.K;
    const int steps = (K + SK * 1024 - 1) / (SK * 1024);
    const int8_t *W = (const int8_t *)s.codes;
    const size_t kb = (size_t)(K >> 5);
    int rows[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) rows[r] = min(row0 + r, b.N - 1);
    float acc[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) acc[r] = 0.0f;
    float ss = 0.0f;

    for (int st0 = 0; st0 < steps; st0 += U) {
        float4 xr[U][4];
        float d[U][RW];
        u32x4 w[U][RW];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k0 = (ks * steps + st0 + u) * 1024 + lane * 16;
            const bool ok = st0 + u < steps && k0 < K;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                xr[u][i] = ok ? *((const float4 *)(s.x + k0) + i) : make_float4(0.f, 0.f, 0.f, 0.f);
            if constexpr (FMT != GPHQ_FMT_Q8) {
#pragma unroll
                for (int r = 0; r < RW; ++r)
                    d[u][r] = ok ? block_scale<FMT>(s.scales, (size_t)rows[r] * kb + (k0 >> 5)) : 0.0f;
            }
#pragma unroll
            for (int r = 0; r < RW; ++r)
                w[u][r] = ok ? __builtin_nontemporal_load((const u32x4 *)(W + (size_t)rows[r] * K + k0))
                             : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if constexpr (PRO == PRO_NORM) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    ss += xr[u][i].x * xr[u][i].x + xr[u][i].y * xr[u][i].y + xr[u][i].z * xr[u][i].z +
                          xr[u][i].w * xr[u][i].w;
            }
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                const float t = dot16(w[u][r], xr[u][0], xr[u][1], xr[u][2], xr[u][3]);
                if constexpr (FMT == GPHQ_FMT_Q8)
                    acc[r] += t;
                else
                    acc[r] = fmaf(d[u][r], t, acc[r]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const float t = wave_sum(acc[r]);
        if (lane == 0) part[rg * RW + r][ks] = t;
    }
    if constexpr (PRO == PRO_NORM) {
        ss = wave_sum(ss);
        if (rg == 0 && lane == 0) pss[ks] = ss;
    }
    finish_rows<FMT, PRO, EPI, RG * RW, SK>(part, pss, s, rowBlock, b.N, K, b.eps);
}

// 4-bit split-nibble codes; requires K % 32 == 0. Lane l takes the 32-value
// block (step * 64 + l): 16 code bytes and 32 activations.
template <int RW, int SK, int WPB, int MAXB, int PRO = PRO_PLAIN, int EPI = EPI_STORE>
__global__ __launch_bounds__(64 * WPB) void gemv4_kernel(const GemvBatch<MAXB> b) {
    constexpr int RG = WPB / SK;
    __shared__ float part[RG * RW][SK];
    __shared__ float pss[SK];
    const GemvSet s = b.set[blockIdx.y];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int rg = wv / SK, ks = wv % SK;
    const int rowBlock = blockIdx.x * (RG * RW);
    const int row0 = rowBlock + rg * RW;
    const int K = b.K;
    const int steps = (K + SK * 2048 - 1) / (SK * 2048);
    const uint8_t *W = (const uint8_t *)s.codes;
    const size_t kb = (size_t)(K >> 5);
    const size_t rowBytes = (size_t)(K >> 1);
    int rows[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) rows[r] = min(row0 + r, b.N - 1);
    float acc[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) acc[r] = 0.0f;
    float ss = 0.0f;

    for (int st = 0; st < steps; ++st) {
        const int k0 = (ks * steps + st) * 2048 + lane * 32;
        const bool ok = k0 < K;
        float4 xs[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) xs[i] = ok ? *((const float4 *)(s.x + k0) + i) : make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (PRO == PRO_NORM) {
#pragma unroll
            for (int i = 0; i < 8; ++i) ss += xs[i].x * xs[i].x + xs[i].y * xs[i].y + xs[i].z * xs[i].z + xs[i].w * xs[i].w;
        }
        float d[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) d[r] = ok ? block_scale<GPHQ_FMT_Q4>(s.scales, (size_t)rows[r] * kb + (k0 >> 5)) : 0.0f;
        u32x4 w[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r)
            w[r] = ok ? __builtin_nontemporal_load((const u32x4 *)(W + (size_t)rows[r] * rowBytes + (k0 >> 1)))
                      : u32x4{0, 0, 0, 0};
        const float4 s4 = xs[0] + xs[1] + xs[2] + xs[3] + xs[4] + xs[5] + xs[6] + xs[7];
        const float sx = (s4.x + s4.y + s4.z + s4.w) * 8.0f;
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            const uint32_t ww[4] = {w[r].x, w[r].y, w[r].z, w[r].w};
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
            acc[r] = fmaf(d[r], (t.x + t.y + t.z + t.w) - sx, acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const float t = wave_sum(acc[r]);
        if (lane == 0) part[rg * RW + r][ks] = t;
    }
    if constexpr (PRO == PRO_NORM) {
        ss = wave_sum(ss);
        if (rg == 0 && lane == 0) pss[ks] = ss;
    }
    finish_rows<GPHQ_FMT_Q4, PRO, EPI, RG * RW, SK>(part, pss, s, rowBlock, b.N, K, b.eps);
}

// Any K, any alignment (Q8 only): one wavefront per row, lanes stride through
// the row one code at a time. Used for shapes the vector path cannot take.
__global__ __launch_bounds__(256) void gemv8_generic_kernel(const GemvBatch<1> b) {
    const GemvSet s = b.set[0];
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= b.N) return;
    const int8_t *w = (const int8_t *)s.codes + (size_t)row * b.K;
    float acc = 0.0f;
    for (int k = lane; k < b.K; k += 64) acc = fmaf(s.x[k], (float)w[k], acc);
    const float t = wave_sum(acc) * ((const float *)s.scales)[row];
    if (lane == 0) s.y[row] = t;
}

// Tile geometry (measured on MI355X at 4096x4096): 4 rows per wavefront,
// K split in 2 slices, 8 wavefronts per block = 16 rows per block.
constexpr int kRW = 4, kSK = 2, kWPB = 8;
constexpr int kRowsPerBlock = (kWPB / kSK) * kRW;
// Q4: 2 rows per wavefront (32 activations per lane per step), 4 slices.
constexpr int kRW4 = 2, kSK4 = 4, kWPB4 = 8;
constexpr int kRowsPerBlock4 = (kWPB4 / kSK4) * kRW4;

template <int MAXB>
static int launch_batch(int fmt, const GemvBatch<MAXB> &b, int count, hipStream_t stream) {
    const unsigned rowsPerBlock = fmt == GPHQ_FMT_Q4 ? kRowsPerBlock4 : kRowsPerBlock;
    const dim3 grid((unsigned)((b.N + rowsPerBlock - 1) / rowsPerBlock), (unsigned)count);
    switch (fmt) {
    case GPHQ_FMT_Q8:
        hipLaunchKernelGGL((gemv8_kernel<GPHQ_FMT_Q8, kRW, kSK, kWPB, MAXB>), grid, dim3(64 * kWPB), 0, stream, b);
        break;
    case GPHQ_FMT_Q8B:
        hipLaunchKernelGGL((gemv8_kernel<GPHQ_FMT_Q8B, kRW, kSK, kWPB, MAXB>), grid, dim3(64 * kWPB), 0, stream, b);
        break;
    case GPHQ_FMT_Q8B_F32:
        hipLaunchKernelGGL((gemv8_kernel<GPHQ_FMT_Q8B_F32, kRW, kSK, kWPB, MAXB>), grid, dim3(64 * kWPB), 0, stream,
                           b);
        break;
    case GPHQ_FMT_Q4:
        hipLaunchKernelGGL((gemv4_kernel<kRW4, kSK4, kWPB4, MAXB>), grid, dim3(64 * kWPB4), 0, stream, b);
        break;
    default:
        return GPHQ_ERR_UNSUPPORTED;
    }
    return launch_status();
}

// One GEMV. Arguments were validated by the caller.
int gemv_launch(int fmt, const void *codes, const void *scales, const float *x, float *y, int K, int N,
                hipStream_t stream) {
    if (N == 0) return GPHQ_OK;
    GemvBatch<1> b{};
    b.set[0] = GemvSet{codes, scales, x, y};
    b.K = K;
    b.N = N;
    if (fmt == GPHQ_FMT_Q8) {
        const bool vec = (K % 16 == 0) && ((uintptr_t)codes % 16 == 0) && ((uintptr_t)x % 16 == 0);
        if (!vec) {
            hipLaunchKernelGGL(gemv8_generic_kernel, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, stream, b);
            return launch_status();
        }
    }
    return launch_batch<1>(fmt, b, 1, stream);
}

// Up to kMaxBatch GEMVs of one shape and format in one launch.
int gemv_batch_launch(int fmt, const void *const *codes, const void *const *scales, const float *const *x,
                      float *const *y, int count, int K, int N, hipStream_t stream) {
    if (N == 0 || count == 0) return GPHQ_OK;
    GemvBatch<kMaxBatch> b{};
    for (int i = 0; i < count; ++i) b.set[i] = GemvSet{codes[i], scales[i], x[i], y[i]};
    b.K = K;
    b.N = N;
    return launch_batch<kMaxBatch>(fmt, b, count, stream);
}

// Tile shape of a decode-step GEMV, chosen from the matrix shape (measured
// on MI355X with rotated weights over 256 MB, one launch per GEMV):
// very tall matrices (the head) take 16-row blocks of four unsplit
// wavefronts; tall ones (gate/up) 16-row blocks with K in two slices; long
// rows (down) 8-row blocks with K in four slices and two steps in flight;
// short, wide-K matrices 4-row blocks with K in four slices (2-row blocks of
// one row per wavefront up to 2048 rows: Qwen3-0.6B's o and down); the rest
// (qkv) 8-row blocks with K in two slices.
template <int FMT, int PRO, int EPI>
static void launch_fused8(const GemvBatch<1> &b, hipStream_t stream) {
    auto go = [&](auto kern, int rows, int threads) {
        hipLaunchKernelGGL(kern, dim3((unsigned)((b.N + rows - 1) / rows)), dim3(threads), 0, stream, b);
    };
    if (b.N >= 65536)
        go(gemv8_kernel<FMT, 4, 1, 4, 1, PRO, EPI, 1>, 16, 256);
    else if (b.N >= 16384)
        go(gemv8_kernel<FMT, 4, 2, 8, 1, PRO, EPI, 1>, 16, 512);
    else if (b.K >= 8192)
        go(gemv8_kernel<FMT, 4, 4, 8, 1, PRO, EPI, 2>, 8, 512);
    else if (b.N <= 2048 && b.K >= 2048)
        go(gemv8_kernel<FMT, 1, 4, 8, 1, PRO, EPI, 1>, 2, 512);
    else if (b.N <= 4096 && b.K >= 2048)
        go(gemv8_kernel<FMT, 2, 4, 8, 1, PRO, EPI, 1>, 4, 512);
    else
        go(gemv8_kernel<FMT, 2, 2, 8, 1, PRO, EPI, 1>, 8, 512);
}

template <int PRO, int EPI>
static int launch_fused(int fmt, const GemvBatch<1> &b, hipStream_t stream) {
    switch (fmt) {
    case GPHQ_FMT_Q8: launch_fused8<GPHQ_FMT_Q8, PRO, EPI>(b, stream); break;
    case GPHQ_FMT_Q8B: launch_fused8<GPHQ_FMT_Q8B, PRO, EPI>(b, stream); break;
    case GPHQ_FMT_Q8B_F32: launch_fused8<GPHQ_FMT_Q8B_F32, PRO, EPI>(b, stream); break;
    case GPHQ_FMT_Q4: {
        const dim3 grid((unsigned)((b.N + kRowsPerBlock4 - 1) / kRowsPerBlock4));
        hipLaunchKernelGGL((gemv4_kernel<kRW4, kSK4, kWPB4, 1, PRO, EPI>), grid, dim3(64 * kWPB4), 0, stream, b);
        break;
    }
    default:
        return GPHQ_ERR_UNSUPPORTED;
    }
    return launch_status();
}

// One decode-step GEMV with a fused prologue/epilogue (pro: PRO_*, epi:
// EPI_*). K % 32 == 0, codes and x 16-byte aligned; for EPI_SWIGLU N is even
// and y receives N/2 values. Arguments were validated by the caller.
int gemv_fused_launch(int fmt, int pro, int epi, const void *codes, const void *scales, const float *x, float *y,
                      int K, int N, float eps, hipStream_t stream) {
    if (N == 0) return GPHQ_OK;
    GemvBatch<1> b{};
    b.set[0] = GemvSet{codes, scales, x, y};
    b.K = K;
    b.N = N;
    b.eps = eps;
    if (pro == PRO_PLAIN && epi == EPI_STORE) return launch_fused<PRO_PLAIN, EPI_STORE>(fmt, b, stream);
    if (pro == PRO_NORM && epi == EPI_STORE) return launch_fused<PRO_NORM, EPI_STORE>(fmt, b, stream);
    if (pro == PRO_PLAIN && epi == EPI_ADD) return launch_fused<PRO_PLAIN, EPI_ADD>(fmt, b, stream);
    if (pro == PRO_NORM && epi == EPI_SWIGLU) return launch_fused<PRO_NORM, EPI_SWIGLU>(fmt, b, stream);
    return GPHQ_ERR_UNSUPPORTED;
}

}  // namespace gphq
