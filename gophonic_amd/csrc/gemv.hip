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
#include <type_traits>

#include "common.h"

namespace gphq {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

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
// as four 4-wide dot products summed (gpu.metal:91-92). Written as explicit
// fmaf chains so every kernel that inlines it rounds the same way (left to
// contraction, the compiler may fuse differently in different kernels, and
// the batch and single-GEMV paths must agree bit for bit).
__device__ __forceinline__ float dot4(uint32_t w, const float4 x) {
    return fmaf(sext_byte_f(w, 3), x.w, fmaf(sext_byte_f(w, 2), x.z, fmaf(sext_byte_f(w, 1), x.y, sext_byte_f(w, 0) * x.x)));
}
__device__ __forceinline__ float dot16(const u32x4 w, const float4 x0, const float4 x1, const float4 x2,
                                       const float4 x3) {
    return ((dot4(w.x, x0) + dot4(w.y, x1)) + dot4(w.z, x2)) + dot4(w.w, x3);
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

// The prologue's norm factor, the Q8 row scale and the epilogue for RW row
// totals t of rows row0.. (one thread).
template <int FMT, int PRO, int EPI, int RW>
__device__ __forceinline__ void finish_group(const GemvSet &s, const float *t, int row0, int N, float inv) {
    if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
        for (int r = 0; r < RW; r += 2) {
            const int row = row0 + r;
            if (row + 1 < N) {
                float g = t[r] * inv, u = t[r + 1] * inv;
                if constexpr (FMT == GPHQ_FMT_Q8) {
                    g = g * ((const float *)s.scales)[row];
                    u = u * ((const float *)s.scales)[row + 1];
                }
                s.y[row >> 1] = g / (1.0f + expf(-g)) * u;
            }
        }
    } else {
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            const int row = row0 + r;
            if (row < N) {
                float v = t[r] * inv;
                if constexpr (FMT == GPHQ_FMT_Q8) v = v * ((const float *)s.scales)[row];
                if constexpr (EPI == EPI_ADD)
                    s.y[row] += v;
                else
                    s.y[row] = v;
            }
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

// Persistent GEMV for the 8-bit formats when K is a multiple of 1024.
//
// A block holds WPB wavefronts: WPB/SK wave groups of SK wavefronts, one per
// K slice of NS*1024 values. Each wavefront loads its slice of x into
// registers once (NS*16 floats per lane) and then walks row groups of RW
// rows: per group it issues NS*RW 128-bit non-temporal weight loads (lane l
// takes bytes [16l, 16l+16) of each 1 KiB step of each row, so one
// wavefront instruction is 1 KiB of one row), scales each 16-value dot
// product by its block scale, and reduces each row across the wavefront
// with DPP. SK > 1 slices meet in LDS (two buffers, one barrier per group)
// and are added in slice order, so results do not depend on the grid.
// The grid is a few blocks per CU; a single GEMV strides its row groups over
// the whole grid (the waves of the GPU stream neighbouring rows), a batch of
// GEMVs gives each wave group a contiguous run of row groups so x is
// reloaded only where the run crosses into the next GEMV. Measured on
// MI355X against the block-per-row-tile kernel above: the Qwen3-8B head
// 661 MB at 6.6-6.8 TB/s (was 5.2), gate/up 20.5 us (was 26.2), down 14 us
// (was 17.2), qkv 7.1 us (was 9.4) per launch.
template <int FMT, int NS, int RW, int SK, int WPB, int PRO, int EPI, int MAXB>
__global__ __launch_bounds__(64 * WPB) void gemvp_kernel(const GemvBatch<MAXB> b, int count, int iters) {
    static_assert(WPB % SK == 0, "wave groups of SK waves");
    static_assert(EPI != EPI_SWIGLU || RW % 2 == 0, "gate and up rows pair within a group");
    static_assert(PRO == PRO_PLAIN || MAXB == 1, "the norm prologue is for single GEMVs");
    constexpr int WG = WPB / SK;
    __shared__ float part[2][WG][RW][SK];
    __shared__ float pss[WG][SK];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wg = wv / SK, ks = wv - wg * SK;
    const int K = b.K, N = b.N;
    const int kbase = ks * (NS * 1024) + lane * 16;
    const size_t kb = (size_t)(K >> 5);
    const int gps = (N + RW - 1) / RW;  // row groups per GEMV
    const int total = gps * count;
    const int wgid = blockIdx.x * WG + wg;
    int g = MAXB == 1 ? wgid : wgid * iters;
    const int gstep = MAXB == 1 ? (int)gridDim.x * WG : 1;
    int set = MAXB == 1 ? 0 : min(g / gps, count - 1);
    float4 xr[NS][4];
    auto load_x = [&](const float *x) {
#pragma unroll
        for (int j = 0; j < NS; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) xr[j][i] = *((const float4 *)(x + kbase + j * 1024) + i);
    };
    load_x(b.set[set].x);
    float inv = 1.0f;
    if constexpr (PRO == PRO_NORM) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < NS; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                ss += xr[j][i].x * xr[j][i].x + xr[j][i].y * xr[j][i].y + xr[j][i].z * xr[j][i].z +
                      xr[j][i].w * xr[j][i].w;
        ss = wave_sum(ss);
        if constexpr (SK > 1) {
            if (lane == 0) pss[wg][ks] = ss;
            __syncthreads();
            ss = pss[wg][0];
#pragma unroll
            for (int i = 1; i < SK; ++i) ss += pss[wg][i];
        }
        inv = 1.0f / sqrtf(ss / (float)K + b.eps);
    }
    for (int it = 0; it < iters; ++it, g += gstep) {
        const bool valid = g < total;
        if constexpr (SK == 1) {
            if (!valid) break;
        }
        int lg = g;
        if constexpr (MAXB > 1) {
            if (valid) {
                const int s2 = g / gps;
                if (s2 != set) {
                    set = s2;
                    load_x(b.set[set].x);
                }
                lg = g - set * gps;
            }
        }
        const GemvSet &s = b.set[set];
        const int8_t *W = (const int8_t *)s.codes;
        const int row0 = lg * RW;
        float acc[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) acc[r] = 0.0f;
        if (valid) {
            u32x4 w[NS][RW];
            float d[NS][RW];
            if constexpr (FMT != GPHQ_FMT_Q8) {
#pragma unroll
                for (int j = 0; j < NS; ++j)
#pragma unroll
                    for (int r = 0; r < RW; ++r)
                        d[j][r] = block_scale<FMT>(s.scales,
                                                   (size_t)min(row0 + r, N - 1) * kb + ((kbase + j * 1024) >> 5));
            }
#pragma unroll
            for (int j = 0; j < NS; ++j)
#pragma unroll
                for (int r = 0; r < RW; ++r)
                    w[j][r] = __builtin_nontemporal_load(
                        (const u32x4 *)(W + (size_t)min(row0 + r, N - 1) * K + kbase + j * 1024));
#pragma unroll
            for (int j = 0; j < NS; ++j)
#pragma unroll
                for (int r = 0; r < RW; ++r) {
                    const float t = dot16(w[j][r], xr[j][0], xr[j][1], xr[j][2], xr[j][3]);
                    if constexpr (FMT == GPHQ_FMT_Q8)
                        acc[r] += t;
                    else
                        acc[r] = fmaf(d[j][r], t, acc[r]);
                }
        }
        float t[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) t[r] = wave_sum(acc[r]);
        if constexpr (SK == 1) {
            if (lane == 0) finish_group<FMT, PRO, EPI, RW>(s, t, row0, N, inv);
        } else {
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < RW; ++r) part[it & 1][wg][r][ks] = t[r];
            }
            __syncthreads();
            if (ks == 0 && lane == 0 && valid) {
#pragma unroll
                for (int r = 0; r < RW; ++r) {
                    float v = part[it & 1][wg][r][0];
#pragma unroll
                    for (int i = 1; i < SK; ++i) v += part[it & 1][wg][r][i];
                    t[r] = v;
                }
                finish_group<FMT, PRO, EPI, RW>(s, t, row0, N, inv);
            }
        }
    }
}

// Batch GEMV (gphq_gemv_batch, 8-bit formats, K = NS * 1024 up to 4096): a
// wavefront holds all of x (NS KiB steps) in registers and walks row groups
// of RW rows (set by set), with the next group's codes and block scales
// requested before the current group's arithmetic (two register buffers); no
// LDS and no barriers. A block owns a contiguous run of WPB * per groups and
// its wavefronts take them in turn (wavefront i: groups i, i + WPB, ...), so
// the block's loads in flight cover one contiguous stretch of the weights.
// Each row's sum is formed as the persistent kernel forms it for the same K:
// SL slices of NS/SL steps, each accumulated in step order and reduced
// across the wavefront, then added in slice order, so a batch launch gives
// the same bits as single launches. Measured on MI355X at config 1 (32 sets
// of 4096 x 4096 Q8B_F32, 605 MB): 88.1-88.5 us per launch with 4-wavefront
// blocks, 8 per CU, against 90.5-91 us when each wavefront walked its own
// contiguous run (8-wavefront blocks, 3 per CU) and 100-103 us for the
// persistent kernel with LDS slice merges.
template <int FMT, int NS, int SL, int RW, int WPB>
__global__ __launch_bounds__(64 * WPB) void gemvb_kernel(const GemvBatch<kMaxBatch> b, int count, int per) {
    static_assert(NS % SL == 0, "slices of whole steps");
    constexpr int K = NS * 1024, SS = NS / SL;
    constexpr size_t kb = K >> 5;
    const int lane = threadIdx.x & 63;
    const int N = b.N;
    const int gps = (N + RW - 1) / RW;
    const int total = gps * count;
    const int base = blockIdx.x * WPB * per;
    int g = base + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int gend = min(base + WPB * per, total);
    if (g >= gend) return;
    float4 xr[NS][4];
    u32x4 w[2][NS][RW];
    float d[2][NS][RW];
    auto issue = [&](int gg, auto bufc) {
        constexpr int buf = decltype(bufc)::value;
        const int set = gg / gps, lg = gg - set * gps;
        const GemvSet &s = b.set[set];
        const int row0 = lg * RW;
        const int8_t *W = (const int8_t *)s.codes;
        if constexpr (FMT != GPHQ_FMT_Q8) {
#pragma unroll
            for (int j = 0; j < NS; ++j)
#pragma unroll
                for (int r = 0; r < RW; ++r)
                    d[buf][j][r] = block_scale<FMT>(s.scales, (size_t)min(row0 + r, N - 1) * kb + j * 32 + (lane >> 1));
        }
#pragma unroll
        for (int j = 0; j < NS; ++j)
#pragma unroll
            for (int r = 0; r < RW; ++r)
                w[buf][j][r] = __builtin_nontemporal_load(
                    (const u32x4 *)(W + (size_t)min(row0 + r, N - 1) * K + j * 1024 + lane * 16));
    };
    auto load_x = [&](int set) {
        const float *x = b.set[set].x;
#pragma unroll
        for (int j = 0; j < NS; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) xr[j][i] = *((const float4 *)(x + j * 1024 + lane * 16) + i);
    };
    auto compute = [&](int gg, auto bufc) {
        constexpr int buf = decltype(bufc)::value;
        const int set = gg / gps, lg = gg - set * gps;
        float t[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) t[r] = 0.0f;
#pragma unroll
        for (int sl = 0; sl < SL; ++sl) {
            float acc[RW];
#pragma unroll
            for (int r = 0; r < RW; ++r) acc[r] = 0.0f;
#pragma unroll
            for (int jj = 0; jj < SS; ++jj) {
                const int j = sl * SS + jj;
#pragma unroll
                for (int r = 0; r < RW; ++r) {
                    const float v = dot16(w[buf][j][r], xr[j][0], xr[j][1], xr[j][2], xr[j][3]);
                    if constexpr (FMT == GPHQ_FMT_Q8)
                        acc[r] += v;
                    else
                        acc[r] = fmaf(d[buf][j][r], v, acc[r]);
                }
            }
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                const float ws = wave_sum(acc[r]);
                t[r] = sl == 0 ? ws : t[r] + ws;
            }
        }
        if (lane == 0) finish_group<FMT, PRO_PLAIN, EPI_STORE, RW>(b.set[set], t, lg * RW, N, 1.0f);
    };
    int cur = g / gps;
    load_x(cur);
    issue(g, std::integral_constant<int, 0>{});
    for (; g < gend; g += 2 * WPB) {
        if (g + WPB < gend) issue(g + WPB, std::integral_constant<int, 1>{});
        if (g / gps != cur) {
            cur = g / gps;
            load_x(cur);
        }
        compute(g, std::integral_constant<int, 0>{});
        if (g + WPB >= gend) break;
        if (g + 2 * WPB < gend) issue(g + 2 * WPB, std::integral_constant<int, 0>{});
        if ((g + WPB) / gps != cur) {
            cur = (g + WPB) / gps;
            load_x(cur);
        }
        compute(g + WPB, std::integral_constant<int, 1>{});
    }
}

// GPTQ int4 GEMV (GPHQ_FMT_GPTQ4_G128 at one activation row): codes int32
// [N][K/8] (nibble i of word j is k = 8j + i), FP16 scales [N][K/128], 4-bit
// zero points u8 [N][K/128]; y[n] = sum_g s_g * sum_{k in g} (q - z_g) *
// half(x[k]), fp32 arithmetic, weights not rounded (the mm path rounds each
// dequantized weight to FP16 first; this path is within 1e-4 relative of the
// float64 value with un-rounded weights, the mm path within about 2^-11).
//
// Persistent like gemvp_kernel: a wavefront holds its K slice of half(x) in
// registers (NS steps of 2048 values; lane l takes values 32l..32l+31 of a
// step, one 16-byte load of codes) and walks row groups. Per code word the
// low and high nibbles of its bytes are masked out and placed under the FP16
// exponent of 1024 by v_perm_b32, giving pairs (1024 + q), and
// v_dot2_f32_f16 adds their products with the matching half(x) pairs in fp32
// (exact products). Per 128-value group (four lanes) the lane's part is
// s * (dot - (1024 + z) * sum(half(x))), which removes the bias and the zero
// point in one step: about one VALU operation per weight.
template <int NS, int RW, int SK, int WPB>
__global__ __launch_bounds__(64 * WPB) void gemv_gptq_kernel(const uint32_t *__restrict__ codes,
                                                             const uint16_t *__restrict__ scales,
                                                             const uint8_t *__restrict__ zeros,
                                                             const float *__restrict__ x, float *__restrict__ y, int K,
                                                             int N, int iters) {
    static_assert(WPB % SK == 0, "wave groups of SK waves");
    constexpr int WG = WPB / SK;
    __shared__ float part[2][WG][RW][SK];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wg = wv / SK, ks = wv - wg * SK;
    const int kbase = ks * (NS * 2048) + lane * 32;
    const int KG = K >> 7;  // groups per row
    // half(x) pairs in the nibble order of one code word: (x0,x2), (x4,x6), (x1,x3), (x5,x7).
    f16x2 xh[NS][4][4];
    float sx[NS];
#pragma unroll
    for (int st = 0; st < NS; ++st) {
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float4 a = *(const float4 *)(x + kbase + st * 2048 + w * 8);
            const float4 b = *(const float4 *)(x + kbase + st * 2048 + w * 8 + 4);
            const _Float16 h[8] = {(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w,
                                   (_Float16)b.x, (_Float16)b.y, (_Float16)b.z, (_Float16)b.w};
            xh[st][w][0] = f16x2{h[0], h[2]};
            xh[st][w][1] = f16x2{h[4], h[6]};
            xh[st][w][2] = f16x2{h[1], h[3]};
            xh[st][w][3] = f16x2{h[5], h[7]};
#pragma unroll
            for (int i = 0; i < 8; ++i) sum += (float)h[i];
        }
        sx[st] = sum;
    }
    const int groups = (N + RW - 1) / RW;
    const int stride = gridDim.x * WG;
    int g = blockIdx.x * WG + wg;
    for (int it = 0; it < iters; ++it, g += stride) {
        const bool valid = g < groups;
        if constexpr (SK == 1) {
            if (!valid) break;
        }
        const int row0 = g * RW;
        float acc[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) acc[r] = 0.0f;
        if (valid) {
            u32x4 w[NS][RW];
            uint16_t sc[NS][RW];
            uint8_t zp[NS][RW];
#pragma unroll
            for (int st = 0; st < NS; ++st)
#pragma unroll
                for (int r = 0; r < RW; ++r) {
                    const size_t row = (size_t)min(row0 + r, N - 1);
                    const int gi = (kbase + st * 2048) >> 7;
                    sc[st][r] = scales[row * KG + gi];
                    zp[st][r] = zeros[row * KG + gi];
                    w[st][r] = __builtin_nontemporal_load(
                        (const u32x4 *)(codes + row * (size_t)(K >> 3) + ((kbase + st * 2048) >> 3)));
                }
#pragma unroll
            for (int st = 0; st < NS; ++st)
#pragma unroll
                for (int r = 0; r < RW; ++r) {
                    const uint32_t ww[4] = {w[st][r].x, w[st][r].y, w[st][r].z, w[st][r].w};
                    float dot = 0.0f;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t lo = ww[q] & 0x0F0F0F0Fu, hi = (ww[q] >> 4) & 0x0F0F0F0Fu;
                        const f16x2 p0 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u));
                        const f16x2 p1 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u));
                        const f16x2 p2 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u));
                        const f16x2 p3 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u));
                        dot = __builtin_amdgcn_fdot2(p0, xh[st][q][0], dot, false);
                        dot = __builtin_amdgcn_fdot2(p1, xh[st][q][1], dot, false);
                        dot = __builtin_amdgcn_fdot2(p2, xh[st][q][2], dot, false);
                        dot = __builtin_amdgcn_fdot2(p3, xh[st][q][3], dot, false);
                    }
                    const float sg = half_bits_to_float(sc[st][r]);
                    const float zb = 1024.0f + (float)(zp[st][r] & 15);
                    acc[r] = fmaf(sg, fmaf(-zb, sx[st], dot), acc[r]);
                }
        }
        float t[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) t[r] = wave_sum(acc[r]);
        if constexpr (SK == 1) {
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < RW; ++r)
                    if (row0 + r < N) y[row0 + r] = t[r];
            }
        } else {
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < RW; ++r) part[it & 1][wg][r][ks] = t[r];
            }
            __syncthreads();
            if (ks == 0 && lane == 0 && valid) {
#pragma unroll
                for (int r = 0; r < RW; ++r) {
                    float v = part[it & 1][wg][r][0];
#pragma unroll
                    for (int i = 1; i < SK; ++i) v += part[it & 1][wg][r][i];
                    if (row0 + r < N) y[row0 + r] = v;
                }
            }
        }
    }
}

template <int NS, int RW, int SK, int WPB>
static int go_gptq(const uint32_t *codes, const uint16_t *scales, const uint8_t *zeros, const float *x, float *y,
                   int K, int N, int bpc, hipStream_t stream) {
    constexpr int WG = WPB / SK;
    const long groups = (N + RW - 1) / RW;
    const long blocks = std::max(1L, std::min((groups + WG - 1) / WG, (long)device_cus() * bpc));
    const int iters = (int)((groups + blocks * WG - 1) / (blocks * WG));
    hipLaunchKernelGGL((gemv_gptq_kernel<NS, RW, SK, WPB>), dim3((unsigned)blocks), dim3(64 * WPB), 0, stream, codes,
                       scales, zeros, x, y, K, N, iters);
    return launch_status();
}

// One GPTQ4_G128 row (gphq_mm with m = 1) when K is a multiple of 2048 up to
// 16 * 2048 and x is 16-byte aligned; GPHQ_ERR_UNSUPPORTED otherwise (the
// caller then uses the mm kernel).
int gemv_gptq_launch(const void *codes, const void *scales, const uint8_t *zeros, const float *x, float *y, int K,
                     int N, hipStream_t stream) {
    if (K % 2048 || (uintptr_t)x % 16) return GPHQ_ERR_UNSUPPORTED;
    const uint32_t *c = (const uint32_t *)codes;
    const uint16_t *s = (const uint16_t *)scales;
    // Launch shapes from sweeps on MI355X at the config-5 shapes (K = 4096 ->
    // N = 12288: 9.8 -> 9.0 us with 4-wavefront blocks; K = 12288 -> N = 4096:
    // 10.8 -> 9.5 us with 8 rows per wavefront group, one group per block).
    // Issuing the next row group's loads before the current one is reduced
    // measured slower at both.
    switch (K / 2048) {
    case 1: return go_gptq<1, 4, 1, 4>(c, s, zeros, x, y, K, N, 2, stream);
    case 2: return go_gptq<1, 4, 2, 4>(c, s, zeros, x, y, K, N, 2, stream);
    case 3: return go_gptq<1, 2, 3, 6>(c, s, zeros, x, y, K, N, 2, stream);
    case 4: return go_gptq<1, 2, 4, 8>(c, s, zeros, x, y, K, N, 1, stream);
    case 6: return go_gptq<1, 8, 6, 6>(c, s, zeros, x, y, K, N, 1, stream);
    case 8: return go_gptq<1, 2, 8, 16>(c, s, zeros, x, y, K, N, 1, stream);
    }
    return GPHQ_ERR_UNSUPPORTED;
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

// Launch shape of the persistent kernel: NS K steps of 1024 per wavefront,
// RW rows per group, SK slices, WPB wavefronts per block, BPC blocks per CU.
struct PersistentShape {
    int ns, rw, sk, wpb, bpc;
};

// Shapes measured on MI355X (Q8B rows, one launch per GEMV in a HIP graph,
// weights rotating through more than 256 MB): Qwen3-8B head / gate-up / qkv
// / o / down and Qwen3-0.6B head / qkv / gate-up / o / down. A batch of
// GEMVs (config 1: 32 of 4096 x 4096) takes its own shape. False when K is
// not a multiple of 1024 or the slices do not fit 16 wavefronts.
static bool persistent_shape(int K, int N, bool batch, PersistentShape &p) {
    if (K % 1024) return false;
    switch (K / 1024) {
    case 1: p = {1, 2, 1, 4, 4}; return true;
    case 2: p = {2, 2, 1, 4, 2}; return true;
    case 3: p = N > 4096 ? PersistentShape{3, 2, 1, 4, 2} : PersistentShape{1, 2, 3, 6, 4}; return true;
    case 4:
        if (batch)
            p = {2, 4, 2, 4, 2};
        else
            p = N >= 16384 ? PersistentShape{2, 2, 2, 8, 2}
                : N > 4096 ? PersistentShape{1, 4, 4, 8, 4} : PersistentShape{2, 4, 2, 8, 6};
        return true;
    case 6: case 8: case 12: case 16: p = {2, 2, K / 2048, K / 1024, 2}; return true;
    }
    return false;
}

template <int FMT, int NS, int RW, int SK, int WPB, int PRO, int EPI, int MAXB>
static int go_persistent(const GemvBatch<MAXB> &b, int count, int bpc, hipStream_t stream) {
    constexpr int WG = WPB / SK;
    const long total = (long)((b.N + RW - 1) / RW) * count;
    const long blocks = std::max(1L, std::min((total + WG - 1) / WG, (long)device_cus() * bpc));
    const int iters = (int)((total + blocks * WG - 1) / (blocks * WG));
    hipLaunchKernelGGL((gemvp_kernel<FMT, NS, RW, SK, WPB, PRO, EPI, MAXB>), dim3((unsigned)blocks), dim3(64 * WPB), 0,
                       stream, b, count, iters);
    return launch_status();
}

template <int FMT, int PRO, int EPI, int MAXB>
static int launch_persistent(const GemvBatch<MAXB> &b, int count, const PersistentShape &p, hipStream_t stream) {
#define GPHQ_PERSISTENT(NS, RW, SK, WPB)                                   \
    if (p.ns == NS && p.rw == RW && p.sk == SK && p.wpb == WPB)            \
        return go_persistent<FMT, NS, RW, SK, WPB, PRO, EPI, MAXB>(b, count, p.bpc, stream);
    if constexpr (MAXB > 1) {
        GPHQ_PERSISTENT(2, 4, 2, 4)
    }
    GPHQ_PERSISTENT(1, 2, 1, 4) GPHQ_PERSISTENT(2, 2, 1, 4) GPHQ_PERSISTENT(3, 2, 1, 4)
    GPHQ_PERSISTENT(1, 2, 3, 6) GPHQ_PERSISTENT(2, 2, 2, 8) GPHQ_PERSISTENT(1, 4, 4, 8) GPHQ_PERSISTENT(2, 4, 2, 8)
    GPHQ_PERSISTENT(2, 2, 3, 6) GPHQ_PERSISTENT(2, 2, 4, 8) GPHQ_PERSISTENT(2, 2, 6, 12) GPHQ_PERSISTENT(2, 2, 8, 16)
#undef GPHQ_PERSISTENT
    return GPHQ_ERR_UNSUPPORTED;
}

// The persistent path for one format, or GPHQ_ERR_UNSUPPORTED when the shape
// is not one it takes (the caller then uses the per-tile kernel).
// The batch kernel for K = 1024 .. 4096 (slices as persistent_shape's batch
// shape for that K): RW = 2 rows per group, 4 wavefronts per block, 8 blocks
// per CU (measured at config 1). The kernel's registers allow 3 wavefronts
// per SIMD, so 3 blocks of a CU are resident at once and the rest start as
// blocks finish.
template <int FMT, int NS, int SL>
static int go_batch(const GemvBatch<kMaxBatch> &b, int count, hipStream_t stream) {
    constexpr int RW = 2, WPB = 4, BPC = 8;
    const long total = (long)((b.N + RW - 1) / RW) * count;
    const long blocks = std::max(1L, std::min((total + WPB - 1) / WPB, (long)device_cus() * BPC));
    const int per = (int)((total + blocks * WPB - 1) / (blocks * WPB));
    hipLaunchKernelGGL((gemvb_kernel<FMT, NS, SL, RW, WPB>), dim3((unsigned)blocks), dim3(64 * WPB), 0, stream, b,
                       count, per);
    return launch_status();
}

template <int FMT>
static int launch_batch_b(const GemvBatch<kMaxBatch> &b, int count, hipStream_t stream) {
    switch (b.K) {
    case 1024: return go_batch<FMT, 1, 1>(b, count, stream);
    case 2048: return go_batch<FMT, 2, 1>(b, count, stream);
    case 3072: return b.N > 4096 ? go_batch<FMT, 3, 1>(b, count, stream) : go_batch<FMT, 3, 3>(b, count, stream);
    case 4096: return go_batch<FMT, 4, 2>(b, count, stream);
    }
    return GPHQ_ERR_UNSUPPORTED;
}

template <int PRO, int EPI, int MAXB>
static int try_persistent(int fmt, const GemvBatch<MAXB> &b, int count, hipStream_t stream) {
    if constexpr (MAXB > 1 && PRO == PRO_PLAIN && EPI == EPI_STORE) {
        int st = GPHQ_ERR_UNSUPPORTED;
        switch (fmt) {
        case GPHQ_FMT_Q8: st = launch_batch_b<GPHQ_FMT_Q8>(b, count, stream); break;
        case GPHQ_FMT_Q8B: st = launch_batch_b<GPHQ_FMT_Q8B>(b, count, stream); break;
        case GPHQ_FMT_Q8B_F32: st = launch_batch_b<GPHQ_FMT_Q8B_F32>(b, count, stream); break;
        }
        if (st != GPHQ_ERR_UNSUPPORTED) return st;
    }
    PersistentShape p;
    if (!persistent_shape(b.K, b.N, MAXB > 1, p)) return GPHQ_ERR_UNSUPPORTED;
    switch (fmt) {
    case GPHQ_FMT_Q8: return launch_persistent<GPHQ_FMT_Q8, PRO, EPI, MAXB>(b, count, p, stream);
    case GPHQ_FMT_Q8B: return launch_persistent<GPHQ_FMT_Q8B, PRO, EPI, MAXB>(b, count, p, stream);
    case GPHQ_FMT_Q8B_F32: return launch_persistent<GPHQ_FMT_Q8B_F32, PRO, EPI, MAXB>(b, count, p, stream);
    }
    return GPHQ_ERR_UNSUPPORTED;
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
    const int st = try_persistent<PRO_PLAIN, EPI_STORE, 1>(fmt, b, 1, stream);
    if (st != GPHQ_ERR_UNSUPPORTED) return st;
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
    const int st = try_persistent<PRO_PLAIN, EPI_STORE, kMaxBatch>(fmt, b, count, stream);
    if (st != GPHQ_ERR_UNSUPPORTED) return st;
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
    const int st = try_persistent<PRO, EPI, 1>(fmt, b, 1, stream);
    if (st != GPHQ_ERR_UNSUPPORTED) return st;
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
