// Multi-vector GEMV: y[v] = dequant(W) . x[v] for V input vectors that share
// one read of the weights (qwen3lm gemvQ8BVector<V>, gpu.metal:239-314, the
// decode-lane kernels of gpu_darwin.go:1121-1281), for any V up to
// kMaxVecLanes and the Q8, Q8B, Q8B_F32 and Q4 formats.
//
// Design: with fp32 VALU arithmetic every extra vector costs one FMA per
// weight, so 16 lanes would be VALU-bound. Here the vectors go through MFMA:
//   * vec_prep_kernel scales each vector by an exact power of two 2^e (its
//     max into [2^14, 2^15)) and splits it into FP16 hi + lo parts
//     (x*2^e = hi + lo + r, |r| <= 2^-22 |x*2^e|), laid out as MFMA A
//     fragments: rows 2v (hi) and 2v+1 (lo), per 32-value block.
//   * gemv_vec_kernel widens each 32-value block of 16 weight rows to FP16
//     (int8 and 4-bit codes are exact in FP16), runs one
//     v_mfma_f32_16x16x32_f16 per 16 A rows (products exact in fp32), and
//     folds the block result into fp32 accumulators with the block scale:
//     acc = fma(d, C, acc), the per-block scaling of the qwen3lm kernels.
//   * K is split over wavefronts; partial sums meet in LDS in slice order;
//     y[v][n] = (acc_hi + acc_lo) * 2^-e_v (Q8: times the row scale).
// VALU work per weight no longer grows with V.
//
// Decode-step forms (gemv_vec_fused_launch): with norm set, the prep pass
// also sums x^2 and folds 1/sqrt(mean(x^2) + eps) into the vector's output
// scale (PRO_NORM, gpu.metal:251-261); the epilogue stores, adds into y
// (EPI_ADD) or pairs interleaved gate/up rows into g/(1+exp(-g))*u
// (EPI_SWIGLU, gpu.metal:284-290), as gemvQ8BVector does per vector.
#include "common.h"

namespace gphq {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kMaxVecLanes = 32;

// A fragments for block kb of M-tile t: 1 KiB = 64 lanes x 8 FP16; lane l
// holds A row t*16 + l%16, values kb*32 + (l/16)*8 .. +8.
__host__ __device__ inline size_t vec_a_offset(int t, int kb, int KB, int lane) {
    return ((size_t)t * KB + kb) * 512 + (size_t)lane * 8;
}

// One block per vector: power-of-two scale, hi/lo split, A-fragment layout.
// With norm, inv also carries 1/sqrt(mean(x^2) + eps).
__global__ __launch_bounds__(256) void vec_prep_kernel(const float *__restrict__ x, long stride, int V, int K, int KB,
                                                       _Float16 *__restrict__ A, float *__restrict__ inv, int norm,
                                                       float eps) {
    __shared__ float smax[4];
    __shared__ int snan[4];
    __shared__ float sss[4];
    const int v = blockIdx.x;
    const float *xv = x + (size_t)v * stride;
    float m = 0.0f, ss = 0.0f;
    int nan = 0;
    constexpr int UNR = 8;
    for (int k0 = 0; k0 < K; k0 += 256 * UNR) {
        float t[UNR];
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int k = k0 + u * 256 + (int)threadIdx.x;
            t[u] = k < K ? xv[k] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            nan |= (t[u] != t[u]);
            m = fmaxf(m, fabsf(t[u]));
            ss += t[u] * t[u];
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        m = fmaxf(m, __shfl_xor(m, off));
        nan |= __shfl_xor(nan, off);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) {
        smax[threadIdx.x >> 6] = m;
        snan[threadIdx.x >> 6] = nan;
        sss[threadIdx.x >> 6] = ss;
    }
    __syncthreads();
    float mm = 0.0f;
    int anyNan = 0;
    for (int i = 0; i < 4; ++i) {
        mm = fmaxf(mm, smax[i]);
        anyNan |= snan[i];
    }
    int e = 0;
    if (!anyNan && mm > 0.0f && !isinf(mm)) {
        int ex;
        (void)frexpf(mm, &ex);
        e = min(max(15 - ex, -100), 100);
    }
    const float s = ldexpf(1.0f, e);
    if (threadIdx.x == 0) {
        float f = ldexpf(1.0f, -e);
        if (norm) f = f / sqrtf(((sss[0] + sss[1]) + (sss[2] + sss[3])) / (float)K + eps);
        inv[v] = f;
    }
    // Each thread writes one 8-value chunk of row 2v (hi) and of row 2v+1 (lo).
    const int rowHi = 2 * v, rowLo = 2 * v + 1;
    for (int c = threadIdx.x; c < KB * 4; c += blockDim.x) {
        const int kb = c >> 2, g = c & 3;
        f16x8 hi, lo;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int k = kb * 32 + g * 8 + i;
            const float xs = k < K ? __fmul_rn(xv[k], s) : 0.0f;
            const _Float16 h = (_Float16)xs;
            hi[i] = h;
            lo[i] = (_Float16)(xs - (float)h);
        }
        *(f16x8 *)(A + vec_a_offset(rowHi >> 4, kb, KB, g * 16 + (rowHi & 15))) = hi;
        *(f16x8 *)(A + vec_a_offset(rowLo >> 4, kb, KB, g * 16 + (rowLo & 15))) = lo;
    }
}

struct VecArgs {
    const void *codes;
    const void *scales;
    const _Float16 *A;
    const float *inv;
    float *y;
    long ystride;
    int V, K, N, KB;
};

__device__ __forceinline__ _Float16 sext8h(uint32_t v, int i) { return (_Float16)(int)((int32_t)(v << (24 - 8 * i)) >> 24); }

// MT M-tiles (16 A rows each = 8 vectors), SK K-slices per block, RG groups of
// 16 weight rows per block.
enum { VEC_STORE = 0, VEC_ADD = 1, VEC_SWIGLU = 2 };

template <int FMT, int MT, int SK, int RG, int EPI = VEC_STORE>
__global__ __launch_bounds__(64 * SK * RG) void gemv_vec_kernel(const VecArgs a) {
    __shared__ f32x4 red[SK * RG * MT * 64];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int ks = wv % SK, rg = wv / SK;
    const int n0 = (blockIdx.x * RG + rg) * 16;
    const int n = min(n0 + (lane & 15), a.N - 1);  // weight row this lane loads
    const int g = lane >> 4;
    const int KB = a.KB;
    const int per = (KB + SK - 1) / SK;
    const int kb0 = ks * per, kb1 = min(KB, kb0 + per);
    f32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int kb = kb0; kb < kb1; ++kb) {
        // B fragment: 8 FP16 weights of row n, values kb*32 + g*8 .. +8.
        f16x8 b;
        float d = 1.0f;
        if constexpr (FMT == GPHQ_FMT_Q4) {
            const u32x2 w = __builtin_nontemporal_load(
                (const u32x2 *)((const uint8_t *)a.codes + (size_t)n * (a.K >> 1) + kb * 16 + (g & 1) * 8));
            const int sh = (g >> 1) * 4;
#pragma unroll
            for (int i = 0; i < 8; ++i)
                b[i] = (_Float16)(int)((((i < 4 ? w.x : w.y) >> (8 * (i & 3) + sh)) & 15)) - (_Float16)8.0f;
        } else {
            const u32x2 w =
                __builtin_nontemporal_load((const u32x2 *)((const int8_t *)a.codes + (size_t)n * a.K + kb * 32 + g * 8));
#pragma unroll
            for (int i = 0; i < 8; ++i) b[i] = sext8h(i < 4 ? w.x : w.y, i & 3);
        }
        if constexpr (FMT == GPHQ_FMT_Q8B || FMT == GPHQ_FMT_Q4)
            d = half_bits_to_float(__builtin_nontemporal_load((const uint16_t *)a.scales + (size_t)n * KB + kb));
        else if constexpr (FMT == GPHQ_FMT_Q8B_F32)
            d = __builtin_nontemporal_load((const float *)a.scales + (size_t)n * KB + kb);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const f16x8 av = *(const f16x8 *)(a.A + vec_a_offset(t, kb, KB, lane));
            const f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            if constexpr (FMT == GPHQ_FMT_Q8) {
                acc[t] += c;
            } else {
                // Output lane l holds C[4*(l/16)+i][l%16]; column l%16 is
                // weight row n0 + l%16, the row whose block scale this lane
                // loaded.
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(d, c[i], acc[t][i]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) red[((rg * SK + ks) * MT + t) * 64 + lane] = acc[t];
    __syncthreads();
    if (ks != 0) return;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        f32x4 s = red[((rg * SK) * MT + t) * 64 + lane];
#pragma unroll
        for (int q = 1; q < SK; ++q) s += red[((rg * SK + q) * MT + t) * 64 + lane];
        // Rows 4*(l/16)+i of tile t: pairs (hi, lo) of vectors t*8 + 2*(l/16) + {0, 1}.
        const int col = n0 + (lane & 15);
        float rs = 1.0f;
        if constexpr (FMT == GPHQ_FMT_Q8) rs = ((const float *)a.scales)[min(col, a.N - 1)];
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int v = t * 8 + 2 * (lane >> 4) + p;
            float val = (s[2 * p] + s[2 * p + 1]) * a.inv[min(v, a.V - 1)];
            if constexpr (FMT == GPHQ_FMT_Q8) val *= rs;
            if constexpr (EPI == VEC_SWIGLU) {
                // Lane l^1 holds column col^1: the up row of gate row col.
                const float u = __shfl_xor(val, 1);
                if (v < a.V && col < a.N && (col & 1) == 0)
                    a.y[(size_t)v * a.ystride + (col >> 1)] = val / (1.0f + expf(-val)) * u;
            } else if (v < a.V && col < a.N) {
                if constexpr (EPI == VEC_ADD)
                    a.y[(size_t)v * a.ystride + col] += val;
                else
                    a.y[(size_t)v * a.ystride + col] = val;
            }
        }
    }
}

size_t gemv_vec_workspace_bytes(int V, int K) {
    const int MT = (2 * V + 15) / 16;
    const int KB = (K + 31) / 32;
    return (size_t)MT * KB * 1024 + (size_t)kMaxVecLanes * 4 + 256;
}

template <int FMT, int MT, int EPI>
static int launch_vec(const VecArgs &a, hipStream_t stream) {
    constexpr int SK = 4, RG = 2;
    const unsigned blocks = (unsigned)((a.N + 16 * RG - 1) / (16 * RG));
    hipLaunchKernelGGL((gemv_vec_kernel<FMT, MT, SK, RG, EPI>), dim3(blocks), dim3(64 * SK * RG), 0, stream, a);
    return launch_status();
}

template <int FMT, int EPI = VEC_STORE>
static int launch_vec_fmt(const VecArgs &a, hipStream_t stream) {
    const int MT = (2 * a.V + 15) / 16;
    switch (MT) {
    case 1: return launch_vec<FMT, 1, EPI>(a, stream);
    case 2: return launch_vec<FMT, 2, EPI>(a, stream);
    case 3: return launch_vec<FMT, 3, EPI>(a, stream);
    case 4: return launch_vec<FMT, 4, EPI>(a, stream);
    }
    return GPHQ_ERR_UNSUPPORTED;
}

// y[v*ystride + j] for v < V. Arguments were validated by the caller.
int gemv_vec_launch(int fmt, const void *codes, const void *scales, const float *x, long xstride, float *y,
                    long ystride, int V, int K, int N, void *work, hipStream_t stream) {
    if (N == 0 || V == 0) return GPHQ_OK;
    const int KB = (K + 31) / 32;
    const int MT = (2 * V + 15) / 16;
    _Float16 *A = (_Float16 *)work;
    float *inv = (float *)((char *)work + (size_t)MT * KB * 1024);
    // A rows past 2V in the last M-tile are never written; they only feed the
    // matching C rows, which are never stored.
    hipLaunchKernelGGL(vec_prep_kernel, dim3(V), dim3(256), 0, stream, x, xstride, V, K, KB, A, inv, 0, 0.0f);
    GPHQ_TRY(launch_status());
    VecArgs a{codes, scales, A, inv, y, ystride, V, K, N, KB};
    switch (fmt) {
    case GPHQ_FMT_Q8: return launch_vec_fmt<GPHQ_FMT_Q8>(a, stream);
    case GPHQ_FMT_Q8B: return launch_vec_fmt<GPHQ_FMT_Q8B>(a, stream);
    case GPHQ_FMT_Q8B_F32: return launch_vec_fmt<GPHQ_FMT_Q8B_F32>(a, stream);
    case GPHQ_FMT_Q4: return launch_vec_fmt<GPHQ_FMT_Q4>(a, stream);
    }
    return GPHQ_ERR_UNSUPPORTED;
}

template <int EPI>
static int launch_vec_epi(int fmt, const VecArgs &a, hipStream_t stream) {
    switch (fmt) {
    case GPHQ_FMT_Q8: return launch_vec_fmt<GPHQ_FMT_Q8, EPI>(a, stream);
    case GPHQ_FMT_Q8B: return launch_vec_fmt<GPHQ_FMT_Q8B, EPI>(a, stream);
    case GPHQ_FMT_Q8B_F32: return launch_vec_fmt<GPHQ_FMT_Q8B_F32, EPI>(a, stream);
    case GPHQ_FMT_Q4: return launch_vec_fmt<GPHQ_FMT_Q4, EPI>(a, stream);
    }
    return GPHQ_ERR_UNSUPPORTED;
}

// Decode-step multi-vector GEMV: norm (0/1) selects PRO_NORM, epi is 0 store,
// 1 add, 2 SwiGLU (y then holds N/2 values per vector). V <= kMaxVecLanes,
// K % 32 == 0; validated by the caller.
int gemv_vec_fused_launch(int fmt, int norm, int epi, const void *codes, const void *scales, const float *x,
                          long xstride, float *y, long ystride, int V, int K, int N, float eps, void *work,
                          hipStream_t stream) {
    if (N == 0 || V == 0) return GPHQ_OK;
    const int KB = (K + 31) / 32;
    const int MT = (2 * V + 15) / 16;
    _Float16 *A = (_Float16 *)work;
    float *inv = (float *)((char *)work + (size_t)MT * KB * 1024);
    hipLaunchKernelGGL(vec_prep_kernel, dim3(V), dim3(256), 0, stream, x, xstride, V, K, KB, A, inv, norm, eps);
    GPHQ_TRY(launch_status());
    VecArgs a{codes, scales, A, inv, y, ystride, V, K, N, KB};
    if (epi == VEC_ADD) return launch_vec_epi<VEC_ADD>(fmt, a, stream);
    if (epi == VEC_SWIGLU) return launch_vec_epi<VEC_SWIGLU>(fmt, a, stream);
    return launch_vec_epi<VEC_STORE>(fmt, a, stream);
}

}  // namespace gphq
