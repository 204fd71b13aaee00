// Multi-vector GEMV: y[v] = dequant(W) . x[v] for V input vectors that share
// one read of the weights (qwen3lm gemvQ8BVector<V>, gpu.metal:239-314, the
// decode-lane kernels of gpu_darwin.go:1121-1281), for any V up to
// kMaxVecLanes and the Q8, Q8B, Q8B_F32 and Q4 formats, with the decode
// step's prologue (PRO_NORM) and epilogues (store, residual add, SwiGLU).
//
// Design: with fp32 VALU arithmetic every extra vector costs one FMA per
// weight, so 16 lanes would be VALU-bound. Here the vectors go through MFMA:
//   * vec_prep_blocks_kernel scales each 32-value block of each vector by an
//     exact power of two 2^e (its max into [2^14, 2^15)) and splits it into
//     FP16 hi + lo parts (x*2^e = hi + lo + r, |r| <= 2^-22 |x*2^e|), laid out
//     as MFMA A fragments: rows 2v (hi) and 2v+1 (lo) of tile v/8;
//   * gemv_vec2_kernel widens each 32-value block of 16 weight rows to FP16
//     (int8 and 4-bit codes are exact in FP16), runs one
//     v_mfma_f32_16x16x32_f16 per 16 A rows (products exact in fp32), and
//     folds the block result into fp32 accumulators with the weight block
//     scale and the activation block's 2^-e: acc = fma(d*2^-e, C, acc), the
//     per-block scaling of the qwen3lm kernels;
//   * K is split over wavefronts; partial sums meet in a fixed LDS tree;
//     y[v][n] = acc_hi + acc_lo (Q8: times the row scale; PRO_NORM: times
//     1/sqrt(mean(x^2) + eps) from the prep pass's block sums of squares).
// VALU work per weight does not grow with V.
#include "common.h"

namespace gphq {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Eight codes (two dwords) to FP16, exactly: each byte b, biased to
// u = b + 128 (8-bit codes) or taken as a nibble, is placed under the FP16
// exponent of 1024 (bits 0x64uu = 1024 + u) by one v_perm_b32 per pair, and
// one packed FP16 subtraction removes 1024 + bias.
__device__ __forceinline__ f16x8 bytes_to_f16x8(uint32_t u0, uint32_t u1, _Float16 bias) {
    const f16x2 b2 = {bias, bias};
    const f16x2 p0 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u)) - b2;
    const f16x2 p1 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u)) - b2;
    const f16x2 p2 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u)) - b2;
    const f16x2 p3 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u)) - b2;
    return f16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}
__device__ __forceinline__ f16x8 i8x8_to_f16(u32x2 w) {
    return bytes_to_f16x8(w.x ^ 0x80808080u, w.y ^ 0x80808080u, (_Float16)1152.0f);
}
// Nibbles (sh = 0 low, 4 high) of eight bytes, minus 8.
__device__ __forceinline__ f16x8 u4x8_to_f16(u32x2 w, int sh) {
    return bytes_to_f16x8((w.x >> sh) & 0x0F0F0F0Fu, (w.y >> sh) & 0x0F0F0F0Fu, (_Float16)1032.0f);
}

// 2^e for |e| <= 100 and the e placing m (>= 0) in [2^14, 2^15), from the
// float's exponent bits (m = 0, NaN, Inf and denormals clamp to +-100).
__device__ __forceinline__ int pow2_exponent(float m) {
    const int biased = (int)(__builtin_bit_cast(uint32_t, m) >> 23);
    return min(max(141 - biased, -100), 100);
}
__device__ __forceinline__ float pow2f(int e) { return __builtin_bit_cast(float, (uint32_t)(127 + e) << 23); }


enum { VEC_STORE = 0, VEC_ADD = 1, VEC_SWIGLU = 2 };

constexpr int kMaxVecLanes = 32;

// A fragments for block kb of M-tile t: 1 KiB = 64 lanes x 8 FP16; lane l
// holds A row t*16 + l%16, values kb*32 + (l/16)*8 .. +8.
__host__ __device__ inline size_t vec_a_offset(int t, int kb, int KB, int lane) {
    return ((size_t)t * KB + kb) * 512 + (size_t)lane * 8;
}

// ---- multi-vector GEMV with per-block activation scales ----------------------
// vec_prep_blocks_kernel: one thread per (vector v, 32-value block kb). The
// block's values are scaled by 2^e (its max into [2^14, 2^15)) and split into
// FP16 hi + lo, written as the MFMA A fragments of rows 2v (hi) and 2v+1 (lo)
// of tile v/8; inv[v][kb] = 2^-e and ssq[v][kb] = the block's sum of squares
// (for PRO_NORM). Every thread is independent, so the pass takes one short
// launch for any vector count.
__global__ __launch_bounds__(256) void vec_prep_blocks_kernel(const float *__restrict__ x, long stride, int V, int KB,
                                                              _Float16 *__restrict__ A, float *__restrict__ inv,
                                                              float *__restrict__ ssq) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= V * KB) return;
    const int v = idx / KB, kb = idx - v * KB;
    const float4 *xp = (const float4 *)(x + (size_t)v * stride + (size_t)kb * 32);
    float xs[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 q = xp[i];
        xs[4 * i] = q.x, xs[4 * i + 1] = q.y, xs[4 * i + 2] = q.z, xs[4 * i + 3] = q.w;
    }
    float mx = 0.0f, ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        mx = fmaxf(mx, fabsf(xs[i]));
        ss += xs[i] * xs[i];
    }
    const int e = pow2_exponent(mx);
    const float sc = pow2f(e);
    const int t = v >> 3, rHi = (2 * v) & 15, rLo = rHi + 1;
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
        f16x8 hi, lo;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float y = xs[gq * 8 + i] * sc;  // exact: a power-of-two scaling
            const _Float16 h = (_Float16)y;
            hi[i] = h;
            lo[i] = (_Float16)(y - (float)h);
        }
        *(f16x8 *)(A + vec_a_offset(t, kb, KB, gq * 16 + rHi)) = hi;
        *(f16x8 *)(A + vec_a_offset(t, kb, KB, gq * 16 + rLo)) = lo;
    }
    inv[idx] = pow2f(-e);
    ssq[idx] = ss;
}

struct Vec2Args {
    const void *codes;
    const void *scales;
    const _Float16 *A;
    const float *inv;  // [V][KB]
    const float *ssq;  // [V][KB]
    float *y;
    long ystride;
    int V, K, N, KB;
    float eps;
    float *part;  // K-split stationary path: [parts][V][N] partial sums
};

// Multi-vector GEMV over prepared A fragments: each wavefront applies its A
// fragments to RT tiles of 16 weight rows, U blocks at a time. All U*RT*MT
// MFMAs of a step are issued before their results are scaled and summed
// (acc += d * 2^-e_v * C), which keeps the MFMA latency off the critical path.
// VALU work per weight is the code conversion (v_perm + packed FP16
// subtract). K is split over the SK wavefronts of the block; partial sums meet
// in a fixed LDS tree, and PRO_NORM's sum of squares is read from the prep
// pass's block sums in block order.
template <int FMT, int MT, int SK, int RT, int U, int EPI, bool NORM>
__global__ __launch_bounds__(64 * SK) void gemv_vec2_kernel(const Vec2Args a) {
    static_assert((SK & (SK - 1)) == 0, "SK is a power of two");
    __shared__ f32x4 red[(SK > 1 ? SK / 2 : 1) * RT * MT * 64];
    const int lane = threadIdx.x & 63;
    const int ks = threadIdx.x >> 6;
    const int g = lane >> 4, m = lane & 15;
    const int n0 = blockIdx.x * (RT * 16);
    const int KB = a.KB;
    const int per = ((KB + SK - 1) / SK + U - 1) / U * U;  // whole U-groups per wavefront
    const int kb0 = ks * per, kb1 = min(KB, kb0 + per);
    const int8_t *wrow[RT];
    const uint8_t *srow[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int row = min(n0 + rt * 16 + m, a.N - 1);
        wrow[rt] = FMT == GPHQ_FMT_Q4 ? (const int8_t *)a.codes + (size_t)row * (a.K >> 1) + (g & 1) * 8
                                      : (const int8_t *)a.codes + (size_t)row * a.K + g * 8;
        srow[rt] = (const uint8_t *)a.scales + (size_t)row * KB * (FMT == GPHQ_FMT_Q8B_F32 ? 4 : 2);
    }
    // The lane's C rows 4g..4g+3 of tile t are vectors t*8 + 2g (hi, lo) and t*8 + 2g + 1.
    const float *invp[MT][2];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int p = 0; p < 2; ++p) invp[t][p] = a.inv + (size_t)min(t * 8 + 2 * g + p, a.V - 1) * KB;
    f32x4 acc[RT][MT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int kbs = kb0; kbs < kb1; kbs += U) {
        f16x8 av[U][MT];
        u32x2 w[U][RT];
        float d[U][RT], iv[U][MT][2];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kb = min(kbs + u, KB - 1);
            const bool ok = kbs + u < kb1;
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                av[u][t] = *(const f16x8 *)(a.A + vec_a_offset(t, kb, KB, lane));
                iv[u][t][0] = ok ? invp[t][0][kb] : 0.0f;
                iv[u][t][1] = ok ? invp[t][1][kb] : 0.0f;
            }
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                w[u][rt] = *(const u32x2 *)(wrow[rt] + (size_t)kb * (FMT == GPHQ_FMT_Q4 ? 16 : 32));
                if constexpr (FMT == GPHQ_FMT_Q8B || FMT == GPHQ_FMT_Q4)
                    d[u][rt] = half_bits_to_float(((const uint16_t *)srow[rt])[kb]);
                else if constexpr (FMT == GPHQ_FMT_Q8B_F32)
                    d[u][rt] = ((const float *)srow[rt])[kb];
                else
                    d[u][rt] = 1.0f;
            }
        }
        f32x4 c[U][RT][MT];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const f16x8 b = FMT == GPHQ_FMT_Q4 ? u4x8_to_f16(w[u][rt], (g >> 1) * 4) : i8x8_to_f16(w[u][rt]);
#pragma unroll
                for (int t = 0; t < MT; ++t)
                    c[u][rt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[u][t], b, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    const float d0 = d[u][rt] * iv[u][t][0], d1 = d[u][rt] * iv[u][t][1];
                    acc[rt][t][0] = fmaf(d0, c[u][rt][t][0], acc[rt][t][0]);
                    acc[rt][t][1] = fmaf(d0, c[u][rt][t][1], acc[rt][t][1]);
                    acc[rt][t][2] = fmaf(d1, c[u][rt][t][2], acc[rt][t][2]);
                    acc[rt][t][3] = fmaf(d1, c[u][rt][t][3], acc[rt][t][3]);
                }
    }
#pragma unroll
    for (int half = SK / 2; half >= 1; half >>= 1) {
        if (ks >= half && ks < 2 * half) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int t = 0; t < MT; ++t) red[(((ks - half) * RT + rt) * MT + t) * 64 + lane] = acc[rt][t];
        }
        __syncthreads();
        if (ks < half) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int t = 0; t < MT; ++t) acc[rt][t] += red[((ks * RT + rt) * MT + t) * 64 + lane];
        }
        __syncthreads();
    }
    if (ks != 0) return;
    float nf[MT][2];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int p = 0; p < 2; ++p) nf[t][p] = 1.0f;
    if constexpr (NORM) {
        // Each vector's block sums of squares, added by the whole wavefront in
        // a fixed order; lane group g keeps vectors t*8 + 2g + {0, 1}.
#pragma unroll
        for (int t = 0; t < MT; ++t) {
#pragma unroll
            for (int vv = 0; vv < 8; ++vv) {
                const float *q = a.ssq + (size_t)min(t * 8 + vv, a.V - 1) * KB;
                float part = 0.0f;
                for (int kb = lane; kb < KB; kb += 64) part += q[kb];
                const float tot = wave_sum(part);
                if ((vv >> 1) == g) nf[t][vv & 1] = 1.0f / sqrtf(tot / (float)a.K + a.eps);
            }
        }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int col = n0 + rt * 16 + m;
        float rs = 1.0f;
        if constexpr (FMT == GPHQ_FMT_Q8) rs = ((const float *)a.scales)[min(col, a.N - 1)];
#pragma unroll
        for (int t = 0; t < MT; ++t) {
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const int v = t * 8 + 2 * g + p;
                float val = (acc[rt][t][2 * p] + acc[rt][t][2 * p + 1]) * nf[t][p];
                if constexpr (FMT == GPHQ_FMT_Q8) val *= rs;
                if constexpr (EPI == VEC_SWIGLU) {
                    const float up = __shfl_xor(val, 1);  // lane l^1 holds column col^1
                    if (v < a.V && col < a.N && (col & 1) == 0)
                        a.y[(size_t)v * a.ystride + (col >> 1)] = val / (1.0f + expf(-val)) * up;
                } else if (v < a.V && col < a.N) {
                    if constexpr (EPI == VEC_ADD)
                        a.y[(size_t)v * a.ystride + col] += val;
                    else
                        a.y[(size_t)v * a.ystride + col] = val;
                }
            }
        }
    }
}


// ---- stationary activations: up to 16 vectors, 8-bit formats -------------------
// For V <= 16 vectors and K a multiple of 512 up to 4096 the activations stay
// in registers and the weights are transposed through LDS:
//   * vech_prep_kernel (one block per A row, 16 blocks, x read once) scales
//     each vector by one power of two 2^e (its max into [2^14, 2^15)) and
//     splits it into
//     FP16 hi + lo, as two 16-row A tiles (tile 0 hi, tile 1 lo; row v =
//     vector v, rows past V zero). Against the per-block split above, values
//     smaller than 2^-17 of the vector's maximum lose relative precision, but
//     their error stays below 2^-38 max|x| per product;
//   * vech_kernel: each wavefront of a block owns one K slice of 16 blocks and
//     keeps that slice's A fragments (hi and lo) in registers for the whole
//     launch. It walks 16-row tiles (persistent grid): weights are loaded as
//     8 rows x 128 bytes per instruction (whole cache lines; lane l of row
//     r takes 16-byte chunk (l & 7) ^ (r >> 1)), written to the wavefront's
//     LDS region and read back as MFMA B fragments (slot m*8 + (c ^ (m >> 1))
//     is bank-conflict free), while the next tile's loads are in flight. Per
//     block: hi and lo MFMAs accumulate into one 16x16 result (16 vectors x
//     16 rows), scaled by the weight block scale into fp32 accumulators; the
//     K slices meet in LDS in slice order. Each wavefront parks a tile's
//     partial sums in one of kVechCH LDS slots and moves on; every kVechCH
//     tiles one barrier pair lets wavefront w add up slot w's slices and run
//     that tile's epilogue, instead of two barriers and a one-wavefront
//     epilogue per tile.
// Measured on MI355X with 16 vectors (Qwen3-8B shapes, Q8B): the head 154 us
// (was 383 us with the per-block kernel), gate/up 34 us (was 83), qkv 16.5 us
// (was 33), o 13 us (was 20).
constexpr int kVechNB = 16;        // K blocks of 32 values per wavefront slice
constexpr int kVechMaxSlices = 8;  // 512 threads; the kernel holds ~230 VGPRs
constexpr int kVechCH = 8;         // tiles whose slice sums are reduced together

// One block of 1024 threads per vector; thread t holds float4 units t, t +
// 1024, .. of the vector (K <= 4 * 1024 * kPrepUnits), so the vector is read
// once: the maximum and the sum of squares come from registers, and the same
// registers are split into hi and lo.
constexpr int kPrepUnits = 8;
__global__ __launch_bounds__(1024) void vech_prep_kernel(const float *__restrict__ x, long stride, int V, int K,
                                                         _Float16 *__restrict__ A, float *__restrict__ inv,
                                                         float *__restrict__ ssq, const VecFold f) {
    typedef _Float16 f16x4v __attribute__((ext_vector_type(4)));
    __shared__ float red[2][16];
    const int v = blockIdx.x;  // 16 blocks; rows v >= V are written as zero
    const bool live = v < V;
    const float *xv = x + (size_t)min(v, V - 1) * stride;
    const int U = K / 4;
    float4 q[kPrepUnits];
#pragma unroll
    for (int j = 0; j < kPrepUnits; ++j) {
        const int u = threadIdx.x + j * 1024;
        q[j] = (live && u < U) ? *(const float4 *)(xv + 4 * u) : float4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    if (f.parts) {
        // The pending residual add of a K-split GEMV: x += (sum of its parts
        // in order) * its vector scale (* the Q8 row scale), in
        // vech_finish_kernel's order, written back to x.
        const float pinv = live ? f.inv[v] : 0.0f;
#pragma unroll
        for (int j = 0; j < kPrepUnits; ++j) {
            const int u = threadIdx.x + j * 1024;
            if (!live || u >= U) continue;
            float4 sum = float4{0.0f, 0.0f, 0.0f, 0.0f};
            for (int pp = 0; pp < f.parts; ++pp) {
                const float4 t = *(const float4 *)(f.part + ((size_t)pp * V + v) * K + 4 * u);
                sum.x += t.x, sum.y += t.y, sum.z += t.z, sum.w += t.w;
            }
            float4 val{__fmul_rn(sum.x, pinv), __fmul_rn(sum.y, pinv), __fmul_rn(sum.z, pinv), __fmul_rn(sum.w, pinv)};
            if (f.rowScale) {
                const float4 rs = *(const float4 *)(f.rowScale + 4 * u);
                val = float4{__fmul_rn(val.x, rs.x), __fmul_rn(val.y, rs.y), __fmul_rn(val.z, rs.z), __fmul_rn(val.w, rs.w)};
            }
            q[j] = float4{__fadd_rn(q[j].x, val.x), __fadd_rn(q[j].y, val.y), __fadd_rn(q[j].z, val.z),
                          __fadd_rn(q[j].w, val.w)};
            *(float4 *)(const_cast<float *>(xv) + 4 * u) = q[j];
        }
    }
    float mx = 0.0f, ss = 0.0f;
#pragma unroll
    for (int j = 0; j < kPrepUnits; ++j) {
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(q[j].x), fabsf(q[j].y)), fmaxf(fabsf(q[j].z), fabsf(q[j].w))));
        ss += q[j].x * q[j].x + q[j].y * q[j].y + q[j].z * q[j].z + q[j].w * q[j].w;
    }
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[0][threadIdx.x >> 6] = mx, red[1][threadIdx.x >> 6] = ss;
    __syncthreads();
    mx = red[0][0];
#pragma unroll
    for (int w = 1; w < 16; ++w) mx = fmaxf(mx, red[0][w]);
    const int e = pow2_exponent(mx);
    const float sc = live ? pow2f(e) : 0.0f;
    const int KB = K / 32;
#pragma unroll
    for (int j = 0; j < kPrepUnits; ++j) {
        const int u = threadIdx.x + j * 1024;
        if (u >= U) break;
        // Unit u: block u / 8, 8-value group (u % 8) / 2, half u % 2.
        const int kb = u >> 3, gq = (u >> 1) & 3, half = u & 1;
        const float xs[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
        f16x4v hi, lo;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float y = xs[i] * sc;  // exact: a power-of-two scaling (or zero)
            const _Float16 h = (_Float16)y;
            hi[i] = h;
            lo[i] = (_Float16)(y - (float)h);
        }
        *(f16x4v *)(A + vec_a_offset(0, kb, KB, gq * 16 + v) + half * 4) = hi;
        *(f16x4v *)(A + vec_a_offset(1, kb, KB, gq * 16 + v) + half * 4) = lo;
    }
    if (threadIdx.x == 0 && live) {
        inv[v] = pow2f(-e);
        float t = red[1][0];
#pragma unroll
        for (int w = 1; w < 16; ++w) t += red[1][w];
        ssq[v] = t;
    }
}

template <int FMT, int SK, int EPI, bool NORM, bool SPLIT>
__global__ __launch_bounds__(64 * SK) void vech_kernel(const Vec2Args a, int iters) {
    constexpr int NB = kVechNB, STEPS = NB / 4;
    // Scale bytes per row and slice in 16-byte loads (Q8's row scale is applied at the end).
    constexpr int SC = FMT == GPHQ_FMT_Q8B ? NB * 2 / 16 : FMT == GPHQ_FMT_Q8B_F32 ? NB * 4 / 16 : 1;
    __shared__ u32x4 stage[SK][STEPS * 128];
    constexpr int CH = SK < kVechCH ? SK : kVechCH;
    __shared__ f32x4 part[SK > 1 ? CH * SK * 64 : 1];  // [slot][slice][lane]
    const int lane = threadIdx.x & 63;
    const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, m = lane & 15;
    const int KB = a.KB;
    // SPLIT: blockIdx.y picks which SK slices of K this block holds.
    const int kb0 = ((SPLIT ? (int)blockIdx.y * SK : 0) + ks) * NB;
    const int tiles = (a.N + 15) / 16;
    u32x4 *st = stage[ks];
    u32x4 R[STEPS][2];
    uint32_t S[SC * 4], Sn[SC * 4];  // the slice's block scales of this lane's row, as words
    auto gload = [&](int t2, uint32_t (&sd)[SC * 4]) {
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
            const int mm = h2 * 8 + (lane >> 3);
            const int c = (lane & 7) ^ (mm >> 1);
            const int row = min(t2 * 16 + mm, a.N - 1);
            const int8_t *src = (const int8_t *)a.codes + (size_t)row * a.K + kb0 * 32 + c * 16;
#pragma unroll
            for (int s = 0; s < STEPS; ++s) R[s][h2] = __builtin_nontemporal_load((const u32x4 *)(src + s * 128));
        }
        if constexpr (FMT != GPHQ_FMT_Q8) {
            const int row = min(t2 * 16 + m, a.N - 1);
            const uint8_t *sr = (const uint8_t *)a.scales + ((size_t)row * KB + kb0) * (FMT == GPHQ_FMT_Q8B ? 2 : 4);
#pragma unroll
            for (int q = 0; q < SC; ++q) {
                const u32x4 w4 = *(const u32x4 *)(sr + q * 16);
                sd[4 * q] = w4.x, sd[4 * q + 1] = w4.y, sd[4 * q + 2] = w4.z, sd[4 * q + 3] = w4.w;
            }
        }
    };
    auto lwrite = [&]() {
#pragma unroll
        for (int s = 0; s < STEPS; ++s)
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) st[s * 128 + h2 * 64 + lane] = R[s][h2];
    };
    int tt = blockIdx.x;
    if (tt < tiles) {
        gload(tt, S);
        lwrite();
    }
    f16x8 ah[NB], al[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        ah[b] = *(const f16x8 *)(a.A + vec_a_offset(0, kb0 + b, KB, lane));
        al[b] = *(const f16x8 *)(a.A + vec_a_offset(1, kb0 + b, KB, lane));
    }
    // The scale of each of the lane's 4 vectors (with the RMSNorm factor),
    // read once: read in the epilogue, each would wait for the previous
    // tile's stores as well.
    float vscale[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int vc = min(4 * g + i, a.V - 1);
        vscale[i] = a.inv[vc];
        if constexpr (NORM) vscale[i] = vscale[i] * (1.0f / sqrtf(a.ssq[vc] / (float)a.K + a.eps));
    }
    for (int it = 0; it < iters; ++it, tt += gridDim.x) {
        const bool valid = tt < tiles;
        const bool more = tt + (int)gridDim.x < tiles;
        if (more) gload(tt + gridDim.x, Sn);
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
        if (valid) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int c = 2 * (b & 3) + (g >> 1);
                const u32x2 wv =
                    *(const u32x2 *)((const uint32_t *)(st + (b >> 2) * 128 + m * 8 + (c ^ (m >> 1))) + (g & 1) * 2);
                float d = 1.0f;
                if constexpr (FMT == GPHQ_FMT_Q8B) {
                    const uint32_t sw = S[b / 2];
                    d = half_bits_to_float((uint16_t)((b & 1) ? sw >> 16 : sw));
                } else if constexpr (FMT == GPHQ_FMT_Q8B_F32) {
                    d = __builtin_bit_cast(float, S[b]);
                }
                const f16x8 bf = i8x8_to_f16(wv);
                f32x4 cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[b], bf, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[b], bf, cc, 0, 0, 0);
                if constexpr (FMT == GPHQ_FMT_Q8) {
                    acc += cc;
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[i] = fmaf(d, cc[i], acc[i]);
                }
            }
        }
        if (more) {
            lwrite();  // after this tile's LDS reads (LDS operations of a wavefront run in order)
#pragma unroll
            for (int q = 0; q < SC * 4; ++q) S[q] = Sn[q];
        }
        // Lane (g, m) holds vectors 4g..4g+3 of row t*16 + m.
        auto epilogue = [&](int t, const f32x4 &r) {
            const int col = t * 16 + m;
            if constexpr (SPLIT) {  // this part's sums; vech_finish_kernel applies the rest
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int v = 4 * g + i;
                    if (v < a.V && col < a.N) a.part[((size_t)blockIdx.y * a.V + v) * a.N + col] = r[i];
                }
                return;
            }
            float rs = 1.0f;
            if constexpr (FMT == GPHQ_FMT_Q8) rs = ((const float *)a.scales)[min(col, a.N - 1)];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int v = 4 * g + i;
                // inv is a power of two, so r * (inv * f) rounds like (r * inv) * f.
                float val = r[i] * vscale[i];
                if constexpr (FMT == GPHQ_FMT_Q8) val *= rs;
                if constexpr (EPI == VEC_SWIGLU) {
                    const float up = __shfl_xor(val, 1);  // lane m^1 holds row col^1
                    if (v < a.V && col < a.N && (col & 1) == 0)
                        a.y[(size_t)v * a.ystride + (col >> 1)] = val / (1.0f + expf(-val)) * up;
                } else if (v < a.V && col < a.N) {
                    if constexpr (EPI == VEC_ADD)
                        a.y[(size_t)v * a.ystride + col] += val;
                    else
                        a.y[(size_t)v * a.ystride + col] = val;
                }
            }
        };
        if constexpr (SK > 1) {
            const int slot = it % CH;
            part[(slot * SK + ks) * 64 + lane] = acc;
            if (slot != CH - 1 && it != iters - 1) continue;  // the same for every wavefront
            __syncthreads();
            if (ks <= slot) {
                // Wavefront ks reduces slot ks (tile tt - (slot - ks) blocks
                // back) in slice order, as one wavefront adding the others'.
                const f32x4 *ps = part + ks * SK * 64 + lane;
                f32x4 r = ps[0];
                for (int k2 = 1; k2 < SK; ++k2) r += ps[k2 * 64];
                const int t = tt - (slot - ks) * (int)gridDim.x;
                if (t < tiles) epilogue(t, r);
            }
            __syncthreads();
        } else {
            if (!valid) break;
            epilogue(tt, acc);
        }
    }
}

// The K-split stationary path's finish: thread (v, row) sums the parts in
// order, then applies the vector's scale, the norm, the Q8 row scale and the
// epilogue as vech_kernel does (SwiGLU: one thread per row pair).
template <int FMT, int EPI, bool NORM>
__global__ __launch_bounds__(256) void vech_finish_kernel(const Vec2Args a, int parts) {
    const int per = EPI == VEC_SWIGLU ? a.N / 2 : a.N;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= a.V * per) return;
    const int v = idx / per, r = idx - v * per;
    auto row_value = [&](int col) {
        float sum = 0.0f;
        for (int p = 0; p < parts; ++p) sum += a.part[((size_t)p * a.V + v) * a.N + col];
        float val = __fmul_rn(sum, a.inv[v]);
        if constexpr (NORM) val = __fmul_rn(val, 1.0f / sqrtf(a.ssq[v] / (float)a.K + a.eps));
        if constexpr (FMT == GPHQ_FMT_Q8) val = __fmul_rn(val, ((const float *)a.scales)[col]);
        return val;
    };
    if constexpr (EPI == VEC_SWIGLU) {
        const float gate = row_value(2 * r), up = row_value(2 * r + 1);
        a.y[(size_t)v * a.ystride + r] = gate / (1.0f + expf(-gate)) * up;
    } else if constexpr (EPI == VEC_ADD) {
        float *yp = a.y + (size_t)v * a.ystride + r;
        *yp = __fadd_rn(*yp, row_value(r));  // the same rounding as a folded add (vech_prep_kernel)
    } else {
        a.y[(size_t)v * a.ystride + r] = row_value(r);
    }
}

// Whether the stationary-activation kernel takes this GEMV.
static bool vech_takes(int fmt, int V, int K) {
    return fmt != GPHQ_FMT_Q4 && V >= 1 && V <= 16 && K % (32 * kVechNB) == 0 &&
           K / (32 * kVechNB) <= kVechMaxSlices;
}

// K parts of the split stationary path (K above one block's kVechMaxSlices
// slices, split evenly), or 0 when it does not apply.
static int vech_split_parts(int fmt, int V, int K) {
    if (fmt == GPHQ_FMT_Q4 || V < 1 || V > 16 || K % (32 * kVechNB)) return 0;
    const int slices = K / (32 * kVechNB);
    if (slices <= kVechMaxSlices) return 0;
    const int parts = (slices + kVechMaxSlices - 1) / kVechMaxSlices;
    return slices % parts == 0 && parts <= 8 && K <= 4 * 1024 * kPrepUnits ? parts : 0;
}

size_t gemv_vec_split_bytes(int V, int K, int N) {
    const int parts = vech_split_parts(GPHQ_FMT_Q8B, V, K);
    return parts ? (size_t)parts * V * N * 4 : 0;
}

static int vech_cus() {
    static int cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (!cached[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

template <int FMT, int SK, int EPI, bool NORM>
static int go_vech(const Vec2Args &a, hipStream_t stream) {
    const int tiles = (a.N + 15) / 16;
    const int perCu = std::max(1, 8 / SK);  // about 8 wavefronts per CU
    const int blocks = std::max(1, std::min(tiles, vech_cus() * perCu));
    const int iters = (tiles + blocks - 1) / blocks;
    hipLaunchKernelGGL((vech_kernel<FMT, SK, EPI, NORM, false>), dim3((unsigned)blocks), dim3(64 * SK), 0, stream, a,
                       iters);
    return launch_status();
}

// K-split stationary path: blocks of kVechMaxSlices slices, one grid row per
// K part (about 8 wavefronts per CU in all), then the ordered finish.
template <int FMT, int EPI, bool NORM>
static int go_vech_split(const Vec2Args &a, int parts, hipStream_t stream, bool finish) {
    constexpr int SK = kVechMaxSlices;
    const int tiles = (a.N + 15) / 16;
    const int blocks = std::max(1, std::min(tiles, vech_cus() / parts));
    const int iters = (tiles + blocks - 1) / blocks;
    hipLaunchKernelGGL((vech_kernel<FMT, SK, VEC_STORE, false, true>), dim3((unsigned)blocks, (unsigned)parts),
                       dim3(64 * SK), 0, stream, a, iters);
    GPHQ_TRY(launch_status());
    if (!finish) return GPHQ_OK;  // the next preparation adds the parts (VecFold)
    const int per = EPI == VEC_SWIGLU ? a.N / 2 : a.N;
    hipLaunchKernelGGL((vech_finish_kernel<FMT, EPI, NORM>), dim3((unsigned)((a.V * per + 255) / 256)), dim3(256), 0,
                       stream, a, parts);
    return launch_status();
}

template <int EPI, bool NORM>
static int launch_vech_split(int fmt, const Vec2Args &a, int parts, hipStream_t stream, bool finish = true) {
    switch (fmt) {
    case GPHQ_FMT_Q8: return go_vech_split<GPHQ_FMT_Q8, EPI, NORM>(a, parts, stream, finish);
    case GPHQ_FMT_Q8B: return go_vech_split<GPHQ_FMT_Q8B, EPI, NORM>(a, parts, stream, finish);
    case GPHQ_FMT_Q8B_F32: return go_vech_split<GPHQ_FMT_Q8B_F32, EPI, NORM>(a, parts, stream, finish);
    }
    return GPHQ_ERR_UNSUPPORTED;
}

template <int FMT, int EPI, bool NORM>
static int launch_vech_sk(const Vec2Args &a, hipStream_t stream) {
    switch (a.K / (32 * kVechNB)) {
    case 1: return go_vech<FMT, 1, EPI, NORM>(a, stream);
    case 2: return go_vech<FMT, 2, EPI, NORM>(a, stream);
    case 3: return go_vech<FMT, 3, EPI, NORM>(a, stream);
    case 4: return go_vech<FMT, 4, EPI, NORM>(a, stream);
    case 5: return go_vech<FMT, 5, EPI, NORM>(a, stream);
    case 6: return go_vech<FMT, 6, EPI, NORM>(a, stream);
    case 7: return go_vech<FMT, 7, EPI, NORM>(a, stream);
    case 8: return go_vech<FMT, 8, EPI, NORM>(a, stream);
    }
    return GPHQ_ERR_UNSUPPORTED;
}

template <int EPI, bool NORM>
static int launch_vech(int fmt, const Vec2Args &a, hipStream_t stream) {
    switch (fmt) {
    case GPHQ_FMT_Q8: return launch_vech_sk<GPHQ_FMT_Q8, EPI, NORM>(a, stream);
    case GPHQ_FMT_Q8B: return launch_vech_sk<GPHQ_FMT_Q8B, EPI, NORM>(a, stream);
    case GPHQ_FMT_Q8B_F32: return launch_vech_sk<GPHQ_FMT_Q8B_F32, EPI, NORM>(a, stream);
    }
    return GPHQ_ERR_UNSUPPORTED;
}

size_t gemv_vec_workspace_bytes(int V, int K) {
    const int MT = std::max(2, (2 * V + 15) / 16);  // the stationary path uses two tiles
    const int KB = (K + 31) / 32;
    return (size_t)MT * KB * 1024 + 2 * (size_t)V * KB * 4 + 256;
}

// Tile shapes measured on MI355X (Qwen3-8B projections, 4 and 16 vectors):
// up to 8192 rows, 16-row blocks of four K-slices with four blocks in flight;
// taller matrices, 64-row blocks of eight K-slices with two in flight.
template <int FMT, int MT, int EPI, bool NORM>
static int launch_vec2(const Vec2Args &a, hipStream_t stream) {
    if (a.N <= 8192) {
        hipLaunchKernelGGL((gemv_vec2_kernel<FMT, MT, 4, 1, 4, EPI, NORM>), dim3((unsigned)((a.N + 15) / 16)),
                           dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL((gemv_vec2_kernel<FMT, MT, 8, 4, 2, EPI, NORM>), dim3((unsigned)((a.N + 63) / 64)),
                           dim3(512), 0, stream, a);
    }
    return launch_status();
}

template <int FMT, int EPI, bool NORM>
static int launch_vec2_mt(const Vec2Args &a, hipStream_t stream) {
    switch ((2 * a.V + 15) / 16) {
    case 1: return launch_vec2<FMT, 1, EPI, NORM>(a, stream);
    case 2: return launch_vec2<FMT, 2, EPI, NORM>(a, stream);
    case 3: return launch_vec2<FMT, 3, EPI, NORM>(a, stream);
    case 4: return launch_vec2<FMT, 4, EPI, NORM>(a, stream);
    }
    return GPHQ_ERR_UNSUPPORTED;
}

template <int EPI, bool NORM>
static int launch_vec2_fmt(int fmt, const Vec2Args &a, hipStream_t stream) {
    switch (fmt) {
    case GPHQ_FMT_Q8: return launch_vec2_mt<GPHQ_FMT_Q8, EPI, NORM>(a, stream);
    case GPHQ_FMT_Q8B: return launch_vec2_mt<GPHQ_FMT_Q8B, EPI, NORM>(a, stream);
    case GPHQ_FMT_Q8B_F32: return launch_vec2_mt<GPHQ_FMT_Q8B_F32, EPI, NORM>(a, stream);
    case GPHQ_FMT_Q4: return launch_vec2_mt<GPHQ_FMT_Q4, EPI, NORM>(a, stream);
    }
    return GPHQ_ERR_UNSUPPORTED;
}

// Multi-vector GEMV, optionally with the decode step's prologue and epilogue:
// norm (0/1) selects PRO_NORM, epi is VEC_STORE, VEC_ADD or VEC_SWIGLU (y then
// holds N/2 values per vector). V <= kMaxVecLanes, K % 32 == 0, x rows 16-byte
// aligned; work holds gemv_vec_workspace_bytes(V, K). Validated by the caller.
// Whether a preparation for (fmt, V, K) goes through vech_prep_kernel, so a
// pending K-split residual add (VecFold) can be handed to it.
bool gemv_vec_prep_folds(int fmt, int V, int K) {
    return vech_split_parts(fmt, V, K) != 0 || vech_takes(fmt, V, K);
}

// fold: a K-split GEMV's residual add into x left pending by an earlier call
// (applied by this call's preparation, before it reads x); defer: when this
// call is a K-split residual add without a norm, its finish is left to the
// caller's next preparation and described in *defer (parts 0 otherwise).
int gemv_vec_fused_launch(int fmt, int norm, int epi, const void *codes, const void *scales, const float *x,
                          long xstride, float *y, long ystride, int V, int K, int N, float eps, void *work,
                          hipStream_t stream, float *split, size_t split_bytes, const VecFold &fold, VecFold *defer) {
    if (defer) *defer = VecFold{};
    if (N == 0 || V == 0) return fold.parts ? GPHQ_ERR_UNSUPPORTED : GPHQ_OK;
    const int KB = K / 32;
    const int parts = vech_split_parts(fmt, V, K);
    if (fold.parts && !gemv_vec_prep_folds(fmt, V, K)) return GPHQ_ERR_UNSUPPORTED;
    if (parts && split && split_bytes >= (size_t)parts * V * N * 4 && (epi != VEC_SWIGLU || N % 2 == 0)) {
        _Float16 *A = (_Float16 *)work;
        float *inv = (float *)((char *)work + (size_t)2 * KB * 1024);
        float *ssq = inv + V;
        hipLaunchKernelGGL(vech_prep_kernel, dim3(16), dim3(1024), 0, stream, x, xstride, V, K, A, inv, ssq, fold);
        GPHQ_TRY(launch_status());
        Vec2Args a{codes, scales, A, inv, ssq, y, ystride, V, K, N, KB, eps};
        a.part = split;
        if (epi == VEC_ADD && !norm && defer) {
            const int rc = launch_vech_split<VEC_ADD, false>(fmt, a, parts, stream, false);
            if (rc != GPHQ_OK) return rc;
            *defer = VecFold{split, inv, fmt == GPHQ_FMT_Q8 ? (const float *)scales : nullptr, parts};
            return GPHQ_OK;
        }
        if (epi == VEC_ADD) return norm ? launch_vech_split<VEC_ADD, true>(fmt, a, parts, stream)
                                        : launch_vech_split<VEC_ADD, false>(fmt, a, parts, stream);
        if (epi == VEC_SWIGLU) return norm ? launch_vech_split<VEC_SWIGLU, true>(fmt, a, parts, stream)
                                           : launch_vech_split<VEC_SWIGLU, false>(fmt, a, parts, stream);
        return norm ? launch_vech_split<VEC_STORE, true>(fmt, a, parts, stream)
                    : launch_vech_split<VEC_STORE, false>(fmt, a, parts, stream);
    }
    if (vech_takes(fmt, V, K)) {
        _Float16 *A = (_Float16 *)work;
        float *inv = (float *)((char *)work + (size_t)2 * KB * 1024);
        float *ssq = inv + V;
        hipLaunchKernelGGL(vech_prep_kernel, dim3(16), dim3(1024), 0, stream, x, xstride, V, K, A, inv, ssq, fold);
        GPHQ_TRY(launch_status());
        const Vec2Args a{codes, scales, A, inv, ssq, y, ystride, V, K, N, KB, eps};
        if (epi == VEC_ADD) return norm ? launch_vech<VEC_ADD, true>(fmt, a, stream)
                                        : launch_vech<VEC_ADD, false>(fmt, a, stream);
        if (epi == VEC_SWIGLU) return norm ? launch_vech<VEC_SWIGLU, true>(fmt, a, stream)
                                           : launch_vech<VEC_SWIGLU, false>(fmt, a, stream);
        return norm ? launch_vech<VEC_STORE, true>(fmt, a, stream) : launch_vech<VEC_STORE, false>(fmt, a, stream);
    }
    const int MT = (2 * V + 15) / 16;
    _Float16 *A = (_Float16 *)work;
    float *inv = (float *)((char *)work + (size_t)MT * KB * 1024);
    float *ssq = inv + (size_t)V * KB;
    // A rows past 2V in the last tile are never written; they only feed C
    // rows that are never stored.
    if (KB > 0) {
        hipLaunchKernelGGL(vec_prep_blocks_kernel, dim3((unsigned)((V * KB + 255) / 256)), dim3(256), 0, stream, x,
                           xstride, V, KB, A, inv, ssq);
        GPHQ_TRY(launch_status());
    }
    const Vec2Args a{codes, scales, A, inv, ssq, y, ystride, V, K, N, KB, eps};
    if (epi == VEC_ADD) return norm ? launch_vec2_fmt<VEC_ADD, true>(fmt, a, stream)
                                    : launch_vec2_fmt<VEC_ADD, false>(fmt, a, stream);
    if (epi == VEC_SWIGLU) return norm ? launch_vec2_fmt<VEC_SWIGLU, true>(fmt, a, stream)
                                       : launch_vec2_fmt<VEC_SWIGLU, false>(fmt, a, stream);
    return norm ? launch_vec2_fmt<VEC_STORE, true>(fmt, a, stream) : launch_vec2_fmt<VEC_STORE, false>(fmt, a, stream);
}

// y[v*ystride + j] for v < V (gphq_gemv_vec). Arguments were validated by the caller.
int gemv_vec_launch(int fmt, const void *codes, const void *scales, const float *x, long xstride, float *y,
                    long ystride, int V, int K, int N, void *work, hipStream_t stream) {
    return gemv_vec_fused_launch(fmt, 0, VEC_STORE, codes, scales, x, xstride, y, ystride, V, K, N, 0.0f, work,
                                 stream, nullptr, 0, VecFold{}, nullptr);
}

}  // namespace gphq
