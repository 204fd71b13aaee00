// Block-32 int8 GEMM on MI355X: benchmark configuration 2 as worded there
// (activations and weights each with one fp32 scale per 32-value block). The
// reference has no such function: its q8gemm int8 path scales per row
// (int8.go:106-211, gphq_q8gemm_*). Each 32-value block is quantized with
// WorkspaceI8's per-row rule (int8.go:106-168), and the product sums, per
// output and in block order, acc = fmaf(float(dot_b), da[r][b] * dw[c][b], acc)
// with dot_b the exact int32 block product, so results are bit-exact against
// the oracle's restatement of that sum.
//
// v_mfma_i32_32x32x32_i8 takes exactly one 32-value block per instruction, so
// every block's int32 products come out of one MFMA with a zero accumulator;
// the fp32 scale-accumulate that follows is VALU work (three instructions per
// output and block), which bounds this kernel well below the int8 MFMA rate.
#include <type_traits>

#include "common.h"

using namespace gphq;

namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// One thread per (row, 32-value block): scale = max/127 and inverse = 127/max
// (both 0 unless 0 < max < inf, int8.go:106-119), codes RNE(x * inverse)
// saturated to int8 (int8.go:163-168; a NaN product gives 0).
__global__ __launch_bounds__(256) void q8b_quantize_kernel(const float *__restrict__ x, int rows, int k, long stride,
                                                           int8_t *__restrict__ q, float *__restrict__ d) {
    const int kb = k >> 5;
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)rows * kb) return;
    const int r = (int)(idx / kb), b = (int)(idx - (long)r * kb);
    const float4 *src = (const float4 *)(x + r * stride + b * 32);
    float v[32];
    float mx = 0.0f;
    bool nan = false;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 f = src[i];
        v[4 * i] = f.x, v[4 * i + 1] = f.y, v[4 * i + 2] = f.z, v[4 * i + 3] = f.w;
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        nan |= v[i] != v[i];
        mx = fmaxf(mx, fabsf(v[i]));
    }
    float s = 0.0f, inv = 0.0f;
    if (!nan && mx > 0.0f && mx != INFINITY) {
        s = __fdiv_rn(mx, 127.0f);
        inv = __fdiv_rn(127.0f, mx);
    }
    d[idx] = s;
    int32_t packed[8];
#pragma unroll
    for (int w = 0; w < 8; ++w) {
        uint32_t word = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float p = __fmul_rn(v[4 * w + j], inv);
            float c = p != p ? 0.0f : rintf(p);
            c = fminf(127.0f, fmaxf(-128.0f, c));
            word |= (uint32_t)(uint8_t)(int8_t)(int)c << (8 * j);
        }
        packed[w] = (int32_t)word;
    }
    int32_t *dst = (int32_t *)(q + (long)r * k + b * 32);
    *(i32x4 *)dst = i32x4{packed[0], packed[1], packed[2], packed[3]};
    *(i32x4 *)(dst + 4) = i32x4{packed[4], packed[5], packed[6], packed[7]};
}

struct Q8bArgs {
    const int8_t *qa;
    const float *da;
    const int8_t *qw;
    const float *dw;
    float *y;
    int m, k, n, gridM, gridN;
};

// 16-byte chunk c of a row of KSB*32 bytes in LDS, swizzled within each
// 128-byte half by the row (big_swz), so fragment reads of consecutive rows
// at one chunk hit distinct banks.
__device__ __forceinline__ int q8b_swz(int row, int c) { return (c & ~7) | big_swz(row, c & 7); }

// BM x BN output tiles, WGM x WGN wavefronts of (BM/WGM) x (BN/WGN) as 32x32
// MFMA tiles. Per K step of KSB blocks (KSB*32 bytes) both code tiles pass
// through LDS in rows of 16-byte chunks (q8b_swz), the step's block scales as
// [block][row] floats; double buffered, the next step's global loads one step
// ahead in registers. Rows past m or n load row m-1 / n-1 and are not
// stored; blocks past k are skipped, and so are the scale-accumulates of a
// tile's rows 16..31 when they are all past m.
//
// Per block the wavefront issues the MFMAs of block b+1 before the
// scale-accumulate of block b (two sets of int32 results), so the matrix
// cores run beside the VALU chain; the chain itself keeps block order.
template <int BM, int BN, int WGM, int WGN, int KSB>
__global__ __launch_bounds__(64 * WGM * WGN) void q8b_gemm_kernel(const Q8bArgs a) {
    constexpr int NT = 64 * WGM * WGN;
    constexpr int TI = BM / WGM / 32, TJ = BN / WGN / 32;
    constexpr int CH = 2 * KSB;                          // 16-byte chunks per row and step
    constexpr int AL = BM * CH / NT, BL = BN * CH / NT;  // chunks per thread and step
    constexpr int SU = (BM + BN) * (KSB / 4);            // float4 scale units per step
    constexpr int SL = (SU + NT - 1) / NT;
    static_assert(AL * NT == BM * CH && BL * NT == BN * CH && KSB % 4 == 0, "loader split");
    __shared__ i32x4 As[2][BM * CH];
    __shared__ i32x4 Bs[2][BN * CH];
    __shared__ float Sa[2][KSB][BM];
    __shared__ float Sb[2][KSB][BN];
    int bm, bn;
    tile_order(blockIdx.x, a.gridM, a.gridN, bm, bn);
    const int t = threadIdx.x, lane = t & 63, wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wv / WGN, wn = wv % WGN;
    const int m0 = bm * BM, n0 = bn * BN;
    const int kb = a.k >> 5, steps = (kb + KSB - 1) / KSB;

    // Loader: unit u = i*NT + t is row u/CH, 16-byte chunk u%CH of the
    // step's bytes; chunks past k load zeros. Scale unit v = i*NT + t is one
    // float4 (four blocks) of A's row v (v < BM*KSB/4 ordering: row-major over
    // rows, then quads) or of B's row.
    // A full step (every chunk inside k, the usual case) loads without
    // per-chunk conditions. first marks the loads of step 1, which stay in
    // registers across the first step: relaxed atomic loads, so that the
    // compiler does not merge them with the in-loop loads of the same
    // registers into one load at the top of the loop (which would wait for
    // each step's codes as they are stored).
    i32x4 ar[AL], br[BL];
    float4 sr[SL];
    auto ld = [&](const int8_t *p, bool first) -> i32x4 {
        if (!first) return *(const i32x4 *)p;
        const long lo = __hip_atomic_load((const long *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        const long hi = __hip_atomic_load((const long *)p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        return i32x4{(int)lo, (int)(lo >> 32), (int)hi, (int)(hi >> 32)};
    };
    auto gload = [&](int st, bool first) {
        const int kbyte = st * KSB * 32;
        if (kbyte + KSB * 32 <= a.k) {
#pragma unroll
            for (int i = 0; i < AL; ++i) {
                const int u = i * NT + t, row = u / CH, ch = u % CH;
                ar[i] = ld(a.qa + (long)min(m0 + row, a.m - 1) * a.k + kbyte + ch * 16, first);
            }
#pragma unroll
            for (int i = 0; i < BL; ++i) {
                const int u = i * NT + t, row = u / CH, ch = u % CH;
                br[i] = ld(a.qw + (long)min(n0 + row, a.n - 1) * a.k + kbyte + ch * 16, first);
            }
        } else {
#pragma unroll
            for (int i = 0; i < AL; ++i) {
                const int u = i * NT + t, row = u / CH, ch = u % CH;
                const int gr = min(m0 + row, a.m - 1);
                ar[i] = kbyte + ch * 16 < a.k ? ld(a.qa + (long)gr * a.k + kbyte + ch * 16, first) : i32x4{0, 0, 0, 0};
            }
#pragma unroll
            for (int i = 0; i < BL; ++i) {
                const int u = i * NT + t, row = u / CH, ch = u % CH;
                const int gr = min(n0 + row, a.n - 1);
                br[i] = kbyte + ch * 16 < a.k ? ld(a.qw + (long)gr * a.k + kbyte + ch * 16, first) : i32x4{0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int i = 0; i < SL; ++i) {
            const int v = i * NT + t;
            float4 f = float4{0.f, 0.f, 0.f, 0.f};
            if (v < SU) {
                const int quad = v % (KSB / 4), row = v / (KSB / 4);
                const int b0 = st * KSB + quad * 4;
                float sv[4];
                if (row < BM) {
                    const float *sp = a.da + (long)min(m0 + row, a.m - 1) * kb;
#pragma unroll
                    for (int e = 0; e < 4; ++e) sv[e] = b0 + e < kb ? sp[b0 + e] : 0.0f;
                } else {
                    const float *sp = a.dw + (long)min(n0 + row - BM, a.n - 1) * kb;
#pragma unroll
                    for (int e = 0; e < 4; ++e) sv[e] = b0 + e < kb ? sp[b0 + e] : 0.0f;
                }
                f = float4{sv[0], sv[1], sv[2], sv[3]};
            }
            sr[i] = f;
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < AL; ++i) {
            const int u = i * NT + t, row = u / CH;
            As[buf][row * CH + q8b_swz(row, u % CH)] = ar[i];
        }
#pragma unroll
        for (int i = 0; i < BL; ++i) {
            const int u = i * NT + t, row = u / CH;
            Bs[buf][row * CH + q8b_swz(row, u % CH)] = br[i];
        }
#pragma unroll
        for (int i = 0; i < SL; ++i) {
            const int v = i * NT + t;
            if (v < SU) {
                const int quad = v % (KSB / 4), row = v / (KSB / 4);
                float *dst = row < BM ? &Sa[buf][quad * 4][row] : &Sb[buf][quad * 4][row - BM];
                const int stride = row < BM ? BM : BN;
                dst[0] = sr[i].x, dst[stride] = sr[i].y, dst[2 * stride] = sr[i].z, dst[3 * stride] = sr[i].w;
            }
        }
    };

    f32x16 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = f32x16{};
    // Row tile i's rows 16..31 hold rows of the matrix (else their
    // scale-accumulates are skipped; the wave takes the branch as one).
    bool hi[TI], allhi = true;
#pragma unroll
    for (int i = 0; i < TI; ++i) {
        hi[i] = m0 + wm * (32 * TI) + 32 * i + 16 < a.m;
        allhi = allhi && hi[i];
    }
    gload(0, false);
    lstore(0);
    if (steps > 1) gload(1, true);
    __syncthreads();
    const int fr = lane & 31, fh = lane >> 5;
    for (int st = 0; st < steps; ++st) {
        const int cur = st & 1;
        const int nb = min(KSB, kb - st * KSB);
        // The step's MFMAs run in units (block b, row tile i, column tile j),
        // block-major; unit u+1's MFMA is issued before unit u's
        // scale-accumulate, so the matrix cores work beside the VALU chain.
        constexpr int UN = KSB * TI * TJ;
        auto issue = [&](int u, i32x16 &d) {
            const int b = u / (TI * TJ), i = (u / TJ) % TI, j = u % TJ;
            const int c = 2 * b + fh;
            const int ra = wm * (32 * TI) + 32 * i + fr, rb = wn * (32 * TJ) + 32 * j + fr;
            d = __builtin_amdgcn_mfma_i32_32x32x32_i8(As[cur][ra * CH + q8b_swz(ra, c)],
                                                     Bs[cur][rb * CH + q8b_swz(rb, c)], i32x16{}, 0, 0, 0);
        };
        // acc = fmaf(float(dot), da * dw, acc) for unit u. This lane's 16
        // results of a tile are 4 runs of 4 consecutive rows; its column's
        // weight scale is one float. FULL: a whole step of blocks and every
        // row tile's rows 16..31 inside m (no conditions in the loop).
        auto apply = [&](auto full_c, int u, const i32x16 &d) {
            constexpr bool FULL = decltype(full_c)::value;
            const int b = u / (TI * TJ), i = (u / TJ) % TI, j = u % TJ;
            const float sb = Sb[cur][b][wn * (32 * TJ) + 32 * j + fr];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (!FULL && q >= 2 && !hi[i]) continue;
                const float4 s4 = *(const float4 *)&Sa[cur][b][wm * (32 * TI) + 32 * i + 8 * q + 4 * fh];
                const float sa[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float s = __fmul_rn(sa[e], sb);
                    acc[i][j][4 * q + e] = __builtin_fmaf((float)d[4 * q + e], s, acc[i][j][4 * q + e]);
                }
            }
        };
        auto units = [&](auto full_c) {
            constexpr bool FULL = decltype(full_c)::value;
            const int un = FULL ? UN : nb * TI * TJ;
            i32x16 d0, d1;
            issue(0, d0);
#pragma unroll
            for (int u = 0; u < UN; u += 2) {
                if (FULL || u < un) {
                    if (FULL || u + 1 < un) issue(u + 1, d1);
                    apply(full_c, u, d0);
                }
                if (FULL || u + 1 < un) {
                    if (u + 2 < UN && (FULL || u + 2 < un)) issue(u + 2, d0);
                    apply(full_c, u + 1, d1);
                }
            }
        };
        if (nb == KSB && allhi)
            units(std::true_type{});
        else
            units(std::false_type{});
        if (st + 1 < steps) {
            lstore(cur ^ 1);
            if (st + 2 < steps) gload(st + 2, false);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int col = n0 + wn * (32 * TJ) + 32 * j + fr;
            if (col >= a.n) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm * (32 * TI) + 32 * i + 8 * (e >> 2) + 4 * fh + (e & 3);
                if (row < a.m) a.y[(long)row * a.n + col] = acc[i][j][e];
            }
        }
}

// M <= 16 * TI: one wavefront (and block) per 16 weight rows, all
// activation rows in TI tiles of 16. A step is 128 bytes of K (four
// blocks): the wavefront loads its 16 weight rows and 16 * TI activation
// rows with 16-byte loads, eight lanes per row (whole 128-byte lines), their
// block scales with one float per lane, and keeps D steps of loads in
// flight in a register ring. Each step passes through the wavefront's own
// LDS (rows padded to 144 bytes), from which every block is one
// v_mfma_i32_16x16x32_i8 per activation tile (lane l supplies bytes
// 8(l/16)..+8 of the block for row or column l%16 and receives rows
// 4(l/16)..+3 of column l%16). The chain per output is the tiled kernel's,
// in block order: acc = fmaf(float(dot_b), da * dw, acc), so the results
// are the same bit for bit.
template <int TI, int D>
__global__ __launch_bounds__(64) void q8b_small_kernel(const Q8bArgs a) {
    constexpr int RS = 144;             // LDS row stride of the code tiles, bytes
    constexpr int AR = 16 * TI;         // activation rows
    static_assert(D % 2 == 0, "the ring pairs with two LDS buffers");
    __shared__ __align__(16) int8_t wl[2][16 * RS];
    __shared__ __align__(16) int8_t al[2][AR * RS];
    __shared__ float swl[2][16][4];                // [buffer][weight row][block of the step]
    __shared__ __align__(16) float sal[2][4][AR];  // [buffer][block of the step][activation row]
    const int lane = threadIdx.x, kb = a.k >> 5, steps = kb >> 2;
    const int n0 = blockIdx.x * 16;
    const int lr = lane >> 3, lc = lane & 7;  // loader: row lr (+8h), 16-byte chunk lc
    const int c = lane & 15, g = lane >> 4;   // MFMA lane: row/column c, byte group g
    const int8_t *wp[2];
    wp[0] = a.qw + (size_t)min(n0 + lr, a.n - 1) * a.k + lc * 16;
    wp[1] = a.qw + (size_t)min(n0 + lr + 8, a.n - 1) * a.k + lc * 16;
    const int8_t *ap[2 * TI];
#pragma unroll
    for (int h = 0; h < 2 * TI; ++h) ap[h] = a.qa + (size_t)min(lr + 8 * h, a.m - 1) * a.k + lc * 16;
    // Scales: lane l takes block l%4 of the step of weight row l/4 and of
    // activation rows l/4 + 16i.
    const float *dwp = a.dw + (size_t)min(n0 + (lane >> 2), a.n - 1) * kb + (lane & 3);
    const float *dap[TI];
#pragma unroll
    for (int i = 0; i < TI; ++i) dap[i] = a.da + (size_t)min((lane >> 2) + 16 * i, a.m - 1) * kb + (lane & 3);
    i32x4 wr[D][2], ar[D][2 * TI];
    float sw[D], sa[D][TI];
    auto load = [&](int p, int st, bool first) {
        const size_t off = (size_t)st * 128;
        auto ld = [&](const int8_t *q, bool stream) -> i32x4 {
            if (!first) return stream ? __builtin_nontemporal_load((const i32x4 *)q) : *(const i32x4 *)q;
            // Relaxed atomic loads for the first fill: with plain loads at
            // both the ring's entry and its refill the compiler merges them
            // into one load at the top of the loop, which waits for each
            // step as it is used.
            const long lo = __hip_atomic_load((const long *)q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            const long hi = __hip_atomic_load((const long *)q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            return i32x4{(int)lo, (int)(lo >> 32), (int)hi, (int)(hi >> 32)};
        };
        auto lf = [&](const float *q) -> float {
            return first ? __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) : *q;
        };
        wr[p][0] = ld(wp[0] + off, true);
        wr[p][1] = ld(wp[1] + off, true);
#pragma unroll
        for (int h = 0; h < 2 * TI; ++h) ar[p][h] = ld(ap[h] + off, false);
        sw[p] = lf(dwp + 4 * st);
#pragma unroll
        for (int i = 0; i < TI; ++i) sa[p][i] = lf(dap[i] + 4 * st);
    };
    // Ring slot p to LDS buffer buf (this wavefront alone reads it back).
    auto stage = [&](int p, int buf) {
        *(i32x4 *)&wl[buf][lr * RS + lc * 16] = wr[p][0];
        *(i32x4 *)&wl[buf][(lr + 8) * RS + lc * 16] = wr[p][1];
#pragma unroll
        for (int h = 0; h < 2 * TI; ++h) *(i32x4 *)&al[buf][(lr + 8 * h) * RS + lc * 16] = ar[p][h];
        swl[buf][lane >> 2][lane & 3] = sw[p];
#pragma unroll
        for (int i = 0; i < TI; ++i) sal[buf][lane & 3][(lane >> 2) + 16 * i] = sa[p][i];
    };
    f32x4 acc[TI];
#pragma unroll
    for (int i = 0; i < TI; ++i) acc[i] = f32x4{};
#pragma unroll
    for (int p = 0; p < D; ++p) load(p, min(p, steps - 1), true);
    stage(0, 0);
    load(0, min(D, steps - 1), false);
    // Step st is computed from LDS buffer st&1 while step st+1 is staged
    // into the other one, so the LDS round trip of a step overlaps the MFMAs
    // and scale-accumulates of the one before.
    for (int s0 = 0; s0 < steps; s0 += D) {
#pragma unroll
        for (int p = 0; p < D; ++p) {
            const int st = s0 + p, cur = p & 1;  // D is even, so st&1 == p&1
            const int pn = (p + 1) % D;
            stage(pn, cur ^ 1);
            load(pn, min(st + 1 + D, steps - 1), false);
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const long wv = *(const long *)&wl[cur][c * RS + 32 * b + 8 * g];
                const float w1 = swl[cur][c][b];
#pragma unroll
                for (int i = 0; i < TI; ++i) {
                    const long av = *(const long *)&al[cur][(16 * i + c) * RS + 32 * b + 8 * g];
                    const i32x4 d = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, wv, i32x4{}, 0, 0, 0);
                    const float4 s4 = *(const float4 *)&sal[cur][b][16 * i + 4 * g];
                    const float s_[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[i][e] = __builtin_fmaf((float)d[e], __fmul_rn(s_[e], w1), acc[i][e]);
                }
            }
            __builtin_amdgcn_wave_barrier();
            if (st + 1 >= steps) break;
        }
    }
    const int col = n0 + c;
    if (col < a.n) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = 16 * i + 4 * g + e;
                if (row < a.m) a.y[(size_t)row * a.n + col] = acc[i][e];
            }
    }
}

// M = 1, K = 1024 KS: one wavefront per RG weight rows, streamed as whole
// rows (lane l takes bytes 16 l..+16 of each 1 KiB segment, so a load
// instruction covers 1 KiB of one row), RB rows of loads per batch and up to
// 128 VGPRs of them in flight (at K = 4096 all four rows at once). A row's
// block products are two lanes' sdot4 chains (exact int32) added by a lane
// swap; float(dot_b) and the scale product da[b] * dw[r][b] go to LDS, formed
// by the lanes that hold them, and once the RG rows are in, lane r runs
// output r's chain in block order, acc = fmaf(float(dot_b), da[b] * dw[r][b],
// acc): the same arithmetic as the tiled kernels, so the same bits. Measured
// on MI355X at config 2's shape (K = 4096, N = 12288, 56.6 MB a launch):
// 12.9-13.0 us with 4 rows per wavefront (3072 wavefronts), 13.2 with 8,
// 14.1 with 16, 13.4 with 2, against 19.3-19.8 us for q8b_small_kernel, whose
// wavefronts read 128 bytes of 16 rows per step.
template <int KS, int RG>
__global__ __launch_bounds__(64) void q8b_gemv_kernel(const Q8bArgs a) {
    constexpr int KB = 32 * KS;                                  // blocks per row
    constexpr int RB0 = KS >= 16 ? 1 : 16 / KS;
    constexpr int RB = RB0 < RG ? RB0 : RG;                      // rows per batch (RB * KS 16-byte loads)
    constexpr int NB = RG / RB;                                  // batches
    constexpr int NBUF0 = 32 / (RB * KS) > 0 ? 32 / (RB * KS) : 1;  // at most 128 VGPRs of codes in flight
    constexpr int NBUF = NB < NBUF0 ? NB : NBUF0;                // batches in flight
    static_assert(NB * RB == RG, "whole batches");
    constexpr int SPL = KB / 64;            // scale floats per lane and row
    static_assert(KS % 2 == 0 && KS <= 16, "whole 64-lane scale rows");
    __shared__ float dots[RG][KB + 1];      // float(dot); +1: lane r's chain reads stride KB + 1 words
    __shared__ float sw[RG][KB + 1];
    const int lane = threadIdx.x;
    const int n0 = blockIdx.x * RG;
    // The activation row: lane l's bytes of each segment, then its scales.
    i32x4 xa[KS];
#pragma unroll
    for (int j = 0; j < KS; ++j) xa[j] = *(const i32x4 *)(a.qa + 1024 * j + 16 * lane);
    i32x4 wr[NBUF][RB][KS];
    float sr[NBUF][RB][SPL];
    auto load = [&](int buf, int bt) {
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int row = min(n0 + bt * RB + r, a.n - 1);
            const int8_t *wp = a.qw + (size_t)row * a.k + 16 * lane;
#pragma unroll
            for (int j = 0; j < KS; ++j) wr[buf][r][j] = __builtin_nontemporal_load((const i32x4 *)(wp + 1024 * j));
            const float *sp = a.dw + (size_t)row * KB + SPL * lane;
#pragma unroll
            for (int i = 0; i < SPL; ++i) sr[buf][r][i] = sp[i];
        }
    };
#pragma unroll
    for (int b = 0; b < NBUF; ++b) load(b, b);
    float dar[SPL];  // the activation's block scales of this lane's scale slots
#pragma unroll
    for (int i = 0; i < SPL; ++i) dar[i] = a.da[SPL * lane + i];
#pragma unroll
    for (int bt = 0; bt < NB; ++bt) {
        const int buf = bt % NBUF;
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int rr = bt * RB + r;
#pragma unroll
            for (int j = 0; j < KS; ++j) {
                int d = __builtin_amdgcn_sdot4(wr[buf][r][j][0], xa[j][0], 0, false);
                d = __builtin_amdgcn_sdot4(wr[buf][r][j][1], xa[j][1], d, false);
                d = __builtin_amdgcn_sdot4(wr[buf][r][j][2], xa[j][2], d, false);
                d = __builtin_amdgcn_sdot4(wr[buf][r][j][3], xa[j][3], d, false);
                // Lanes 2t and 2t + 1 hold the halves of block 32 j + t.
                d += __builtin_amdgcn_mov_dpp(d, 0xB1, 0xF, 0xF, true);  // quad_perm [1,0,3,2]
                if (!(lane & 1)) dots[rr][32 * j + (lane >> 1)] = (float)d;
            }
            // The chain's scale products da[b] * dw[r][b], formed here in parallel.
#pragma unroll
            for (int i = 0; i < SPL; ++i) sw[rr][SPL * lane + i] = __fmul_rn(dar[i], sr[buf][r][i]);
        }
        if (bt + NBUF < NB) load(buf, bt + NBUF);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < RG && n0 + lane < a.n) {
        float acc = 0.0f;
#pragma unroll 8
        for (int b = 0; b < KB; ++b) acc = __builtin_fmaf(dots[lane][b], sw[lane][b], acc);
        a.y[n0 + lane] = acc;
    }
}

template <int KS, int RG = 4>
int go_gemv(const Q8bArgs &a, hipStream_t st) {
    hipLaunchKernelGGL((q8b_gemv_kernel<KS, RG>), dim3((unsigned)((a.n + RG - 1) / RG)), dim3(64), 0, st, a);
    return launch_status();
}

template <int TI, int D>
int go_small(const Q8bArgs &a, hipStream_t st) {
    hipLaunchKernelGGL((q8b_small_kernel<TI, D>), dim3((unsigned)((a.n + 15) / 16)), dim3(64), 0, st, a);
    return launch_status();
}

// Ring depth 8 steps for one activation tile, 4 for two (registers).
template <int TI>
int launch_small(const Q8bArgs &a, hipStream_t st) {
    return go_small<TI, TI == 1 ? 8 : 4>(a, st);
}

template <int BM, int BN, int WGM, int WGN, int KSB>
int launch_q8b(Q8bArgs a, hipStream_t st) {
    a.gridM = (a.m + BM - 1) / BM;
    a.gridN = (a.n + BN - 1) / BN;
    hipLaunchKernelGGL((q8b_gemm_kernel<BM, BN, WGM, WGN, KSB>), dim3((unsigned)(a.gridM * a.gridN)),
                       dim3(64 * WGM * WGN), 0, st, a);
    return launch_status();
}

}  // namespace

extern "C" {

int gphq_q8b_quantize(const float *x_dev, int64_t rows, int64_t k, int64_t x_stride, int8_t *q_dev, float *d_dev,
                      void *stream) {
    if (rows < 0 || k < 0 || k % 32 || x_stride < k || x_stride % 4 || rows > INT32_MAX || k > INT32_MAX)
        return GPHQ_ERR_DIMENSIONS;
    if (rows == 0 || k == 0) return GPHQ_OK;
    if (!x_dev || !q_dev || !d_dev) return GPHQ_ERR_DIMENSIONS;
    const long items = (long)rows * (k / 32);
    hipLaunchKernelGGL(q8b_quantize_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       x_dev, (int)rows, (int)k, (long)x_stride, q_dev, d_dev);
    return launch_status();
}

int gphq_q8b_gemm(const int8_t *qa_dev, const float *da_dev, const int8_t *qw_dev, const float *dw_dev, float *y_dev,
                  int64_t m, int64_t k, int64_t n, void *stream) {
    if (m < 0 || k < 0 || n < 0 || k % 32 || m > INT32_MAX || k > INT32_MAX || n > INT32_MAX)
        return GPHQ_ERR_DIMENSIONS;
    if (m == 0 || n == 0) return GPHQ_OK;
    if (!qa_dev || !da_dev || !qw_dev || !dw_dev || !y_dev) return GPHQ_ERR_DIMENSIONS;
    if (k == 0) return fill_f32(y_dev, (size_t)m * n, 0.0f, (hipStream_t)stream);
    Q8bArgs a{qa_dev, da_dev, qw_dev, dw_dev, y_dev, (int)m, (int)k, (int)n, 0, 0};
    hipStream_t st = (hipStream_t)stream;
    // Shapes measured on MI355X at K = 4096, N = 12288: from M = 256,
    // 128 x 192 tiles of eight wavefronts (one per CU at M = 512); from
    // M = 33, 64 x 64 tiles with 256-byte K steps; one row at K = 2048, 4096,
    // 8192 or 12288, whole weight rows streamed per wavefront; otherwise up
    // to 32 rows (k a multiple of 128), one wavefront per 16 weight rows with
    // a ring of steps in flight.
    if (m >= 256) return launch_q8b<128, 192, 4, 2, 4>(a, st);
    if (m > 32) return launch_q8b<64, 64, 2, 2, 8>(a, st);
    if (k % 128) return launch_q8b<64, 64, 2, 2, 4>(a, st);
    if (m == 1) {
        switch (k) {
        case 2048: return go_gemv<2>(a, st);
        case 4096: return go_gemv<4>(a, st);
        case 8192: return go_gemv<8>(a, st);
        case 12288: return go_gemv<12>(a, st);
        }
    }
    if (m > 16) return launch_small<2>(a, st);
    return launch_small<1>(a, st);
}

}  // extern "C"
