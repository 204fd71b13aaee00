// int8 x int8 GEMM with exact int32 accumulation (q8gemm MulPanelsI8 /
// MulStripsI8 semantics, q8gemm/int8.go:170-253):
//   dst[m*stride + n] = (float32(sum_k qa[m,k]*qw[n,k]) * colScale[n]) * rowScale[m]
// and the per-row activation quantizer of WorkspaceI8 (int8.go:100-168).
//
// Device layout ("tile layout"): an R x K int8 matrix is stored as
// [ceil(R/16)][ceil(K/64)][64 lanes][16 bytes]; lane l of group (rt, kt) holds
// row rt*16 + l%16, columns kt*64 + (l/16)*16 .. +16. One 1 KiB group is one
// operand fragment of v_mfma_i32_16x16x64_i8 for both A (rows = activation
// rows) and B (rows = weight rows / output columns), so every fragment load is
// a single contiguous 1 KiB wavefront load. Padding (rows past R, K past the
// logical K) is zero in the weights, so padded K never changes a sum.
//
// GEMM: a block is WM x WN x SK wavefronts; wavefront (wm, wn, ks) owns a
// (16*TM) x (16*TN) output tile and the ks-th slice of the K tiles. It loads
// U K-steps of A and B fragments straight from HBM/L2 into registers, then
// issues TM*TN MFMAs per step. With SK > 1 the int32 partial tiles are added
// in LDS (exact, so any split gives identical bits). The epilogue converts
// int32 -> fp32 (round to nearest even, like Go's float32(int32)) and applies
// the two scale multiplies in the reference's order. Blocks are renumbered so
// that consecutive blocks on one XCD share a weight column tile, which is then
// read from HBM once into that XCD's L2.
#include "common.h"

namespace gphq {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

__host__ __device__ inline size_t tile_offset(long r, long k, long kt) {
    return ((size_t)(r >> 4) * kt + (k >> 6)) * 1024 + (size_t)((((k & 63) >> 4) << 4) + (r & 15)) * 16 + (k & 15);
}

// The batched pass's int8 activations ("row tiles"): the same 1 KiB groups of
// 16 rows x 64 bytes, each row's 64 bytes contiguous inside the group, so a
// row-at-a-time packer writes 64-byte pieces. The direct-to-LDS GEMM gathers
// a group into the tile layout's lane order within its own 1 KiB.
__host__ __device__ inline size_t rowtile_offset(long r, long k, long kt) {
    return ((size_t)(r >> 4) * kt + (k >> 6)) * 1024 + (size_t)(r & 15) * 64 + (k & 63);
}

// ---- weight packing: row-major int8 [rows][K] -> tile layout ---------------
// One thread per 16-byte lane chunk of the destination; rows past `rows`
// (inside the last 16-row tile) and K padding are written as zero.
__global__ void i8_pack_tiles_kernel(const int8_t *__restrict__ src, int8_t *__restrict__ dst, int rows, int K,
                                     int row0, int rowTiles, int kt) {
    const size_t chunk = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // 16-byte chunk index
    const size_t total = (size_t)rowTiles * kt * 64;
    if (chunk >= total) return;
    const int lane = (int)(chunk & 63);
    const size_t g = chunk >> 6;
    const int ktile = (int)(g % kt);
    const int rtile = (int)(g / kt) + (row0 >> 4);
    const int r = rtile * 16 + (lane & 15);  // absolute row
    const int kbase = ktile * 64 + (lane >> 4) * 16;
    int8_t v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int k = kbase + i;
        const int rr = r - row0;
        v[i] = (rr >= 0 && rr < rows && k < K) ? src[(size_t)rr * K + k] : (int8_t)0;
    }
    int8_t *d = dst + ((size_t)rtile * kt + ktile) * 1024 + (size_t)lane * 16;
    // Rows outside [row0, row0+rows) of a shared tile keep their bytes.
    const int rr = r - row0;
    if (rr >= 0 && rr < rows) {
#pragma unroll
        for (int i = 0; i < 16; ++i) d[i] = v[i];
    }
}

// ---- activation quantizer ---------------------------------------------------
// Workspace Pack fused: per row (one block each), MaxAbs with NaN propagation
// (gemm.go:138-150), SetRowScale, then quantize every column into the tile
// layout (and zero the row's K padding).
__global__ __launch_bounds__(256) void i8_pack_rows_kernel(const float *__restrict__ x, long stride, int K, int kt,
                                                           int8_t *__restrict__ act, float *__restrict__ rowScale,
                                                           float *__restrict__ rowInv) {
    __shared__ float smax[4];
    __shared__ int snan[4];
    const int row = blockIdx.x;
    const float *xr = x + (size_t)row * stride;
    float m = 0.0f;
    int nan = 0;
    // Eight independent loads per thread per trip, so a row's reads are in
    // flight together instead of one L2 round trip after another.
    constexpr int UNR = 8;
    for (int k0 = 0; k0 < K; k0 += 256 * UNR) {
        float v[UNR];
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int k = k0 + u * 256 + (int)threadIdx.x;
            v[u] = k < K ? xr[k] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            nan |= (v[u] != v[u]);
            m = fmaxf(m, fabsf(v[u]));
        }
    }
    // wave max / nan-any
    for (int off = 32; off > 0; off >>= 1) {
        m = fmaxf(m, __shfl_xor(m, off));
        nan |= __shfl_xor(nan, off);
    }
    const int wv = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        smax[wv] = m;
        snan[wv] = nan;
    }
    __syncthreads();
    float mm = 0.0f;
    int anyNan = 0;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) {
        mm = fmaxf(mm, smax[i]);
        anyNan |= snan[i];
    }
    if (anyNan) mm = __builtin_nanf("");
    float scale, inv;
    i8_row_scale(mm, scale, inv);
    if (threadIdx.x == 0) {
        rowScale[row] = scale;
        rowInv[row] = inv;
    }
    // Quantize: each thread takes 16 consecutive columns (one 16-byte lane
    // chunk of the tile layout) and stores them with one 128-bit write.
    for (int c = threadIdx.x; c < kt * 4; c += blockDim.x) {
        const int kb = c * 16;
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t packed = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int k = kb + 4 * j + i;
                const int8_t q = k < K ? quantize_i8(__fmul_rn(xr[k], inv)) : (int8_t)0;
                packed |= (uint32_t)(uint8_t)q << (8 * i);
            }
            w[j] = packed;
        }
        *(uint4 *)(act + tile_offset(row, kb, kt)) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// The same Pack for K a multiple of 16 and 16-byte aligned rows: the row is
// read once, as 16-byte pieces, into registers (CPT chunks of 16 values per
// thread, thread t holding columns 16 (t + 256 c) .. + 15, the chunks past K
// zero), reduced for MaxAbs, and quantized from the registers. Rows with a
// finite positive 127/max quantize without quantize_i8's NaN test (rint,
// v_med3 clamp, v_perm byte packing); the others take quantize_i8 itself: the
// same bytes either way. The 8 rows whose 16-byte pieces share a 128-byte line
// of the tile layout (rows 8q .. 8q + 7) go to blocks b, b + 8, .., b + 56,
// which the dispatcher places on one XCD (round robin over 8), so each line is
// completed in one L2.
template <int CPT>
__global__ __launch_bounds__(256) void i8_pack_rows_vec_kernel(const float *__restrict__ x, long stride, int K,
                                                               int kt, int8_t *__restrict__ act,
                                                               float *__restrict__ rowScale,
                                                               float *__restrict__ rowInv, int rows) {
    __shared__ float smx[4];
    __shared__ int snan[4];
    const int bx = blockIdx.x, row = (bx & ~63) + 8 * (bx & 7) + ((bx >> 3) & 7);
    if (row >= rows) return;
    float4 v[CPT][4];
    load_row_chunks<CPT>(v, x + (size_t)row * stride, K);
    zero_past_end<CPT>(v, K);
    float mx = 0.0f;
    int nan = 0;
#pragma unroll
    for (int c = 0; c < CPT; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            mx = fmaxf(fmaxf(fmaxf(mx, fabsf(v[c][q].x)), fmaxf(fabsf(v[c][q].y), fabsf(v[c][q].z))), fabsf(v[c][q].w));
            nan |= (v[c][q].x != v[c][q].x) | (v[c][q].y != v[c][q].y) | (v[c][q].z != v[c][q].z) |
                   (v[c][q].w != v[c][q].w);
        }
    for (int off = 32; off > 0; off >>= 1) {
        mx = fmaxf(mx, __shfl_xor(mx, off));
        nan |= __shfl_xor(nan, off);
    }
    if ((threadIdx.x & 63) == 0) {
        smx[threadIdx.x >> 6] = mx;
        snan[threadIdx.x >> 6] = nan;
    }
    __syncthreads();
    float m = fmaxf(fmaxf(smx[0], smx[1]), fmaxf(smx[2], smx[3]));
    if (snan[0] | snan[1] | snan[2] | snan[3]) m = __builtin_nanf("");
    float scale, inv;
    i8_row_scale(m, scale, inv);
    if (threadIdx.x == 0) {
        rowScale[row] = scale;
        rowInv[row] = inv;
    }
    const bool plain = inv > 0.0f && inv < INFINITY;  // the same for the whole block
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int kb = 16 * ((int)threadIdx.x + 256 * c);
        if (kb >= kt * 64) continue;
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float e[4] = {v[c][q].x, v[c][q].y, v[c][q].z, v[c][q].w};
            if (plain) {
                int b[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    b[i] = (int)__builtin_amdgcn_fmed3f(rintf(__fmul_rn(e[i], inv)), -128.0f, 127.0f);
                w[q] = __builtin_amdgcn_perm((uint32_t)b[1], (uint32_t)b[0], 0x0c0c0400u) |
                       __builtin_amdgcn_perm((uint32_t)b[3], (uint32_t)b[2], 0x04000c0cu);
            } else {
                uint32_t packed = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) packed |= (uint32_t)(uint8_t)quantize_i8(__fmul_rn(e[i], inv)) << (8 * i);
                w[q] = packed;
            }
        }
        *(uint4 *)(act + tile_offset(row, kb, kt)) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// PackRange (int8.go:116-163) with row scales already set: quantize columns
// [k0, k1) of every prepared row; k1 == K also zeroes the K padding.
__global__ __launch_bounds__(256) void i8_pack_range_kernel(const float *__restrict__ x, long stride, int K, int kt,
                                                            int k0, int k1, int8_t *__restrict__ act,
                                                            const float *__restrict__ rowInv) {
    const int row = blockIdx.x;
    const float inv = rowInv[row];
    const float *xr = x + (size_t)row * stride;
    const int kend = (k1 == K) ? kt * 64 : k1;
    for (int k = k0 + threadIdx.x; k < kend; k += blockDim.x) {
        const int8_t q = k < K ? quantize_i8(__fmul_rn(xr[k], inv)) : (int8_t)0;
        act[tile_offset(row, k, kt)] = q;
    }
}

// The qwen3lm batched pass's int8 activations, the CPU provider's int8 route
// (qwen3lm/ops.go:96-147: the row is normalized, SetRowScale(MaxAbs), then
// PackRange) over the GPU layer formats: per row v = x * f with f the RMSNorm
// factor (MODE 2, the FP16 packer's sum order) or 1 (MODE 1); SetRowScale of
// max|v| (NaN-propagating); q = quantize(v * inv) written as row tiles
// (rowtile_offset, K a multiple of 64); rowScale[r] = max / 127. One block per row, the row in
// registers (CPT chunks of 16 values per thread). ROT first rotates the row
// as the down projection's input (the online Hadamard, gpu.metal:339-367;
// the CPU path's scaleRow, qwen3lm/ops.go:111-122): x * signs (signs carry
// the 1/sqrt(block) scale), then the butterfly network of each block in LDS
// (K floats of dynamic LDS), the same arithmetic as the decode step's
// rotation kernel.
template <int MODE, int CPT, bool ROT>
__global__ __launch_bounds__(256) void i8_act_rows_kernel(const float *__restrict__ x, long stride, int K, float eps,
                                                          const float *__restrict__ signs, int block,
                                                          int8_t *__restrict__ act, float *__restrict__ rowScale,
                                                          int rows) {
    __shared__ float sss[4], smx[4];
    __shared__ int snan[4];
    // The 2 rows whose 64-byte pieces share a 128-byte line of the row tiles
    // go to blocks b and b + 8, which the dispatcher places on one XCD (round
    // robin over 8), so each line is completed in one L2.
    const int bx = blockIdx.x, row = (bx & ~15) + 2 * (bx & 7) + ((bx >> 3) & 1);
    if (row >= rows) return;
    const float *xr = x + (size_t)row * stride;
    float4 v[CPT][4];
    float ss = 0.0f, mx = 0.0f;
    int nan = 0;
    float4 sg[4];
    if constexpr (ROT) {
        rot_signs(sg, signs, 16 * (int)threadIdx.x, K);
        __builtin_amdgcn_sched_barrier(0);  // the signs are requested first
    }
    load_row_chunks<CPT>(v, xr, K);
    if constexpr (ROT) rotate_row_lds<CPT>(v, sg, K, signs, block);
    zero_past_end<CPT>(v, K);
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if constexpr (MODE == 2)
                ss += v[c][q].x * v[c][q].x + v[c][q].y * v[c][q].y + v[c][q].z * v[c][q].z + v[c][q].w * v[c][q].w;
            mx = fmaxf(fmaxf(fmaxf(mx, fabsf(v[c][q].x)), fmaxf(fabsf(v[c][q].y), fabsf(v[c][q].z))), fabsf(v[c][q].w));
            nan |= (v[c][q].x != v[c][q].x) | (v[c][q].y != v[c][q].y) | (v[c][q].z != v[c][q].z) |
                   (v[c][q].w != v[c][q].w);
        }
    }
    if constexpr (MODE == 2) ss = wave_sum(ss);
    for (int off = 32; off > 0; off >>= 1) {
        mx = fmaxf(mx, __shfl_xor(mx, off));
        nan |= __shfl_xor(nan, off);
    }
    if ((threadIdx.x & 63) == 0) {
        sss[threadIdx.x >> 6] = ss;
        smx[threadIdx.x >> 6] = mx;
        snan[threadIdx.x >> 6] = nan;
    }
    __syncthreads();
    const float f = MODE == 2 ? 1.0f / sqrtf(((sss[0] + sss[1]) + (sss[2] + sss[3])) / (float)K + eps) : 1.0f;
    // max |x * f| is (max |x|) * f: rounding is monotonic.
    float m = __fmul_rn(fmaxf(fmaxf(smx[0], smx[1]), fmaxf(smx[2], smx[3])), f);
    if (snan[0] | snan[1] | snan[2] | snan[3]) m = __builtin_nanf("");
    float scale, inv;
    i8_row_scale(m, scale, inv);
    if (threadIdx.x == 0) rowScale[row] = scale;
    // A row with a finite, nonzero 127/max has only finite products, so
    // quantize_i8's NaN test can go: rint, clamp (v_med3) and convert, the
    // four bytes packed by v_perm. Other rows (NaN, infinite, zero or
    // denormal-range maxima) take quantize_i8 itself. The same bytes either way.
    const bool plain = inv > 0.0f && inv < INFINITY;  // the same for the whole block
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int k = 16 * ((int)threadIdx.x + 256 * c);
        if (k >= K) continue;
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float e[4] = {v[c][q].x, v[c][q].y, v[c][q].z, v[c][q].w};
            if (plain) {
                int b[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float y = MODE == 2 ? __fmul_rn(e[i], f) : e[i];
                    b[i] = (int)__builtin_amdgcn_fmed3f(rintf(__fmul_rn(y, inv)), -128.0f, 127.0f);
                }
                w[q] = __builtin_amdgcn_perm((uint32_t)b[1], (uint32_t)b[0], 0x0c0c0400u) |
                       __builtin_amdgcn_perm((uint32_t)b[3], (uint32_t)b[2], 0x04000c0cu);
            } else {
                uint32_t packed = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float y = MODE == 2 ? __fmul_rn(e[i], f) : e[i];
                    packed |= (uint32_t)(uint8_t)quantize_i8(__fmul_rn(y, inv)) << (8 * i);
                }
                w[q] = packed;
            }
        }
        *(uint4 *)(act + rowtile_offset(row, k, K >> 6)) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// ---- GEMM ------------------------------------------------------------------
struct I8GemmArgs {
    const int8_t *A;      // activations, tile layout, MT x KT groups (row tiles for the batched pass)
    const int8_t *B;      // weights, tile layout, NT x KT groups (row-major [N][K] for the batched pass)
    const float *rowScale;  // [M]
    const float *colScale;  // [N]
    float *dst;
    long stride;
    int M, N, KT, NT;
    int c0, c1;  // output columns [c0, c1)
    int tileN0;  // first 16-column tile covered by the grid
    int gridM, gridN;  // blocks along M and N
    int K;             // row length in bytes of row-major weights (a multiple of 64)
};

// Operand layouts and epilogues of the big-tile kernel.
enum { I8_EPI_STORE = 0, I8_EPI_ADD = 1, I8_EPI_SWIGLU = 2 };

template <int TM, int TN, int WM, int WN, int SK, int U>
__global__ __launch_bounds__(64 * WM * WN * SK) void i8gemm_kernel(const I8GemmArgs a) {
    constexpr int NW = WM * WN * SK;
    __shared__ i32x4 red[(SK > 1) ? (NW * TM * TN * 64) : 1];
    // XCD-aware renumbering: hardware places block b on XCD b % 8. Give the
    // blocks of one XCD consecutive logical ids, M fastest, so they share
    // weight column tiles.
    const int G = a.gridM * a.gridN;
    const int b = blockIdx.x;
    int logical = b;
    if (G % 8 == 0) logical = (b % 8) * (G / 8) + b / 8;
    const int bm = logical % a.gridM, bn = logical / a.gridM;

    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int ks = wv % SK;
    const int wn = (wv / SK) % WN;
    const int wm = wv / (SK * WN);
    const int mt0 = (bm * WM + wm) * TM;                      // first 16-row tile
    const int nt0 = a.tileN0 + (bn * WN + wn) * TN;           // first 16-col tile
    const int MT = (a.M + 15) >> 4;
    const int KT = a.KT;
    const int per = (KT + SK - 1) / SK;
    const int kt0 = ks * per, kt1 = min(KT, kt0 + per);

    size_t aoff[TM], boff[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) aoff[i] = (size_t)min(mt0 + i, MT - 1) * KT * 1024 + (size_t)lane * 16;
#pragma unroll
    for (int j = 0; j < TN; ++j) boff[j] = (size_t)min(nt0 + j, a.NT - 1) * KT * 1024 + (size_t)lane * 16;

    i32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = i32x4{0, 0, 0, 0};

    // Two register buffers: the fragments of batch b+1 are requested before the
    // MFMAs of batch b, so memory latency overlaps the matrix work. Fragments
    // past the slice end are zero and add nothing.
    auto load = [&](i32x4 (&fa)[U][TM], i32x4 (&fb)[U][TN], int kt) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const bool ok = kt + u < kt1;
            const size_t ko = (size_t)(kt + u) * 1024;
#pragma unroll
            for (int i = 0; i < TM; ++i)
                fa[u][i] = ok ? *(const i32x4 *)(a.A + aoff[i] + ko) : i32x4{0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < TN; ++j)
                fb[u][j] = ok ? __builtin_nontemporal_load((const i32x4 *)(a.B + boff[j] + ko)) : i32x4{0, 0, 0, 0};
        }
    };
    auto mma = [&](const i32x4 (&fa)[U][TM], const i32x4 (&fb)[U][TN]) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[u][i], fb[u][j], acc[i][j], 0, 0, 0);
    };
    i32x4 fa0[U][TM], fb0[U][TN], fa1[U][TM], fb1[U][TN];
    int kt = kt0;
    if (kt < kt1) load(fa0, fb0, kt);
    while (kt < kt1) {
        if (kt + U < kt1) load(fa1, fb1, kt + U);
        mma(fa0, fb0);
        kt += U;
        if (kt >= kt1) break;
        if (kt + U < kt1) load(fa0, fb0, kt + U);
        mma(fa1, fb1);
        kt += U;
    }

    if constexpr (SK > 1) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) red[((wv * TM + i) * TN + j) * 64 + lane] = acc[i][j];
        __syncthreads();
        if (ks != 0) return;
#pragma unroll
        for (int s = 1; s < SK; ++s)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] += red[(((wv + s) * TM + i) * TN + j) * 64 + lane];
    }

    // Epilogue. Lane l of a 16x16 output tile holds rows 4*(l/16)+e, column
    // l%16. The scales are read first, unconditionally (clamped indices;
    // outputs outside the matrix are not written): scales read between
    // stores would each wait for the stores too.
    float rsc[TM][4], csc[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) rsc[i][e] = a.rowScale[min((mt0 + i) * 16 + 4 * (lane >> 4) + e, a.M - 1)];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int col = (nt0 + j) * 16 + (lane & 15);
        csc[j] = a.colScale[col >= a.c0 && col < a.c1 ? col : a.c0];
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int col = (nt0 + j) * 16 + (lane & 15);
        if (col < a.c0 || col >= a.c1) continue;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = (mt0 + i) * 16 + 4 * (lane >> 4) + e;
                if (row < a.M)
                    a.dst[(size_t)row * a.stride + col] = __fmul_rn(__fmul_rn((float)acc[i][j][e], csc[j]), rsc[i][e]);
            }
        }
    }
}

// LDS-staged variant for larger M: a block owns a BM x BN output tile; per
// stage the block copies BKT K-tiles of its A rows and B columns (1 KiB
// fragments, contiguous in the tile layout) from global memory into LDS with
// 16-byte loads, double buffered: the next stage's global loads are in flight
// while the wavefronts multiply the current stage out of LDS. Each fragment
// then crosses the L2 -> CU path once per block instead of once per wavefront.
template <int BM, int BN, int WM, int WN, int BKT>
__global__ __launch_bounds__(64 * WM * WN) void i8gemm_lds_kernel(const I8GemmArgs a) {
    constexpr int NT_ = 64 * WM * WN;
    constexpr int TM = BM / 16 / WM, TN = BN / 16 / WN;
    constexpr int AG = (BM / 16) * BKT, BG = (BN / 16) * BKT;  // 1 KiB groups per stage
    constexpr int CH = (AG + BG) * 64;                          // 16-byte chunks per stage
    constexpr int PER = (CH + NT_ - 1) / NT_;
    __shared__ i32x4 lds[2][AG + BG][64];

    const int G = a.gridM * a.gridN;
    const int b = blockIdx.x;
    int logical = b;
    if (G % 8 == 0) logical = (b % 8) * (G / 8) + b / 8;
    const int bm = logical % a.gridM, bn = logical / a.gridM;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wm = wv / WN, wn = wv % WN;
    const int MT = (a.M + 15) >> 4, KT = a.KT;
    const int rt0 = bm * (BM / 16), ct0 = a.tileN0 + bn * (BN / 16);

    auto fetch = [&](int kt0, i32x4 (&reg)[PER]) {
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int c = tid + p * NT_;
            reg[p] = i32x4{0, 0, 0, 0};
            if (c < CH) {
                const int g = c >> 6, l = c & 63;
                const int kk = (g < AG) ? (g % BKT) : ((g - AG) % BKT);
                const int kt = kt0 + kk;
                if (kt < KT) {
                    if (g < AG) {
                        const int rt = min(rt0 + g / BKT, MT - 1);
                        reg[p] = *(const i32x4 *)(a.A + ((size_t)rt * KT + kt) * 1024 + (size_t)l * 16);
                    } else {
                        const int ct = min(ct0 + (g - AG) / BKT, a.NT - 1);
                        reg[p] = __builtin_nontemporal_load(
                            (const i32x4 *)(a.B + ((size_t)ct * KT + kt) * 1024 + (size_t)l * 16));
                    }
                }
            }
        }
    };
    auto stash = [&](int buf, const i32x4 (&reg)[PER]) {
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int c = tid + p * NT_;
            if (c < CH) lds[buf][c >> 6][c & 63] = reg[p];
        }
    };

    i32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = i32x4{0, 0, 0, 0};

    i32x4 reg[PER];
    fetch(0, reg);
    stash(0, reg);
    __syncthreads();
    int buf = 0;
    for (int kt0 = 0; kt0 < KT; kt0 += BKT) {
        const bool more = kt0 + BKT < KT;
        if (more) fetch(kt0 + BKT, reg);
#pragma unroll
        for (int kk = 0; kk < BKT; ++kk) {
            i32x4 fa[TM], fb[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) fa[i] = lds[buf][(wm * TM + i) * BKT + kk][lane];
#pragma unroll
            for (int j = 0; j < TN; ++j) fb[j] = lds[buf][AG + (wn * TN + j) * BKT + kk][lane];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
        if (more) stash(buf ^ 1, reg);
        __syncthreads();
        buf ^= 1;
    }

    // Scales first, unconditionally, as in i8gemm_kernel's epilogue.
    float rsc[TM][4], csc[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e)
            rsc[i][e] = a.rowScale[min((rt0 + wm * TM + i) * 16 + 4 * (lane >> 4) + e, a.M - 1)];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int col = (ct0 + wn * TN + j) * 16 + (lane & 15);
        csc[j] = a.colScale[col >= a.c0 && col < a.c1 ? col : a.c0];
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int col = (ct0 + wn * TN + j) * 16 + (lane & 15);
        if (col < a.c0 || col >= a.c1) continue;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = (rt0 + wm * TM + i) * 16 + 4 * (lane >> 4) + e;
                if (row < a.M)
                    a.dst[(size_t)row * a.stride + col] = __fmul_rn(__fmul_rn((float)acc[i][j][e], csc[j]), rsc[i][e]);
            }
        }
    }
}

// Skinny-M variant (up to 16 * NWV * RT activation rows per block, one block
// per NTB weight column tiles; KT a multiple of SB). Every
// operand fragment goes to LDS with a direct-to-LDS load
// (global_load_lds_dwordx4: one 1 KiB fragment per wavefront instruction, no
// registers held while in flight) into a ring of NS stages of SB K-steps; the
// stage NS - 1 ahead is requested as each stage starts. Each wavefront owns
// RT row tiles of A and loads their fragments itself; the NTB column tiles of
// B are shared, each wavefront loading an equal share. Loads return in issue
// order, so the wait at a stage's start is a count (the loads of the NS - 2
// stages after it may stay in flight). The barrier is s_barrier with
// compiler-only fences around it (ring_barrier; a __syncthreads fence would
// wait for every load in flight), after lgkmcnt(0)
// so that the previous stage's LDS reads have finished before its slot is
// refilled.
template <int NWV, int RT, int NTB, int SB, int NS>
__global__ __launch_bounds__(64 * NWV) void i8gemm_skinny_kernel(const I8GemmArgs a) {
    constexpr int FB = NTB * SB;           // B fragments per stage
    constexpr int FA = NWV * RT * SB;      // A fragments per stage
    static_assert(FB % NWV == 0, "every wavefront issues the same number of stage loads");
    constexpr int DB = FB / NWV;           // B loads per wavefront and stage
    constexpr int D = DB + RT * SB;        // loads per wavefront and stage
    static_assert(D * (NS - 2) < 64, "in-flight loads beyond the vmcnt range");
    __shared__ i32x4 ring[NS][FB + FA][64];

    const int G = a.gridM * a.gridN;
    const int b = blockIdx.x;
    int logical = b;
    if (G % 8 == 0) logical = (b % 8) * (G / 8) + b / 8;
    const int bm = logical % a.gridM, bn = logical / a.gridM;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int MT = (a.M + 15) >> 4, KT = a.KT;
    const int S = KT / SB;
    const int mt0 = (bm * NWV + wv) * RT;
    const int nt0 = a.tileN0 + bn * NTB;

    // Sources of this wavefront's loads at stage 0, in ring order: its B share
    // (fragment f = wv + NWV * d is column tile f / SB, K-step f % SB), then its
    // own A fragments (row tile i, K-step kk at FB + (wv * RT + i) * SB + kk).
    const int8_t *src[D];
    int dst[D];
#pragma unroll
    for (int d = 0; d < DB; ++d) {
        const int f = wv + NWV * d;
        src[d] = a.B + ((size_t)min(nt0 + f / SB, a.NT - 1) * KT + f % SB) * 1024 + (size_t)lane * 16;
        dst[d] = f;
    }
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int kk = 0; kk < SB; ++kk) {
            const int d = DB + i * SB + kk;
            src[d] = a.A + ((size_t)min(mt0 + i, MT - 1) * KT + kk) * 1024 + (size_t)lane * 16;
            dst[d] = FB + (wv * RT + i) * SB + kk;
        }
    auto stage_load = [&](int s) {
        const int slot = s % NS;
#pragma unroll
        for (int d = 0; d < D; ++d)
            lds_dma16(src[d] + (size_t)s * SB * 1024, &ring[slot][dst[d]][0]);
    };

    i32x4 acc[RT][NTB];
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int j = 0; j < NTB; ++j) acc[i][j] = i32x4{0, 0, 0, 0};

#pragma unroll
    for (int p = 0; p < NS - 1; ++p)
        if (p < S) stage_load(p);
    for (int s = 0; s < S; ++s) {
        // Loads of stages s + 1 .. min(S, s + NS - 1) - 1 may remain in flight.
        const int after = min(S - 1 - s, NS - 2);
        if (after == NS - 2)
            wait_vm_lgkm0<D * (NS - 2)>();
        else if (after == 1)
            wait_vm_lgkm0<D>();
        else
            wait_vm_lgkm0<0>();
        ring_barrier();
        if (s + NS - 1 < S) stage_load(s + NS - 1);
        const int slot = s % NS;
#pragma unroll
        for (int kk = 0; kk < SB; ++kk) {
            i32x4 fa[RT], fb[NTB];
#pragma unroll
            for (int i = 0; i < RT; ++i) fa[i] = ring[slot][FB + (wv * RT + i) * SB + kk][lane];
#pragma unroll
            for (int j = 0; j < NTB; ++j) fb[j] = ring[slot][j * SB + kk][lane];
#pragma unroll
            for (int i = 0; i < RT; ++i)
#pragma unroll
                for (int j = 0; j < NTB; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
    }

    // Epilogue as in i8gemm_kernel: scales first, then the stores.
    float rsc[RT][4], csc[NTB];
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) rsc[i][e] = a.rowScale[min((mt0 + i) * 16 + 4 * (lane >> 4) + e, a.M - 1)];
#pragma unroll
    for (int j = 0; j < NTB; ++j) {
        const int col = (nt0 + j) * 16 + (lane & 15);
        csc[j] = a.colScale[col >= a.c0 && col < a.c1 ? col : a.c0];
    }
#pragma unroll
    for (int j = 0; j < NTB; ++j) {
        const int col = (nt0 + j) * 16 + (lane & 15);
        if (col < a.c0 || col >= a.c1) continue;
#pragma unroll
        for (int i = 0; i < RT; ++i) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = (mt0 + i) * 16 + 4 * (lane >> 4) + e;
                if (row < a.M)
                    a.dst[(size_t)row * a.stride + col] = __fmul_rn(__fmul_rn((float)acc[i][j][e], csc[j]), rsc[i][e]);
            }
        }
    }
}

// Large-M variant: BM x BN block tiles (WGM x WGN wavefronts, each a grid of
// 32 x 32 v_mfma_i32_32x32x32_i8 tiles), 128-deep K steps staged through LDS
// as 128-byte rows with the row-swizzled 16-byte chunks of the FP16 big-tile
// GEMM, double-buffered with the next step's global loads in flight;
// XCD-grouped tile order. Exact int32 sums, so the bits equal the other
// kernels'. Operands come in the tile layout (two 64-deep groups per step).
// Epilogue: (float32(sum) * colScale) * rowScale, stored.
template <int BM, int BN, int WGM, int WGN>
__global__ __launch_bounds__(64 * WGM * WGN) void i8gemm_big_kernel(const I8GemmArgs a) {
    typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
    constexpr int NT = 64 * WGM * WGN;
    constexpr int TI = BM / WGM / 32, TJ = BN / WGN / 32;
    constexpr int AL = BM * 8 / NT, BL = BN * 8 / NT;  // 16-byte units per thread and step
    static_assert(AL >= 1 && BL >= 1, "loader split");
    __shared__ i32x4 As[2][BM * 8];
    __shared__ i32x4 Bs[2][BN * 8];
    int bm, bn;
    tile_order(blockIdx.x, a.gridM, a.gridN, bm, bn);
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int wm = wv / WGN, wn = wv % WGN;
    const int rt0 = bm * (BM / 16), ct0 = a.tileN0 + bn * (BN / 16);
    const int MT = (a.M + 15) >> 4, KT = a.KT;
    const int steps = (KT + 1) / 2;
    // Unit u = i*NT + t of a step is 16-row tile u/128, group (u/64)%2 of the
    // step, lane slot u%64 (row slot%16, K bytes 16*(slot/16) of the group).
    auto gload = [&](const int8_t *base, int tile0, int tiles, int u, int st) {
        i32x4 v = i32x4{0, 0, 0, 0};
        const int kt = 2 * st + ((u >> 6) & 1);
        if (kt < KT)
            v = *(const i32x4 *)(base + ((size_t)min(tile0 + (u >> 7), tiles - 1) * KT + kt) * 1024 +
                                 (size_t)(u & 63) * 16);
        return v;
    };
    auto lidx = [](int u) {
        const int r = (u >> 7) * 16 + (u & 15);
        return r * 8 + big_swz(r, ((u >> 6) & 1) * 4 + ((u & 63) >> 4));
    };
    const int aRows = MT, bRows = a.NT;
    i32x4 ar[AL], br[BL];
    auto load = [&](int st) {
#pragma unroll
        for (int i = 0; i < AL; ++i) ar[i] = gload(a.A, rt0, aRows, i * NT + t, st);
#pragma unroll
        for (int i = 0; i < BL; ++i) br[i] = gload(a.B, ct0, bRows, i * NT + t, st);
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < AL; ++i) As[buf][lidx(i * NT + t)] = ar[i];
#pragma unroll
        for (int i = 0; i < BL; ++i) Bs[buf][lidx(i * NT + t)] = br[i];
    };
    i32x16 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = i32x16{};
    load(0);
    store(0);
    if (steps > 1) load(1);
    __syncthreads();
    const int fr = lane & 31, fh = lane >> 5;
    // With two wavefronts per SIMD (8 per block), the second wavefront of each
    // SIMD stores the next step's tiles before its MFMAs and the first after
    // them, so the SIMD's MFMA pipe is fed by one while the other stores
    // (measured: M = 512, 54 -> 52 us).
    const bool early = NT >= 512 && wv >= NT / 128;
    for (int st = 0; st < steps; ++st) {
        const int cur = st & 1;
        if (early && st + 1 < steps) {
            store(cur ^ 1);
            if (st + 2 < steps) load(st + 2);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int c = 2 * s + fh;
            i32x4 fa[TI], fb[TJ];
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                const int r = wm * (32 * TI) + 32 * i + fr;
                fa[i] = As[cur][r * 8 + big_swz(r, c)];
            }
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const int r = wn * (32 * TJ) + 32 * j + fr;
                fb[j] = Bs[cur][r * 8 + big_swz(r, c)];
            }
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
        if (!early && st + 1 < steps) {
            store(cur ^ 1);
            if (st + 2 < steps) load(st + 2);
        }
        __syncthreads();
    }
    // Epilogue as MulPanelsI8: (float32(sum) * colScale) * rowScale. Every
    // scale of the lane's outputs is read up front, unconditionally (rows past
    // M read the last row; they are not written): read inside the store loop,
    // or under a branch, each scale costs a wait, and the wait also drains
    // every store issued before it (stores may alias the scales as far as the
    // compiler knows, and the counter it waits on counts stores too).
    float rsc[TI][16];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e)
            rsc[i][e] = a.rowScale[min((rt0 + (wm * TI + i) * 2) * 16 + 8 * (e >> 2) + 4 * fh + (e & 3), a.M - 1)];
    // The column scales too (a column outside [c0, c1) reads c0's and is not
    // written): a load after a store waits for the store as well.
    float csc[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const int col = (ct0 + (wn * TJ + j) * 2) * 16 + fr;
        csc[j] = a.colScale[col >= a.c0 && col < a.c1 ? col : a.c0];
    }
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const int col = (ct0 + (wn * TJ + j) * 2) * 16 + fr;
        if (col < a.c0 || col >= a.c1) continue;
        const float cs = csc[j];
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = (rt0 + (wm * TI + i) * 2) * 16 + 8 * (e >> 2) + 4 * fh + (e & 3);
                if (row < a.M)
                    a.dst[(size_t)row * a.stride + col] = __fmul_rn(__fmul_rn((float)acc[i][j][e], cs), rsc[i][e]);
            }
    }
}

// Epilogue of the direct-to-LDS kernels, as in i8gemm_kernel: lane l of a
// 16 x 16 tile holds rows 4 (l / 16) + e, column l % 16; scales first, then
// the stores. mt0 / nt0: the wavefront's first row and column tile.
// Measured on MI355X (config 2, M = 512): stores of 16 columns per row wrote
// 1.32x the output's bytes to HBM (WRITE_SIZE); whole 128-byte lines write
// them once.
// The stores of dma_epilogue with the column-tile pairs starting at tile P
// of the wavefront (P = nt0 % 2, so that each pair's 32 columns are one
// 128-byte line of every row): v_permlane16_swap exchanges lanes 16-31 of
// tile j's values with lanes 0-15 of tile j + 1's (and 48-63 with 32-47), so
// each store covers 32 consecutive columns of two rows (two whole 128-byte
// lines) instead of 16 columns of four rows. After the swap, lane l holds
// column (j + bit 4 of l) * 16 + l % 16; the first value is row 8 (l / 32) + e,
// the second row 4 more. The tiles left out of the pairs (the first when P is
// 1, an odd last one) are stored as they are, and their half lines meet the
// neighbouring wavefront's in L2.
template <int TI, int TJ, int EPI, int P>
__device__ __forceinline__ void dma_epilogue_stores(const I8GemmArgs &a, const i32x4 (&acc)[TI][TJ], int mt0,
                                                    int nt0, int lane, const float (&rsc)[TI][4],
                                                    const float (&csc)[TJ]) {
    constexpr int PE = EPI == I8_EPI_SWIGLU ? 0 : P + ((TJ - P) & ~1);  // pairs cover tiles [P, PE)
    if constexpr (PE > P) {
#pragma unroll
        for (int j = P; j < PE; j += 2) {
            const int col = (nt0 + j + ((lane >> 4) & 1)) * 16 + (lane & 15);
            const bool colOk = col >= a.c0 && col < a.c1;
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float v0 = __fmul_rn(__fmul_rn((float)acc[i][j][e], csc[j]), rsc[i][e]);
                    const float v1 = __fmul_rn(__fmul_rn((float)acc[i][j + 1][e], csc[j + 1]), rsc[i][e]);
                    const auto sw = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v0),
                                                                     __builtin_bit_cast(uint32_t, v1), false, false);
                    const int row = (mt0 + i) * 16 + 8 * (lane >> 5) + e;
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const int r = row + 4 * h;
                        const float v = __builtin_bit_cast(float, h ? sw[1] : sw[0]);
                        if (!colOk || r >= a.M) continue;
                        if constexpr (EPI == I8_EPI_STORE)
                            a.dst[(size_t)r * a.stride + col] = v;
                        else
                            __builtin_amdgcn_global_atomic_fadd_f32(a.dst + (size_t)r * a.stride + col, v);
                    }
                }
        }
    }
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        if (PE > P && j >= P && j < PE) continue;  // stored as a pair
        const int col = (nt0 + j) * 16 + (lane & 15);
        const bool colOk = col >= a.c0 && col < a.c1;
        if constexpr (EPI != I8_EPI_SWIGLU) {
            if (!colOk) continue;
        }
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = (mt0 + i) * 16 + 4 * (lane >> 4) + e;
                const float v = __fmul_rn(__fmul_rn((float)acc[i][j][e], csc[j]), rsc[i][e]);
                if constexpr (EPI == I8_EPI_STORE) {
                    if (row < a.M) a.dst[(size_t)row * a.stride + col] = v;
                } else if constexpr (EPI == I8_EPI_ADD) {
                    if (row < a.M) __builtin_amdgcn_global_atomic_fadd_f32(a.dst + (size_t)row * a.stride + col, v);
                } else {
                    // Every lane runs the exchange (DPP quad_perm [1,0,3,2]: lane l ^ 1 holds column col ^ 1).
                    const float u = __builtin_bit_cast(
                        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
                    if (colOk && !(col & 1) && row < a.M)
                        a.dst[(size_t)row * a.stride + (col >> 1)] = v / (1.0f + expf(-v)) * u;
                }
            }
    }
}

// Epilogue of the direct-to-LDS kernels, as in i8gemm_kernel: lane l of a
// 16 x 16 tile holds rows 4 (l / 16) + e, column l % 16; scales first, then
// the stores. mt0 / nt0: the wavefront's first row and column tile.
// Measured on MI355X (config 2, M = 512): stores of 16 columns per row wrote
// 1.32x the output's bytes to HBM (WRITE_SIZE); column-tile pairs from the
// wavefront's first tile 1.19x (wavefronts of 48 columns starting at an odd
// tile paired across lines); pairs that start on a line once.
template <int TI, int TJ, int EPI>
__device__ __forceinline__ void dma_epilogue(const I8GemmArgs &a, const i32x4 (&acc)[TI][TJ], int mt0, int nt0,
                                             int lane) {
    float rsc[TI][4], csc[TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) rsc[i][e] = a.rowScale[min((mt0 + i) * 16 + 4 * (lane >> 4) + e, a.M - 1)];
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const int col = (nt0 + j) * 16 + (lane & 15);
        csc[j] = a.colScale[col >= a.c0 && col < a.c1 ? col : a.c0];
    }
    if (EPI != I8_EPI_SWIGLU && TJ > 2 && (nt0 & 1))
        dma_epilogue_stores<TI, TJ, EPI, 1>(a, acc, mt0, nt0, lane, rsc, csc);
    else
        dma_epilogue_stores<TI, TJ, EPI, 0>(a, acc, mt0, nt0, lane, rsc, csc);
}

// Direct-to-LDS variant: BM x BN block tiles (WGM x WGN wavefronts, each a
// grid of 16 x 16 v_mfma_i32_16x16x64_i8 tiles), a ring of NS stages of one
// 64-deep K-step, every operand fragment (the tile layout's 1 KiB group of
// 16 rows x 64 bytes) loaded with global_load_lds_dwordx4 and read back by
// the lanes that own it (lane l at byte 16 l: no bank conflicts). BROWS (the
// batched pass) takes A as row tiles (rowtile_offset) and B from row-major
// rows (a.K bytes each, K a multiple of 64): each fragment is gathered into
// the same LDS image, lane l reading row l % 16 at byte 16 (l / 16) of the
// step (for A inside one 1 KiB group). The stage NS - 1 ahead is
// requested as each stage starts; the wait is a count, as in the skinny
// kernel. When the fragments of a stage do not split evenly over the
// wavefronts, the first F % NW issue one more. Epilogue (float32(sum) *
// colScale) * rowScale, then a store, an fp32 atomic add into dst
// (I8_EPI_ADD: one owner per element, so exactly dst + v) or the SwiGLU of
// interleaved gate/up columns into dst[row][col / 2] (I8_EPI_SWIGLU, the
// neighbouring column's value by DPP).
template <int BM, int BN, int WGM, int WGN, int NS, bool BROWS, int EPI>
__global__ __launch_bounds__(64 * WGM * WGN) void i8gemm_dma_kernel(const I8GemmArgs a) {
    constexpr int NW = WGM * WGN;
    constexpr int FA = BM / 16, FB = BN / 16, F = FA + FB;  // fragments per stage
    constexpr int DMAX = (F + NW - 1) / NW, DREM = F % NW;  // loads per wavefront and stage
    constexpr int TI = BM / 16 / WGM, TJ = BN / 16 / WGN;
    static_assert(TI * 16 * WGM == BM && TJ * 16 * WGN == BN, "wave grid");
    static_assert(DMAX * (NS - 2) < 64, "in-flight loads beyond the vmcnt range");
    __shared__ i32x4 ring[NS][F][64];
    int bm, bn;
    tile_order(blockIdx.x, a.gridM, a.gridN, bm, bn);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int wm = wv / WGN, wn = wv % WGN;
    const int rt0 = bm * FA, ct0 = a.tileN0 + bn * FB;
    const int MT = (a.M + 15) >> 4, KT = a.KT;
    // Loads of this wavefront: fragment f = wv + NW * d (A tiles first, then B).
    const bool full = DREM == 0 || wv < DREM;  // issues DMAX loads per stage, else DMAX - 1
    const int8_t *src[DMAX];
    int dst[DMAX];
#pragma unroll
    for (int d = 0; d < DMAX; ++d) {
        const int f = min(wv + NW * d, F - 1);
        dst[d] = f;
        if (f < FA) {
            // With BROWS, A comes as row tiles (rowtile_offset): lane l gathers
            // row l % 16's bytes 16 (l / 16) of the group.
            src[d] = a.A + (size_t)min(rt0 + f, MT - 1) * KT * 1024 +
                     (BROWS ? (size_t)(lane & 15) * 64 + (lane >> 4) * 16 : (size_t)lane * 16);
        } else if constexpr (BROWS) {
            src[d] = a.B + (size_t)min((ct0 + (f - FA)) * 16 + (lane & 15), a.N - 1) * a.K + (lane >> 4) * 16;
        } else {
            src[d] = a.B + (size_t)min(ct0 + (f - FA), a.NT - 1) * KT * 1024 + (size_t)lane * 16;
        }
    }
    auto stage_load = [&](int s) {
        const int slot = s % NS;
#pragma unroll
        for (int d = 0; d < DMAX; ++d)
            if (d < DMAX - 1 || full)
                lds_dma16(src[d] + (size_t)s * (BROWS && dst[d] >= FA ? 64 : 1024), &ring[slot][dst[d]][0]);
    };
    i32x4 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = i32x4{0, 0, 0, 0};
#pragma unroll
    for (int p = 0; p < NS - 1; ++p)
        if (p < KT) stage_load(p);
    for (int s = 0; s < KT; ++s) {
        // Loads of the stages after s already requested may stay in flight.
        const int after = min(KT - 1 - s, NS - 2);
        if (after == NS - 2) {
            if (full)
                wait_vm_lgkm0<DMAX * (NS - 2)>();
            else
                wait_vm_lgkm0<(DMAX - 1) * (NS - 2)>();
        } else if (after == 1) {
            if (full)
                wait_vm_lgkm0<DMAX>();
            else
                wait_vm_lgkm0<DMAX - 1>();
        } else {
            wait_vm_lgkm0<0>();
        }
        ring_barrier();
        if (s + NS - 1 < KT) stage_load(s + NS - 1);
        const int slot = s % NS;
        i32x4 fa[TI], fb[TJ];
#pragma unroll
        for (int i = 0; i < TI; ++i) fa[i] = ring[slot][wm * TI + i][lane];
#pragma unroll
        for (int j = 0; j < TJ; ++j) fb[j] = ring[slot][FA + wn * TJ + j][lane];
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    dma_epilogue<TI, TJ, EPI>(a, acc, rt0 + wm * TI, ct0 + wn * TJ, lane);
}

template <int BM, int BN, int WGM, int WGN, int NS, bool BROWS = false, int EPI = I8_EPI_STORE>
static int launch_i8gemm_dma(I8GemmArgs a, hipStream_t stream) {
    const int tiles = (a.c1 + 15) / 16 - a.tileN0;
    a.gridN = (tiles * 16 + BN - 1) / BN;
    a.gridM = (a.M + BM - 1) / BM;
    hipLaunchKernelGGL((i8gemm_dma_kernel<BM, BN, WGM, WGN, NS, BROWS, EPI>), dim3((unsigned)(a.gridM * a.gridN)),
                       dim3(64 * WGM * WGN), 0, stream, a);
    return launch_status();
}

// vmcnt(PER * min(after, MAXA)) and lgkmcnt(0).
template <int PER, int MAXA>
__device__ __forceinline__ void wait_stages_n(int after) {
    if constexpr (MAXA <= 0) {
        wait_vm_lgkm0<0>();
    } else {
        if (after >= MAXA)
            wait_vm_lgkm0<PER * MAXA>();
        else
            wait_stages_n<PER, MAXA - 1>(after);
    }
}

// Ping-pong variant of i8gemm_dma_kernel (8 wavefronts, two per SIMD: a
// probe of the hardware wave id on MI355X places wavefronts w and w + 4 of a
// 512-thread block on one SIMD). The wavefronts of group 0 (0-3) and group 1
// (4-7) run half a K step apart: while one group issues its MFMAs for a step
// (at raised wave priority), the other requests the ring stage NS - 1 ahead,
// reads its fragments of the step from LDS and waits for its share of the
// next stage; a barrier ends each half. Group 1 starts one barrier late and
// group 0 ends with one extra, so every wavefront passes the same number of
// barriers (2 KT + 2). Ordering: a wavefront's share of stage s + 1 is
// complete, and its reads of stage s returned, before the barrier that ends
// its memory half of step s; so both groups' shares of a stage are in LDS
// before the barrier after which group 0 reads it, and the slot that stage
// s + NS - 1 overwrites (stage s - 1's) was last read before the barrier
// preceding the memory half that requests it. Measured on MI355X against
// i8gemm_dma_kernel: the 4096-row int8 pass 54.2-54.4 -> 53.4-53.7 ms (256 x
// 256 tiles, NS = 5), config 2 at M = 512 43.6-44.0 -> 40.8-42.9 us (128 x
// 192 tiles, NS = 6); NS = 4 for the pass gave no gain.
template <int BM, int BN, int WGM, int WGN, int NS, bool BROWS, int EPI>
__global__ __launch_bounds__(64 * WGM * WGN) void i8gemm_pp_kernel(const I8GemmArgs a) {
    constexpr int NW = WGM * WGN;
    static_assert(NW == 8, "two groups of four wavefronts");
    constexpr int FA = BM / 16, FB = BN / 16, F = FA + FB;
    constexpr int DMAX = (F + NW - 1) / NW, DREM = F % NW;
    constexpr int TI = BM / 16 / WGM, TJ = BN / 16 / WGN;
    static_assert(TI * 16 * WGM == BM && TJ * 16 * WGN == BN, "wave grid");
    static_assert(NS >= 3 && DMAX * (NS - 2) < 64, "ring depth");
    __shared__ i32x4 ring[NS][F][64];
    int bm, bn;
    tile_order(blockIdx.x, a.gridM, a.gridN, bm, bn);
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = wv >> 2;
    const int wm = wv / WGN, wn = wv % WGN;
    const int rt0 = bm * FA, ct0 = a.tileN0 + bn * FB;
    const int MT = (a.M + 15) >> 4, KT = a.KT;
    const bool full = DREM == 0 || wv < DREM;
    const int8_t *src[DMAX];
    int dst[DMAX];
#pragma unroll
    for (int d = 0; d < DMAX; ++d) {
        const int f = min(wv + NW * d, F - 1);
        dst[d] = f;
        if (f < FA) {
            src[d] = a.A + (size_t)min(rt0 + f, MT - 1) * KT * 1024 +
                     (BROWS ? (size_t)(lane & 15) * 64 + (lane >> 4) * 16 : (size_t)lane * 16);
        } else if constexpr (BROWS) {
            src[d] = a.B + (size_t)min((ct0 + (f - FA)) * 16 + (lane & 15), a.N - 1) * a.K + (lane >> 4) * 16;
        } else {
            src[d] = a.B + (size_t)min(ct0 + (f - FA), a.NT - 1) * KT * 1024 + (size_t)lane * 16;
        }
    }
    auto stage_load = [&](int s) {
        const int slot = s % NS;
#pragma unroll
        for (int d = 0; d < DMAX; ++d)
            if (d < DMAX - 1 || full)
                lds_dma16(src[d] + (size_t)s * (BROWS && dst[d] >= FA ? 64 : 1024), &ring[slot][dst[d]][0]);
    };
    auto wait_stages = [&](int after) {
        if (full)
            wait_stages_n<DMAX, NS - 2>(after);
        else
            wait_stages_n<DMAX - 1, NS - 2>(after);
    };
    auto barrier = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        ring_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };
    i32x4 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = i32x4{0, 0, 0, 0};
#pragma unroll
    for (int p = 0; p < NS - 1; ++p)
        if (p < KT) stage_load(p);
    wait_stages(min(KT - 1, NS - 2));
    barrier();
    if (grp == 1) barrier();
    i32x4 fa[TI], fb[TJ];
    for (int s = 0; s < KT; ++s) {
        // Memory half: the stage NS - 1 ahead (its slot held stage s - 1, which
        // every wavefront finished reading before the barrier that ended its
        // previous memory half), this step's fragments, then a wait for this
        // wavefront's share of stage s + 1 and for the fragment reads.
        if (s + NS - 1 < KT) stage_load(s + NS - 1);
        const int slot = s % NS;
#pragma unroll
        for (int i = 0; i < TI; ++i) fa[i] = ring[slot][wm * TI + i][lane];
#pragma unroll
        for (int j = 0; j < TJ; ++j) fb[j] = ring[slot][FA + wn * TJ + j][lane];
        wait_stages(min(KT - 2 - s, NS - 2));
        barrier();
        // MFMA half.
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
        __builtin_amdgcn_s_setprio(0);
        barrier();
    }
    if (grp == 0) barrier();
    dma_epilogue<TI, TJ, EPI>(a, acc, rt0 + wm * TI, ct0 + wn * TJ, lane);
}

template <int BM, int BN, int WGM, int WGN, int NS, bool BROWS = false, int EPI = I8_EPI_STORE>
static int launch_i8gemm_pp(I8GemmArgs a, hipStream_t stream) {
    const int tiles = (a.c1 + 15) / 16 - a.tileN0;
    a.gridN = (tiles * 16 + BN - 1) / BN;
    a.gridM = (a.M + BM - 1) / BM;
    hipLaunchKernelGGL((i8gemm_pp_kernel<BM, BN, WGM, WGN, NS, BROWS, EPI>), dim3((unsigned)(a.gridM * a.gridN)),
                       dim3(64 * WGM * WGN), 0, stream, a);
    return launch_status();
}

template <int BM, int BN, int WGM, int WGN>
static int launch_i8gemm_big(I8GemmArgs a, hipStream_t stream) {
    const int tiles = (a.c1 + 15) / 16 - a.tileN0;
    a.gridN = (tiles * 16 + BN - 1) / BN;
    a.gridM = (a.M + BM - 1) / BM;
    hipLaunchKernelGGL((i8gemm_big_kernel<BM, BN, WGM, WGN>), dim3((unsigned)(a.gridM * a.gridN)),
                       dim3(64 * WGM * WGN), 0, stream, a);
    return launch_status();
}

template <int BM, int BN, int WM, int WN, int BKT>
static int launch_i8gemm_lds(I8GemmArgs a, hipStream_t stream) {
    const int tiles = (a.c1 + 15) / 16 - a.tileN0;
    a.gridN = (tiles * 16 + BN - 1) / BN;
    a.gridM = (a.M + BM - 1) / BM;
    const unsigned blocks = (unsigned)(a.gridM * a.gridN);
    hipLaunchKernelGGL((i8gemm_lds_kernel<BM, BN, WM, WN, BKT>), dim3(blocks), dim3(64 * WM * WN), 0, stream, a);
    return launch_status();
}

template <int NWV, int RT, int NTB, int SB, int NS>
static int launch_i8gemm_skinny(I8GemmArgs a, hipStream_t stream) {
    const int tiles = (a.c1 + 15) / 16 - a.tileN0;
    a.gridN = (tiles + NTB - 1) / NTB;
    a.gridM = (a.M + 16 * NWV * RT - 1) / (16 * NWV * RT);
    const unsigned blocks = (unsigned)(a.gridM * a.gridN);
    hipLaunchKernelGGL((i8gemm_skinny_kernel<NWV, RT, NTB, SB, NS>), dim3(blocks), dim3(64 * NWV), 0, stream, a);
    return launch_status();
}

template <int TM, int TN, int WM, int WN, int SK, int U>
static int launch_i8gemm(I8GemmArgs a, hipStream_t stream) {
    const int tiles = (a.c1 + 15) / 16 - a.tileN0;
    a.gridN = (tiles + TN * WN - 1) / (TN * WN);
    a.gridM = (a.M + 16 * TM * WM - 1) / (16 * TM * WM);
    const unsigned blocks = (unsigned)(a.gridM * a.gridN);
    hipLaunchKernelGGL((i8gemm_kernel<TM, TN, WM, WN, SK, U>), dim3(blocks), dim3(64 * WM * WN * SK), 0, stream, a);
    return launch_status();
}

// Columns [c0, c1) of dst for M activation rows. Chooses a tile shape by M;
// every shape gives identical bits (exact int32 sums, same epilogue).
int i8gemm_launch(const int8_t *A, const int8_t *B, const float *rowScale, const float *colScale, float *dst,
                  long stride, int M, int N, int KT, int c0, int c1, hipStream_t stream) {
    if (M == 0 || c0 >= c1) return GPHQ_OK;
    I8GemmArgs a{};
    a.A = A;
    a.B = B;
    a.rowScale = rowScale;
    a.colScale = colScale;
    a.dst = dst;
    a.stride = stride;
    a.M = M;
    a.N = N;
    a.KT = KT;
    a.NT = (N + 15) / 16;
    a.c0 = c0;
    a.c1 = c1;
    a.tileN0 = c0 / 16;
    // Shapes picked by measurement on MI355X at K = 4096, N = 12288 (M = 512:
    // 78.5 us with 128 x 64 LDS tiles, 49.0 with 256 x 128 big tiles, 46.1
    // with 128 x 192, one tile per CU; M = 32 / 64 / 128 / 256: 16.3 / 26 /
    // 27.6 / 38.5 us before the skinny kernel, 11.6 / 12.5 / 18.5 / 32.5 with
    // it).
    // M = 192 / 256 / 384 / 512: 40.6 / 39.4 / 39.7 / 41.1 us with the
    // register-staged big tiles, 24.0 / 24.5 / 35.5 / 36.4 with the
    // direct-to-LDS ones.
    if (M <= 16) return launch_i8gemm<1, 2, 1, 2, 4, 4>(a, stream);
    if (KT % 4 == 0) {  // skinny kernel: whole 4-step stages
        if (M <= 32) return launch_i8gemm_skinny<2, 1, 3, 4, 4>(a, stream);
        if (M <= 64) return launch_i8gemm_skinny<4, 1, 3, 4, 3>(a, stream);
        if (M <= 128) return launch_i8gemm_skinny<4, 2, 3, 4, 3>(a, stream);
    }
    if (M > 128 && M <= 256) return launch_i8gemm_dma<64, 192, 2, 4, 8>(a, stream);
    if (M > 256 && M <= 512) return launch_i8gemm_pp<128, 192, 2, 4, 6>(a, stream);
    if (M <= 64) return launch_i8gemm<4, 1, 1, 2, 4, 4>(a, stream);
    if (M <= 128) return launch_i8gemm_lds<128, 64, 2, 2, 4>(a, stream);
    return launch_i8gemm_big<128, 192, 4, 2>(a, stream);
}

template <int MODE, bool ROT>
static int launch_i8_act_rows(const float *x, long stride, int rows, int K, float eps, const float *signs, int block,
                              int8_t *act, float *rowScale, hipStream_t stream) {
    const int chunks = K / 16;
    const size_t lds = ROT ? rot_lds_bytes(K) : 0;
#define GPHQ_I8ACT(CPT)                                                                                                \
    do {                                                                                                               \
        if (lds > 65536)                                                                                               \
            (void)hipFuncSetAttribute((const void *)i8_act_rows_kernel<MODE, CPT, ROT>,                                \
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);                           \
        hipLaunchKernelGGL((i8_act_rows_kernel<MODE, CPT, ROT>), dim3((unsigned)((rows + 15) & ~15)), dim3(256), lds,  \
                           stream, x, stride, K, eps, signs, block, act, rowScale, rows);                              \
    } while (0)
    if (chunks <= 256)
        GPHQ_I8ACT(1);
    else if (chunks <= 512)
        GPHQ_I8ACT(2);
    else if (chunks <= 768)
        GPHQ_I8ACT(3);
    else
        GPHQ_I8ACT(4);
#undef GPHQ_I8ACT
    return launch_status();
}

// int8 activations of the batched pass (see i8_act_rows_kernel): x rows
// `stride` floats apart and 16-byte aligned, K % 64 == 0, K <= 16384; act is
// in row tiles (rowtile_offset: ceil(rows / 16) * 16 rows of K bytes; rows
// past `rows` in the last tile are not written). signs (device, K values with the
// rotation's scale folded in) rotate each row first, in blocks of `block`;
// null for none.
int lm_i8_act(const float *x, long stride, int rows, int K, bool norm, float eps, const float *signs, int block,
              int8_t *act, float *rowScale, hipStream_t stream) {
    if (rows == 0) return GPHQ_OK;
    if (signs) {
        if (norm) return GPHQ_ERR_UNSUPPORTED;  // no pass normalizes a rotated input
        return launch_i8_act_rows<1, true>(x, stride, rows, K, eps, signs, block, act, rowScale, stream);
    }
    if (norm) return launch_i8_act_rows<2, false>(x, stride, rows, K, eps, nullptr, 0, act, rowScale, stream);
    return launch_i8_act_rows<1, false>(x, stride, rows, K, eps, nullptr, 0, act, rowScale, stream);
}

// One projection of the batched pass on the int8 route: y = (float32(A W^T)
// * w_scale) * a_scale for int8 activations A in row tiles (lm_i8_act)
// and row-major Q8 codes W [N][K] (one fp32 scale per weight row), then epi 0
// stores y[M][N], 1 adds it into y, 2 stores the SwiGLU of interleaved gate/up
// columns into y[M][N/2]; y rows are y_stride floats apart. K % 64 == 0.
// The batched pass's int8 GEMM over columns [a.c0, a.c1) in 256 x BN tiles.
template <int BN>
static int lm_i8_mm_tiles(int epi, const I8GemmArgs &a, hipStream_t stream) {
    constexpr int NS = BN == 256 ? 5 : 6;
    if (epi == 0) return launch_i8gemm_pp<256, BN, 4, 2, NS, true, I8_EPI_STORE>(a, stream);
    if (epi == 1) return launch_i8gemm_pp<256, BN, 4, 2, NS, true, I8_EPI_ADD>(a, stream);
    return launch_i8gemm_pp<256, BN, 4, 2, NS, true, I8_EPI_SWIGLU>(a, stream);
}

int lm_i8_mm(int epi, const int8_t *act, const float *a_scale, const int8_t *codes, const float *w_scale, float *y,
             long y_stride, int M, int K, int N, hipStream_t stream) {
    if (M == 0 || N == 0) return GPHQ_OK;
    I8GemmArgs a{};
    a.A = act;
    a.B = codes;
    a.rowScale = a_scale;
    a.colScale = w_scale;
    a.dst = y;
    a.stride = y_stride;
    a.M = M;
    a.N = N;
    a.K = K;
    a.KT = (K + 63) / 64;
    a.NT = (N + 15) / 16;
    a.c0 = 0;
    a.c1 = N;
    a.tileN0 = 0;
    // 256 x 256 tiles on direct-to-LDS loads, the weights gathered from their
    // rows. Measured on MI355X at M = 4096 (Qwen3-8B's projections, store
    // epilogue) against the register-staged big-tile kernel on row-major
    // operands: QKV 152 -> 141 us, gate/up 527 -> 479, down 207 -> 187; the
    // ping-pong schedule with a 5-stage ring then took the pass 1.5% lower.
    // A grid that is not whole rounds of the chip takes 256 x 256 tiles on the
    // columns that fill whole rounds and 256 x 128 tiles (6-stage ring) on the
    // rest (Qwen3-8B QKV at 4096 rows: 120.7 -> 72.2 + 47.5 us in a kernel
    // trace, 143.7 -> 135.9 us with its activation pack timed by events).
    const long full = whole_round_cols256((M + 255) / 256, (N + 255) / 256);
    if (full > 0) {
        I8GemmArgs b = a;
        b.c1 = (int)(full * 256);
        GPHQ_TRY(lm_i8_mm_tiles<256>(epi, b, stream));
        a.c0 = b.c1;
        a.tileN0 = a.c0 / 16;
        return lm_i8_mm_tiles<128>(epi, a, stream);
    }
    return lm_i8_mm_tiles<256>(epi, a, stream);
}

int i8_pack_tiles(const int8_t *src, int8_t *dst, int rows, int K, int row0, int kt, hipStream_t stream) {
    if (rows == 0) return GPHQ_OK;
    const int rowTiles = ((row0 + rows + 15) >> 4) - (row0 >> 4);
    const size_t chunks = (size_t)rowTiles * kt * 64;
    hipLaunchKernelGGL(i8_pack_tiles_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream, src, dst,
                       rows, K, row0, rowTiles, kt);
    return launch_status();
}

int i8_pack_rows(const float *x, long stride, int rows, int K, int kt, int8_t *act, float *rowScale, float *rowInv,
                 hipStream_t stream) {
    if (rows == 0) return GPHQ_OK;
    // Rows whose values can be read as 16-byte pieces are held in registers
    // (one read of the row); other shapes take the two-pass kernel.
    if (K % 16 == 0 && stride % 4 == 0 && (uintptr_t)x % 16 == 0 && kt <= 256) {
        switch ((kt + 63) / 64) {
#define GPHQ_PACK_VEC(C)                                                                                              \
    case C:                                                                                                           \
        hipLaunchKernelGGL(i8_pack_rows_vec_kernel<C>, dim3((unsigned)((rows + 63) & ~63)), dim3(256), 0, stream, x,  \
                           stride, K, kt, act, rowScale, rowInv, rows);                                               \
        return launch_status();
            GPHQ_PACK_VEC(1)
            GPHQ_PACK_VEC(2)
            GPHQ_PACK_VEC(3)
            GPHQ_PACK_VEC(4)
#undef GPHQ_PACK_VEC
        }
    }
    hipLaunchKernelGGL(i8_pack_rows_kernel, dim3(rows), dim3(256), 0, stream, x, stride, K, kt, act, rowScale, rowInv);
    return launch_status();
}

int i8_pack_range(const float *x, long stride, int rows, int K, int kt, int k0, int k1, int8_t *act,
                  const float *rowInv, hipStream_t stream) {
    if (rows == 0 || (k0 == k1 && k1 != K)) return GPHQ_OK;
    hipLaunchKernelGGL(i8_pack_range_kernel, dim3(rows), dim3(256), 0, stream, x, stride, K, kt, k0, k1, act, rowInv);
    return launch_status();
}

}  // namespace gphq
