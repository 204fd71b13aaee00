// FP16-operand GEMMs with fp32 accumulation on v_mfma_f32_16x16x32_f16:
//
//  * q8gemm MulPanels (q8gemm/gemm.go:228-286, scalar.go:9-20): FP16
//    activations (each row scaled by an exact power of two into [2^14, 2^15))
//    times int8 or FP16 weights, then acc * colScale[c] * rowInverse[r].
//  * qwen3lm mm (gpu.metal:766-927, PRO_PLAIN / EPI_STORE): weights of a GPU
//    format dequantized to FP16 per K step (Q8: half(code); Q8B: half(code) *
//    half(d) rounded to half; Q4: (half(nib) - 8) * d rounded to half),
//    activations half(x), fp32 accumulation; Q8 rows then scaled by their fp32
//    row scale.
//  * GPTQ int4 with group-128 FP16 scales and 4-bit zero points (8 codes per
//    int32): (half(nib) - half(z)) * s rounded to half.
//  * the qwen3lm batched pass's projections (mm_qkv / mm_o / mm_gateup /
//    mm_down, gpu.metal:994-1025): the same tiles with the residual-add and
//    SwiGLU epilogues (gpu.metal:897-927), and Q8B with fp32 block scales
//    (half(code) * half(d), as Q8B once the scale is rounded to FP16).
//
// Fragments: lane l of a 16x64 K step holds row (l % 16), columns
// (l / 16) * 16 .. +16 of both operands (16 FP16 values = two 8-value MFMA
// operands). The two MFMAs per step take values 0..7 and 8..15 of every lane;
// A and B use the same K assignment, so C = A . B^T exactly as a plain K loop.
// Activations are FP16 in the tile layout [M/16][K/64][64][16] (2 KiB per
// group), written by f16_act_pack_kernel. Weights are read in their own
// layout: the int8 tile layout of gemm_i8.hip, an FP16 tile layout, or the
// qwen3lm row-major code arrays.
#include "common.h"
#include "gemm_f16.h"

namespace gphq {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ _Float16 i8h(uint32_t v, int i) { return (_Float16)(int)((int32_t)(v << (24 - 8 * i)) >> 24); }


// Raw codes of one B fragment (16 values of row n at k = kt*64 + g*16): the
// code bytes (GPTQ: two words), and the scale bits (FP16 in the low half, or
// all 32 bits of an fp32 scale) and GPTQ zero point (bits 16..23). The codes
// are read with ordinary (cached) loads: one K step takes 16-64 bytes of a
// row, so each 128-byte line serves two (Q8) to four (GPTQ) consecutive
// steps, and nontemporal loads re-fetched it for each (measured on MI355X:
// GPTQ M = 256, K = 4096 -> N = 12288, 81 -> 67 us; Q8B M = 512, 106 -> 96 us).
struct RawB {
    u32x4 w;
    uint32_t sz;
    bool ok;  // the fragment lies inside K (else it dequantizes to zeros)
};

// A fragment past K is loaded from the row's last 16 values instead and
// zeroed by dequant, so the load is issued on every path and the compiler's
// waits for a register set count only the loads issued before it.
template <int WF>
__device__ __forceinline__ RawB load_raw(const F16GemmArgs &a, int n, int kt, int g) {
    const int k0 = kt * 64 + g * 16;
    RawB r{u32x4{0, 0, 0, 0}, 0, k0 < a.K};
    const int k = r.ok ? k0 : a.K - 16;
    if constexpr (WF == W_Q8_ROW || WF == W_Q8B_ROW || WF == W_Q8BF_ROW) {
        r.w = *(const u32x4 *)((const int8_t *)a.B + (size_t)n * a.K + k);
        if constexpr (WF == W_Q8B_ROW) r.sz = ((const uint16_t *)a.bScale)[(size_t)n * (a.K >> 5) + (k >> 5)];
        if constexpr (WF == W_Q8BF_ROW) r.sz = ((const uint32_t *)a.bScale)[(size_t)n * (a.K >> 5) + (k >> 5)];
    } else if constexpr (WF == W_Q4_ROW) {
        r.w = *(const u32x4 *)((const uint8_t *)a.B + (size_t)n * (a.K >> 1) + (k >> 5) * 16);
        r.sz = ((const uint16_t *)a.bScale)[(size_t)n * (a.K >> 5) + (k >> 5)];
    } else {  // W_GPTQ_ROW
        const u32x2 w2 = *(const u32x2 *)((const uint32_t *)a.B + (size_t)n * (a.K >> 3) + (k >> 3));
        r.w.x = w2.x;
        r.w.y = w2.y;
        const size_t gi = (size_t)n * (a.K >> 7) + (k >> 7);
        r.sz = ((const uint16_t *)a.bScale)[gi] | ((uint32_t)(a.bZero[gi] & 15) << 16);
    }
    return r;
}

// Four int8 codes (one dword) as FP16 pairs (c0, c1), (c2, c3), exactly:
// v_perm_b32 places each code + 128 (the xor) under the exponent byte 0x64,
// giving 1024 + 128 + c, and one packed subtraction leaves c.
__device__ __forceinline__ void i8x4_to_h(uint32_t w, f16x2 &p0, f16x2 &p1) {
    const uint32_t u = w ^ 0x80808080u;
    const f16x2 off = f16x2{(_Float16)1152.0f, (_Float16)1152.0f};
    p0 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - off;
    p1 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - off;
}
// Four nibbles in the low halves of the bytes of w (w & 0x0F0F0F0F) as FP16
// pairs (n - 8).
__device__ __forceinline__ void n4x4_to_h(uint32_t w, f16x2 &p0, f16x2 &p1) {
    const f16x2 off = f16x2{(_Float16)1032.0f, (_Float16)1032.0f};
    p0 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u)) - off;
    p1 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u)) - off;
}
__device__ __forceinline__ f16x8 cat4(f16x2 a, f16x2 b, f16x2 c, f16x2 d) {
    return __builtin_shufflevector(__builtin_shufflevector(a, b, 0, 1, 2, 3), __builtin_shufflevector(c, d, 0, 1, 2, 3),
                                   0, 1, 2, 3, 4, 5, 6, 7);
}

// The same FP16 values as load_b: Q8 half(code); Q8B half(code) * d; Q8B
// with fp32 scales half(code) * half(d); Q4 (half(nib) - 8) * d; GPTQ
// (half(nib) - half(z)) * s, each product rounded to half once (packed FP16
// multiplies round like the scalar ones).
template <int WF>
__device__ __forceinline__ void dequant(const RawB &r, int g, f16x8 &lo, f16x8 &hi) {
    if constexpr (WF == W_Q8_ROW || WF == W_Q8B_ROW || WF == W_Q8BF_ROW) {
        f16x2 p[8];
        i8x4_to_h(r.w.x, p[0], p[1]);
        i8x4_to_h(r.w.y, p[2], p[3]);
        i8x4_to_h(r.w.z, p[4], p[5]);
        i8x4_to_h(r.w.w, p[6], p[7]);
        if constexpr (WF != W_Q8_ROW) {
            _Float16 d;
            if constexpr (WF == W_Q8B_ROW)
                d = __builtin_bit_cast(_Float16, (uint16_t)r.sz);
            else
                d = (_Float16)__builtin_bit_cast(float, r.sz);
            const f16x2 dd = f16x2{d, d};
#pragma unroll
            for (int i = 0; i < 8; ++i) p[i] = p[i] * dd;
        }
        lo = cat4(p[0], p[1], p[2], p[3]);
        hi = cat4(p[4], p[5], p[6], p[7]);
    } else if constexpr (WF == W_Q4_ROW) {
        const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)r.sz);
        const f16x2 dd = f16x2{d, d};
        const int sh = (g & 1) * 4;
        f16x2 p[8];
        n4x4_to_h((r.w.x >> sh) & 0x0F0F0F0Fu, p[0], p[1]);
        n4x4_to_h((r.w.y >> sh) & 0x0F0F0F0Fu, p[2], p[3]);
        n4x4_to_h((r.w.z >> sh) & 0x0F0F0F0Fu, p[4], p[5]);
        n4x4_to_h((r.w.w >> sh) & 0x0F0F0F0Fu, p[6], p[7]);
#pragma unroll
        for (int i = 0; i < 8; ++i) p[i] = p[i] * dd;
        lo = cat4(p[0], p[1], p[2], p[3]);
        hi = cat4(p[4], p[5], p[6], p[7]);
    } else {
        // GPTQ: nibble i of a word is value i. Even nibbles (w & 0x0F0F0F0F) and
        // odd ones ((w >> 4) & 0x0F0F0F0F) are paired by v_perm_b32 into the low
        // bytes of two halves, 0x6400 is or-ed in (1024 + n), and one packed
        // subtraction of 1024 + z leaves n - z exactly.
        const _Float16 sc = __builtin_bit_cast(_Float16, (uint16_t)r.sz);
        const _Float16 zb = (_Float16)(float)(1024 + (int)(r.sz >> 16));
        const f16x2 off = f16x2{zb, zb}, ss = f16x2{sc, sc};
        f16x2 p[8];
        const uint32_t wds[2] = {r.w.x, r.w.y};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t x = wds[h] & 0x0F0F0F0Fu, y = (wds[h] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t sel = (uint32_t)q | (0x0Cu << 8) | ((uint32_t)(4 + q) << 16) | (0x0Cu << 24);
                p[4 * h + q] =
                    (__builtin_bit_cast(f16x2, __builtin_amdgcn_perm(y, x, sel) | 0x64006400u) - off) * ss;
            }
        }
        lo = cat4(p[0], p[1], p[2], p[3]);
        hi = cat4(p[4], p[5], p[6], p[7]);
    }
    if (!r.ok) {
        lo = f16x8{};
        hi = f16x8{};
    }
}

// B fragment: 16 FP16 weights of row `n` (clamped in range), K step kt, lane
// group g (values k = kt*64 + g*16 + 0..15), decoded per format.
template <int WF>
__device__ __forceinline__ void load_b(const F16GemmArgs &a, int n, int kt, int lane, f16x8 &lo, f16x8 &hi) {
    const int g = lane >> 4;
    if constexpr (WF == W_I8_TILE) {
        const u32x4 w = __builtin_nontemporal_load(
            (const u32x4 *)((const int8_t *)a.B + ((size_t)(n >> 4) * a.KT + kt) * 1024 + (size_t)lane * 16));
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) lo[i] = i8h(ww[i >> 2], i & 3);
#pragma unroll
        for (int i = 0; i < 8; ++i) hi[i] = i8h(ww[2 + (i >> 2)], i & 3);
    } else if constexpr (WF == W_F16_TILE) {
        const f16x8 *p = (const f16x8 *)((const _Float16 *)a.B + ((size_t)(n >> 4) * a.KT + kt) * 1024 + (size_t)lane * 16);
        lo = __builtin_nontemporal_load(p);
        hi = __builtin_nontemporal_load(p + 1);
    } else {  // row formats: the same codes and FP16 products as the LDS-tiled kernels
        dequant<WF>(load_raw<WF>(a, n, kt, g), g, lo, hi);
    }
}

// Epilogue of one lane's part of a 16x16 accumulator tile (or of a 4-row
// group of a 32x32 one): rows row0 .. row0 + 3 of column col, with the
// column's scale cs and the rows' scales ri (as epilogue_scales reads them).
// Columns outside [c0, c1) and rows past M are not written. Every lane of the
// wavefront calls it (EPI_SWIGLU exchanges the gate and up values of
// neighbouring lanes).
template <int EPI>
__device__ __forceinline__ void epilogue_scaled(const F16GemmArgs &a, const f32x4 &acc, int row0, int col, float cs,
                                                const float (&ri)[4]) {
    const bool colOk = col >= a.c0 && col < a.c1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int row = row0 + e;
        float v = acc[e];
        // The qwen3lm pass's row scale 2^-e (exact).
        if constexpr (EPI != EPI_PANELS) {
            if (a.rowInv) v = __fmul_rn(v, ri[e]);
        }
        if constexpr (EPI == EPI_SWIGLU) {
            if (a.colScale) v = __fmul_rn(v, cs);
            // The up value of the neighbouring lane (DPP quad_perm [1,0,3,2]).
            const float u = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF,
                                                                               0xF, true));
            if (colOk && !(col & 1) && row < a.M) a.dst[(size_t)row * a.stride + (col >> 1)] = v / (1.0f + expf(-v)) * u;
        } else if (colOk && row < a.M) {
            float *p = a.dst + (size_t)row * a.stride + col;
            if constexpr (EPI == EPI_PANELS) v = __fmul_rn(__fmul_rn(v, cs), ri[e]);
            if constexpr (EPI == EPI_ROWSCALE) v = __fmul_rn(v, cs);
            if constexpr (EPI == EPI_ADD) {
                // One fp32 add into the residual, done in L2 without a return
                // (each element has one owner, so the sum is y + v exactly,
                // and the wave does not wait for the old value).
                if (a.colScale) v = __fmul_rn(v, cs);
                __builtin_amdgcn_global_atomic_fadd_f32(p, v);
            } else {
                *p = v;
            }
        }
    }
}

// The scales epilogue_scaled takes: the column's (1 where the epilogue has
// none) and the four rows' (rows past M read the last row; they are not
// written). Read before any store of the tile: the compiler cannot tell that
// the stores do not alias the scales, so scales read between stores are
// reloaded one at a time.
template <int EPI>
__device__ __forceinline__ float epilogue_col_scale(const F16GemmArgs &a, int col) {
    // Loaded unconditionally (a column outside [c0, c1) reads c0's) and then
    // selected: a load under a lane condition makes later waits drain stores.
    const bool colOk = col >= a.c0 && col < a.c1;
    if constexpr (EPI == EPI_PANELS || EPI == EPI_ROWSCALE) {
        const float v = a.colScale[colOk ? col : a.c0];
        return colOk ? v : 1.0f;
    }
    if constexpr (EPI == EPI_ADD || EPI == EPI_SWIGLU) {
        if (!a.colScale) return 1.0f;
        const float v = a.colScale[colOk ? col : a.c0];
        return colOk ? v : 1.0f;
    }
    return 1.0f;
}
__device__ __forceinline__ void epilogue_row_scales(const F16GemmArgs &a, int row0, float (&ri)[4]) {
    if (!a.rowInv) {
        ri[0] = ri[1] = ri[2] = ri[3] = 1.0f;
        return;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) ri[e] = a.rowInv[min(row0 + e, a.M - 1)];
}

template <int EPI>
__device__ __forceinline__ void epilogue(const F16GemmArgs &a, const f32x4 &acc, int row0, int col) {
    float ri[4];
    epilogue_row_scales(a, row0, ri);
    epilogue_scaled<EPI>(a, acc, row0, col, epilogue_col_scale<EPI>(a, col), ri);
}

template <int WF, int EPI, int TM, int TN, int WM, int WN, int SK, int U>
__global__ __launch_bounds__(64 * WM * WN * SK) void f16gemm_kernel(const F16GemmArgs a) {
    constexpr int NW = WM * WN * SK;
    __shared__ f32x4 red[(SK > 1) ? (NW * TM * TN * 64) : 1];
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
    const int mt0 = (bm * WM + wm) * TM;
    const int nt0 = a.tileN0 + (bn * WN + wn) * TN;
    const int MT = (a.M + 15) >> 4;
    const int KT = a.KT;
    const int per = (KT + SK - 1) / SK;
    const int kt0 = ks * per, kt1 = min(KT, kt0 + per);
    int nrow[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) nrow[j] = min((nt0 + j) * 16 + (lane & 15), a.N - 1);
    size_t aoff[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) aoff[i] = (size_t)min(mt0 + i, MT - 1) * KT * 1024 + (size_t)lane * 16;

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int kt = kt0; kt < kt1; kt += U) {
        f16x8 fa[U][TM][2], fb[U][TN][2];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const bool ok = kt + u < kt1;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                if (ok) {
                    const f16x8 *p = (const f16x8 *)(a.A + aoff[i] + (size_t)(kt + u) * 1024);
                    fa[u][i][0] = p[0];
                    fa[u][i][1] = p[1];
                } else {
                    fa[u][i][0] = f16x8{};
                    fa[u][i][1] = f16x8{};
                }
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                if (ok) {
                    load_b<WF>(a, nrow[j], kt + u, lane, fb[u][j][0], fb[u][j][1]);
                } else {
                    fb[u][j][0] = f16x8{};
                    fb[u][j][1] = f16x8{};
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[u][i][h], fb[u][j][h], acc[i][j], 0, 0, 0);
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

#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < TM; ++i)
            epilogue<EPI>(a, acc[i][j], (mt0 + i) * 16 + 4 * (lane >> 4), (nt0 + j) * 16 + (lane & 15));
}

// ---- LDS-shared B tiles (qwen3lm row formats, M > 64) -------------------------
// Block tile (16*WTM*WGM) x (32*WTN): 2*WGM wavefronts, WGM along M and 2
// along N, each (16*WTM) x (16*WTN) of the output. Per 64-deep K step the
// block's threads dequantize the B tile once into LDS in MFMA fragment order
// (tile j, lane slot g*16 + n%16, 16 values), double-buffered; the raw codes
// of step kt+1 are loaded before the MFMAs of step kt run and written to the
// other buffer after them, with one barrier per step. A fragments come
// straight from the FP16 tile layout (two 16-byte loads per lane and tile),
// one step ahead.
template <int WF, int EPI, int WTM, int WTN, int WGM>
__global__ __launch_bounds__(128 * WGM) void f16gemm_lds_kernel(const F16GemmArgs a) {
    constexpr int NT = 128 * WGM;
    constexpr int BN16 = 2 * WTN;           // 16-row B tiles per block
    constexpr int PAIRS = BN16 * 64 / NT;   // (row, lane group) pairs per thread and step
    static_assert(PAIRS >= 1 && PAIRS * NT == BN16 * 64, "B tile pairs divide over the block");
    __shared__ f16x8 bs[2][BN16][64][2];
    int bm, bn;
    tile_order(blockIdx.x, a.gridM, a.gridN, bm, bn);
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int wm = wv >> 1, wn = wv & 1;
    const int mt0 = (bm * WGM + wm) * WTM;
    const int nt0 = a.tileN0 + bn * BN16;
    const int MT = (a.M + 15) >> 4;
    const int KT = a.KT;
    size_t aoff[WTM];
#pragma unroll
    for (int i = 0; i < WTM; ++i) aoff[i] = (size_t)min(mt0 + i, MT - 1) * KT * 1024 + (size_t)lane * 16;
    // Loader assignment: pair p -> tile p / 64, lane slot p % 64 (row n = tile*16 + slot % 16, group slot / 16).
    int pn[PAIRS], pg[PAIRS], pt[PAIRS], ps[PAIRS];
#pragma unroll
    for (int q = 0; q < PAIRS; ++q) {
        const int p = threadIdx.x + NT * q;
        pt[q] = p >> 6;
        ps[q] = p & 63;
        pg[q] = ps[q] >> 4;
        pn[q] = min((nt0 + pt[q]) * 16 + (ps[q] & 15), a.N - 1);
    }
    auto load_a = [&](int kt, f16x8 (&fa)[WTM][2]) {
#pragma unroll
        for (int i = 0; i < WTM; ++i) {
            const f16x8 *p = (const f16x8 *)(a.A + aoff[i] + (size_t)kt * 1024);
            fa[i][0] = p[0];
            fa[i][1] = p[1];
        }
    };
    f32x4 acc[WTM][WTN];
#pragma unroll
    for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int j = 0; j < WTN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    RawB raw[PAIRS];
#pragma unroll
    for (int q = 0; q < PAIRS; ++q) raw[q] = load_raw<WF>(a, pn[q], 0, pg[q]);
    f16x8 fa[WTM][2], fn[WTM][2];
    load_a(0, fa);
#pragma unroll
    for (int q = 0; q < PAIRS; ++q) dequant<WF>(raw[q], pg[q], bs[0][pt[q]][ps[q]][0], bs[0][pt[q]][ps[q]][1]);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < KT;
        if (more) {
#pragma unroll
            for (int q = 0; q < PAIRS; ++q) raw[q] = load_raw<WF>(a, pn[q], kt + 1, pg[q]);
            load_a(kt + 1, fn);
        }
#pragma unroll
        for (int j = 0; j < WTN; ++j) {
            const f16x8 b0 = bs[cur][wn * WTN + j][lane][0], b1 = bs[cur][wn * WTN + j][lane][1];
#pragma unroll
            for (int i = 0; i < WTM; ++i) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i][0], b0, acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i][1], b1, acc[i][j], 0, 0, 0);
            }
        }
        if (more) {
#pragma unroll
            for (int q = 0; q < PAIRS; ++q)
                dequant<WF>(raw[q], pg[q], bs[cur ^ 1][pt[q]][ps[q]][0], bs[cur ^ 1][pt[q]][ps[q]][1]);
#pragma unroll
            for (int i = 0; i < WTM; ++i) fa[i][0] = fn[i][0], fa[i][1] = fn[i][1];
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < WTN; ++j)
#pragma unroll
        for (int i = 0; i < WTM; ++i)
            epilogue<EPI>(a, acc[i][j], (mt0 + i) * 16 + 4 * (lane >> 4), (nt0 + wn * WTN + j) * 16 + (lane & 15));
}

template <int WF, int EPI, int WTM, int WTN, int WGM>
static int launch_f16gemm_lds(F16GemmArgs a, hipStream_t stream) {
    const int tiles = (a.c1 + 15) / 16 - a.tileN0;
    a.gridN = (tiles + 2 * WTN - 1) / (2 * WTN);
    a.gridM = (a.M + 16 * WTM * WGM - 1) / (16 * WTM * WGM);
    hipLaunchKernelGGL((f16gemm_lds_kernel<WF, EPI, WTM, WTN, WGM>), dim3((unsigned)(a.gridM * a.gridN)),
                       dim3(128 * WGM), 0, stream, a);
    return launch_status();
}

template <int WF, int EPI, int TM, int TN, int WM, int WN, int SK, int U>
static int launch_f16gemm(F16GemmArgs a, hipStream_t stream) {
    const int tiles = (a.c1 + 15) / 16 - a.tileN0;
    a.gridN = (tiles + TN * WN - 1) / (TN * WN);
    a.gridM = (a.M + 16 * TM * WM - 1) / (16 * TM * WM);
    hipLaunchKernelGGL((f16gemm_kernel<WF, EPI, TM, TN, WM, WN, SK, U>), dim3((unsigned)(a.gridM * a.gridN)),
                       dim3(64 * WM * WN * SK), 0, stream, a);
    return launch_status();
}

// ---- BM x BN block tiles (qwen3lm row formats, large M) -----------------------
// WGM x WGN wavefronts, each (BM/WGM) x (BN/WGN) of the output as tiles of
// v_mfma_f32_32x32x16_f16 (256 x 256 with 4 x 2 waves for long GEMMs,
// 128 x 128 with 2 x 2 when fewer, larger-K blocks are wanted). With
// a.splits > 1 block b takes K steps of split b / tiles and writes raw sums
// to a.part; mm_finish_kernel adds the splits in order. Per 64-deep K step
// both operands pass through LDS
// (FP16, 128 bytes per row, 16-byte chunks swizzled by the row so the
// fragment reads of 8 or 16 consecutive rows hit distinct banks), double
// buffered: step kt+1's global loads (A: FP16 tiles, B: raw codes) are issued
// one step ahead into registers, written (B dequantized) to the other buffer
// after step kt's MFMAs, with one barrier per step.
//
// MFMA operands: lane l holds row l % 32 of its matrix (A row m, or weight row
// n) and k values 8*(l/32) .. +7 of the 16-deep sub-step; the result lane l
// holds column n = l % 32, rows 8*(i/4) + 4*(l/32) + i%4 of acc[i].



template <int WF, int EPI_T, int BM, int BN, int WGM, int WGN, int PF>
__global__ __launch_bounds__(64 * WGM * WGN) void f16gemm_big_kernel(const F16GemmArgs a) {
    typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));
    typedef float f32x16 __attribute__((ext_vector_type(16)));
    constexpr int NT = 64 * WGM * WGN;
    constexpr int TI = BM / WGM / 32, TJ = BN / WGN / 32;  // 32x32 tiles per wave
    constexpr int AL = BM * 8 / NT;   // 16-byte A units per thread and step
    constexpr int BL = BN * 4 / NT;   // (row, 16 K values) B pieces per thread and step
    static_assert(AL >= 1 && BL >= 1 && NT % 128 == 0, "loader split");
    __shared__ f16x8v As[2][BM * 8];
    __shared__ f16x8v Bs[2][BN * 8];
    const int tiles = a.gridM * a.gridN;
    const int sp = blockIdx.x / tiles;
    int bm, bn;
    tile_order(blockIdx.x - sp * tiles, a.gridM, a.gridN, bm, bn);
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int wm = wv / WGN, wn = wv % WGN;
    const int m0 = bm * BM, n0 = a.tileN0 * 16 + bn * BN;
    const int MT = (a.M + 15) >> 4, KT = a.KT;
    const int kper = (KT + a.splits - 1) / a.splits;
    const int k0 = sp * kper, k1 = min(KT, k0 + kper);

    // A loader: 2 KB groups (16 rows x 64 K) of the FP16 tile layout, one per
    // 128 threads and load i (group i*NT/128 + t/128). Thread t takes row t%16
    // and 16-byte chunk (t/16)%8 (K values 8*chunk ..) of its group: in the
    // tile layout that is half chunk%2 of fragment lane row + 16*(chunk/2),
    // unit 2*lane + half. Each 8-lane phase of an LDS write (128 bytes a
    // cycle) then covers 8 consecutive rows at one chunk, 8 distinct swizzled
    // slots, and a wavefront's loads still cover 1 KB of the group.
    const int arow = t & 15, achunk = (t >> 4) & 7;
    const _Float16 *abase = a.A + (size_t)(2 * (arow + 16 * (achunk >> 1)) + (achunk & 1)) * 8;
    const int mtb = (m0 >> 4) + (t >> 7);
    // B loader: piece i of thread t is row (i*NT + t)/4 of the tile, 16 K
    // values at 16*(t%4) of the step.
    const int bc = t & 3;

    // PF register sets: step r's loads go to set r % PF, so loads run PF
    // steps ahead of their LDS writes.
    f16x8v ar[PF][AL];
    RawB br[PF][BL];
    auto gload = [&](int set, int kt) {
#pragma unroll
        for (int i = 0; i < AL; ++i)
            ar[set][i] = *(const f16x8v *)(abase + ((size_t)min(mtb + i * (NT / 128), MT - 1) * KT + kt) * 1024);
#pragma unroll
        for (int i = 0; i < BL; ++i)
            br[set][i] = load_raw<WF>(a, min(n0 + ((i * NT + t) >> 2), a.N - 1), kt, bc);
    };
    auto lstore = [&](int set, int buf) {
#pragma unroll
        for (int i = 0; i < AL; ++i) {
            const int r = 16 * (i * (NT / 128) + (t >> 7)) + arow;
            As[buf][r * 8 + big_swz(r, achunk)] = ar[set][i];
        }
#pragma unroll
        for (int i = 0; i < BL; ++i) {
            f16x8 lo, hi;
            dequant<WF>(br[set][i], bc, lo, hi);
            const int r = (i * NT + t) >> 2;
            Bs[buf][r * 8 + big_swz(r, 2 * bc)] = lo;
            Bs[buf][r * 8 + big_swz(r, 2 * bc + 1)] = hi;
        }
    };

    f32x16 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = f32x16{};

    gload(0, k0);
    lstore(0, 0);
#pragma unroll
    for (int r = 1; r <= PF; ++r)
        if (k0 + r < k1) gload(r % PF, k0 + r);
    __syncthreads();
    const int fr = lane & 31, fh = lane >> 5;
    auto frags = [&](int buf, int s, f16x8v (&fa)[TI], f16x8v (&fb)[TJ]) {
        const int c = 2 * s + fh;
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            const int r = wm * (32 * TI) + 32 * i + fr;
            fa[i] = As[buf][r * 8 + big_swz(r, c)];
        }
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int r = wn * (32 * TJ) + 32 * j + fr;
            fb[j] = Bs[buf][r * 8 + big_swz(r, c)];
        }
    };
    // One K step: MFMAs on LDS buffer r & 1, and step r+1's tiles (register
    // set `set` = (r+1) % PF) into the other buffer and step r+1+PF's loads.
    // With two wavefronts per SIMD (8 per block), the second wavefront of each
    // SIMD writes the next tiles before its MFMAs and the first after them, so
    // one of the two keeps the SIMD's MFMA pipe busy while the other
    // dequantizes (measured: 2% on the 4096-row pass).
    const bool early = NT >= 512 && wv >= NT / 128;
    auto step = [&](int r, int set) {
        const int cur = r & 1, kt = k0 + r;
        if (early && kt + 1 < k1) {
            lstore(set, cur ^ 1);
            if (kt + 1 + PF < k1) gload(set, kt + 1 + PF);
        }
        f16x8v fa[2][TI], fb[2][TJ];
        frags(cur, 0, fa[0], fb[0]);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            if (s < 3) frags(cur, s + 1, fa[(s + 1) & 1], fb[(s + 1) & 1]);
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[s & 1][i], fb[s & 1][j], acc[i][j], 0, 0, 0);
        }
        if (!early && kt + 1 < k1) {
            lstore(set, cur ^ 1);
            if (kt + 1 + PF < k1) gload(set, kt + 1 + PF);
        }
        __syncthreads();
    };
    const int nsteps = k1 - k0;
    if constexpr (PF == 1) {
        for (int r = 0; r < nsteps; ++r) step(r, 0);
    } else {
        static_assert(PF == 2, "prefetch depth 1 or 2");
        for (int r = 0; r < nsteps; r += 2) {
            step(r, 1);
            if (r + 1 < nsteps) step(r + 1, 0);
        }
    }
    if (a.splits > 1) {
        // Raw sums of this split: part[sp][row][col - c0].
        const int ld = a.c1 - a.c0;
        float *part = a.part + (size_t)sp * a.M * ld;
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const int col = n0 + wn * (32 * TJ) + 32 * j + fr;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int row = m0 + wm * (32 * TI) + 32 * i + 8 * (e >> 2) + 4 * fh + (e & 3);
                    if (row < a.M && col >= a.c0 && col < a.c1) part[(size_t)row * ld + (col - a.c0)] = acc[i][j][e];
                }
            }
        return;
    }
    // Every scale of the lane's outputs first, then the stores.
    float ri[TI][4][4], cs[TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) epilogue_row_scales(a, m0 + wm * (32 * TI) + 32 * i + 8 * q + 4 * fh, ri[i][q]);
#pragma unroll
    for (int j = 0; j < TJ; ++j) cs[j] = epilogue_col_scale<EPI_T>(a, n0 + wn * (32 * TJ) + 32 * j + fr);
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                epilogue_scaled<EPI_T>(a,
                                       f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                             acc[i][j][4 * q + 3]},
                                       m0 + wm * (32 * TI) + 32 * i + 8 * q + 4 * fh,
                                       n0 + wn * (32 * TJ) + 32 * j + fr, cs[j], ri[i][q]);
}

// Split-K finish (the reference's mm_finish, gpu.metal:953-982, for the store
// epilogues): y[row][col] = sum over splits in order of part[s][row][col],
// times the Q8 row scale for EPI_ROWSCALE. One thread per output.
template <int EPI>
__global__ __launch_bounds__(256) void mm_finish_kernel(const F16GemmArgs a) {
    const int ld = a.c1 - a.c0;
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)a.M * ld) return;
    const int row = (int)(idx / ld), c = (int)(idx - (size_t)row * ld);
    float v = a.part[idx];
    for (int s = 1; s < a.splits; ++s) v += a.part[(size_t)s * a.M * ld + idx];
    if constexpr (EPI == EPI_ROWSCALE) v = __fmul_rn(v, a.colScale[a.c0 + c]);
    a.dst[(size_t)row * a.stride + a.c0 + c] = v;
}

// The same finish, four consecutive outputs of one row per thread (16-byte
// loads and stores; the column range, the stride and the buffers 16-byte
// aligned), the splits added in the same order.
template <int EPI>
__global__ __launch_bounds__(256) void mm_finish4_kernel(const F16GemmArgs a) {
    const unsigned q = (unsigned)(a.c1 - a.c0) / 4u;  // quads per row
    const unsigned idx = blockIdx.x * 256u + threadIdx.x;
    if (idx >= (unsigned)a.M * q) return;
    const unsigned row = idx / q, c = 4u * (idx - row * q);
    const size_t plane = (size_t)a.M * (a.c1 - a.c0);
    float4 v = *(const float4 *)(a.part + 4 * (size_t)idx);
    for (int s = 1; s < a.splits; ++s) {
        const float4 p = *(const float4 *)(a.part + (size_t)s * plane + 4 * (size_t)idx);
        v.x += p.x;
        v.y += p.y;
        v.z += p.z;
        v.w += p.w;
    }
    if constexpr (EPI == EPI_ROWSCALE) {
        const float4 cs = *(const float4 *)(a.colScale + a.c0 + c);
        v.x = __fmul_rn(v.x, cs.x);
        v.y = __fmul_rn(v.y, cs.y);
        v.z = __fmul_rn(v.z, cs.z);
        v.w = __fmul_rn(v.w, cs.w);
    }
    *(float4 *)(a.dst + (size_t)row * a.stride + a.c0 + c) = v;
}

template <int WF, int EPI, int BM, int BN, int WGM, int WGN, int PF>
static int launch_f16gemm_big(F16GemmArgs a, hipStream_t stream) {
    a.gridN = (a.c1 - a.tileN0 * 16 + BN - 1) / BN;
    a.gridM = (a.M + BM - 1) / BM;
    if (a.splits < 1) a.splits = 1;
    hipLaunchKernelGGL((f16gemm_big_kernel<WF, EPI, BM, BN, WGM, WGN, PF>),
                       dim3((unsigned)(a.gridM * a.gridN * a.splits)), dim3(64 * WGM * WGN), 0, stream, a);
    GPHQ_TRY(launch_status());
    if (a.splits == 1) return GPHQ_OK;
    const size_t outs = (size_t)a.M * (a.c1 - a.c0);
    const bool quads = (a.c1 - a.c0) % 4 == 0 && a.c0 % 4 == 0 && a.stride % 4 == 0 && (uintptr_t)a.dst % 16 == 0 &&
                       (uintptr_t)a.part % 16 == 0 && outs / 4 < (size_t)UINT32_MAX - 256 &&
                       (EPI != EPI_ROWSCALE || (uintptr_t)a.colScale % 16 == 0);
    if (quads)
        hipLaunchKernelGGL((mm_finish4_kernel<EPI>), dim3((unsigned)((outs / 4 + 255) / 256)), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL((mm_finish_kernel<EPI>), dim3((unsigned)((outs + 255) / 256)), dim3(256), 0, stream, a);
    return launch_status();
}

// K splits for a 128 x 128-tile GEMM whose grid has `tiles` blocks and
// `outs` outputs: doubled while the grid is under 512 blocks, the doubled
// count's partial sums stay within 32 MiB (the finish kernel reads them all),
// K divides, and each split keeps at least 4 K steps (at most 16;
// mm_split_count must agree with the scratch the caller sized). Measured on
// the GPTQ shapes at M = 256: K = 12288 -> N = 4096 takes 8 splits (98.7 ->
// 77 us), K = 4096 -> N = 12288 stays at 2.
int mm_split_count(long tiles, int KT, long outs) {
    int s = 1;
    while (s < 16 && tiles * s < 512 && (long)(2 * s) * outs * 4 <= (32L << 20) && KT % (2 * s) == 0 &&
           KT / (2 * s) >= 4)
        s *= 2;
    return s;
}

template <int WF, int EPI>
static int launch_by_m(F16GemmArgs a, hipStream_t stream) {
    // Measured on MI355X at K = 4096, N = 12288 (Q8B): M <= 16 in 32-row
    // blocks with K split 8 ways, 26.7 us; M = 32 / 64 36.9 / 41.5 us.
    if (a.M <= 16) return launch_f16gemm<WF, EPI, 1, 2, 1, 1, 8, 2>(a, stream);
    if (a.M <= 64) return launch_f16gemm<WF, EPI, 4, 2, 1, 2, 4, 2>(a, stream);
    if constexpr (WF != W_I8_TILE && WF != W_F16_TILE) {
        const long width = a.c1 - a.tileN0 * 16;
        // 256 x 256 block tiles when they fill the chip, loads two K steps
        // ahead (4096-row pass 78.0 -> 77.5 ms against one step; no spills).
        // A grid that is not whole rounds of the chip takes 256 x 256 tiles on
        // the columns that fill whole rounds and 256 x 128 tiles on the rest
        // (Qwen3-8B QKV at 4096 rows: 384 tiles as 256 + 256 half tiles,
        // 288.2 -> 159.9 + 99.1 us in a kernel trace; smaller tiles for the O
        // projection's single round measured slower: 205 -> 238-246 us with
        // its activation pack).
        const long big = (long)((a.M + 255) / 256) * ((width + 255) / 256);
        if (a.M >= 512 && big >= 256) {
            const long full = whole_round_cols256((a.M + 255) / 256, (width + 255) / 256);
            if (full == 0) return launch_f16gemm_big<WF, EPI, 256, 256, 4, 2, 2>(a, stream);
            F16GemmArgs b = a;
            b.c1 = (int)std::min<long>(a.c1, (long)a.tileN0 * 16 + full * 256);
            GPHQ_TRY((launch_f16gemm_big<WF, EPI, 256, 256, 4, 2, 2>(b, stream)));
            F16GemmArgs c = a;
            c.c0 = b.c1;
            c.tileN0 = c.c0 / 16;
            c.splits = 1;
            return launch_f16gemm_big<WF, EPI, 256, 128, 4, 2, 1>(c, stream);
        }
        // 128 x 128 tiles, with K split over extra blocks when the caller gave
        // scratch for the partial sums (store epilogues only).
        const long mid = (long)((a.M + 127) / 128) * ((width + 127) / 128);
        if constexpr (WF == W_GPTQ_ROW && EPI == EPI_PLAIN) {
            // 129..256 rows: one 256-row block per 128 columns with 2 K splits
            // when that makes at least 192 blocks (measured at M = 256, K = 4096
            // -> N = 12288: 66.8 -> 59.1 us; K = 12288 -> N = 4096 keeps 128 x 128
            // tiles and 8 splits). The caller's scratch covers the 128 x 128
            // split count, at least 2 here.
            if (a.M > 128 && a.M <= 256 && a.part && (width + 127) / 128 * 2 >= 192 &&
                mm_split_count(mid, a.KT, (long)a.M * (a.c1 - a.c0)) >= 2) {
                a.splits = 2;
                return launch_f16gemm_big<WF, EPI, 256, 128, 4, 2, 1>(a, stream);
            }
        }
        a.splits = 1;
        if constexpr (EPI == EPI_PLAIN || EPI == EPI_ROWSCALE)
            if (a.part) a.splits = mm_split_count(mid, a.KT, (long)a.M * (a.c1 - a.c0));
        if (mid * a.splits >= 128) return launch_f16gemm_big<WF, EPI, 128, 128, 2, 2, 2>(a, stream);
    }
    if constexpr (WF != W_I8_TILE && WF != W_F16_TILE) {
        // 256 x 128 block tiles when they fill the chip, else 128 x 128 or 128 x 64.
        const long ntiles = ((a.c1 + 15) / 16 - a.tileN0 + 7) / 8;
        if ((long)((a.M + 255) / 256) * ntiles >= 256) return launch_f16gemm_lds<WF, EPI, 4, 4, 4>(a, stream);
        if ((long)((a.M + 127) / 128) * ntiles >= 256) return launch_f16gemm_lds<WF, EPI, 4, 4, 2>(a, stream);
        return launch_f16gemm_lds<WF, EPI, 4, 2, 2>(a, stream);
    }
    return launch_f16gemm<WF, EPI, 4, 2, 2, 2, 1, 1>(a, stream);
}

// Dispatch over weight format and epilogue. All arguments were validated.
int f16gemm_launch(int wf, int epi, F16GemmArgs a, hipStream_t stream) {
    if (a.M == 0 || a.c0 >= a.c1) return GPHQ_OK;
    a.NT = (a.N + 15) / 16;
    a.tileN0 = a.c0 / 16;
#define GPHQ_F16_CASE(W, E) \
    if (wf == W && epi == E) return launch_by_m<W, E>(a, stream);
    GPHQ_F16_CASE(W_I8_TILE, EPI_PANELS)
    GPHQ_F16_CASE(W_F16_TILE, EPI_PANELS)
    GPHQ_F16_CASE(W_Q8_ROW, EPI_ROWSCALE)
    GPHQ_F16_CASE(W_Q8B_ROW, EPI_PLAIN)
    GPHQ_F16_CASE(W_Q4_ROW, EPI_PLAIN)
    GPHQ_F16_CASE(W_GPTQ_ROW, EPI_PLAIN)
    GPHQ_F16_CASE(W_Q8BF_ROW, EPI_PLAIN)
    GPHQ_F16_CASE(W_Q8_ROW, EPI_ADD)
    GPHQ_F16_CASE(W_Q8B_ROW, EPI_ADD)
    GPHQ_F16_CASE(W_Q8BF_ROW, EPI_ADD)
    GPHQ_F16_CASE(W_Q4_ROW, EPI_ADD)
    GPHQ_F16_CASE(W_Q8_ROW, EPI_SWIGLU)
    GPHQ_F16_CASE(W_Q8B_ROW, EPI_SWIGLU)
    GPHQ_F16_CASE(W_Q8BF_ROW, EPI_SWIGLU)
    GPHQ_F16_CASE(W_Q4_ROW, EPI_SWIGLU)
#undef GPHQ_F16_CASE
    return GPHQ_ERR_UNSUPPORTED;
}

// ---- activation packing ------------------------------------------------------
// Row scale of q8gemm Workspace.SetRowScale (gemm.go:127-135): 2^e with
// e = clamp(15 - exp(max), -100, 100) when max is finite and positive, else 1.
__device__ __forceinline__ void f16_row_scale(float m, float &scale, float &inv) {
    int e = 0;
    if (m > 0.0f && !isinf(m) && m == m) {
        int ex;
        (void)frexpf(m, &ex);
        e = min(max(15 - ex, -100), 100);
    }
    scale = ldexpf(1.0f, e);
    inv = ldexpf(1.0f, -e);
}

// One block per row. mode 0: q8gemm Workspace.Pack (power-of-two row scale from
// MaxAbs, then f16(x * scale)); mode 1: qwen3lm mm activations, half(x);
// mode 2: PackRange with the row scales already on the device, converting only
// columns [k0, k1) (and the K padding when k1 == K). Writes the FP16 tile
// layout; modes 0 and 1 convert whole rows and zero the K padding.
__global__ __launch_bounds__(256) void f16_act_pack_kernel(const float *__restrict__ x, long stride, int K, int kt,
                                                           int mode, int k0, int k1, _Float16 *__restrict__ act,
                                                           float *__restrict__ rowScale,
                                                           float *__restrict__ rowInv) {
    __shared__ float smax[4];
    __shared__ int snan[4];
    const int row = blockIdx.x;
    const float *xr = x + (size_t)row * stride;
    float scale = 1.0f, inv = 1.0f;
    if (mode == 0) {
        float m = 0.0f;
        int nan = 0;
        constexpr int UNR = 8;
        for (int kb = 0; kb < K; kb += 256 * UNR) {
            float v[UNR];
#pragma unroll
            for (int u = 0; u < UNR; ++u) {
                const int k = kb + u * 256 + (int)threadIdx.x;
                v[u] = k < K ? xr[k] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < UNR; ++u) {
                nan |= (v[u] != v[u]);
                m = fmaxf(m, fabsf(v[u]));
            }
        }
        for (int off = 32; off > 0; off >>= 1) {
            m = fmaxf(m, __shfl_xor(m, off));
            nan |= __shfl_xor(nan, off);
        }
        if ((threadIdx.x & 63) == 0) {
            smax[threadIdx.x >> 6] = m;
            snan[threadIdx.x >> 6] = nan;
        }
        __syncthreads();
        float mm = 0.0f;
        int anyNan = 0;
        for (int i = 0; i < (int)(blockDim.x >> 6); ++i) {
            mm = fmaxf(mm, smax[i]);
            anyNan |= snan[i];
        }
        if (anyNan) mm = __builtin_nanf("");
        f16_row_scale(mm, scale, inv);
        if (threadIdx.x == 0) {
            rowScale[row] = scale;
            rowInv[row] = inv;
        }
    } else if (mode == 2) {
        scale = rowScale[row];
    }
    if (mode != 2) {
        for (int c = threadIdx.x; c < kt * 4; c += blockDim.x) {
            const int kb = c * 16;
            f16x8 h[2];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int k = kb + i;
                h[i >> 3][i & 7] = k < K ? (_Float16)__fmul_rn(xr[k], scale) : (_Float16)0.0f;
            }
            const size_t off =
                ((size_t)(row >> 4) * kt + (kb >> 6)) * 1024 + (size_t)(((kb & 63) >> 4) * 16 + (row & 15)) * 16;
            *(f16x8 *)(act + off) = h[0];
            *(f16x8 *)(act + off + 8) = h[1];
        }
    } else {
        const int kend = (k1 == K) ? kt * 64 : k1;
        for (int k = k0 + (int)threadIdx.x; k < kend; k += blockDim.x) {
            const size_t off = ((size_t)(row >> 4) * kt + (k >> 6)) * 1024 +
                               (size_t)(((k & 63) >> 4) * 16 + (row & 15)) * 16 + (k & 15);
            act[off] = k < K ? (_Float16)__fmul_rn(xr[k], scale) : (_Float16)0.0f;
        }
    }
}

int f16_act_pack(const float *x, long stride, int rows, int K, int kt, int mode, int k0, int k1, _Float16 *act,
                 float *rowScale, float *rowInv, hipStream_t stream) {
    if (rows == 0) return GPHQ_OK;
    hipLaunchKernelGGL(f16_act_pack_kernel, dim3(rows), dim3(256), 0, stream, x, stride, K, kt, mode, k0, k1, act,
                       rowScale, rowInv);
    return launch_status();
}

// Whole-row activation packing held in registers: one block of 256 threads
// per row, thread t converting the 16-value chunks t, t + 256, ... (up to
// CPT of them), each read as four 16-byte loads and written as one 32-byte
// slot of the FP16 tile layout. MODE 0: half(x); 1: half(x * 2^e); 2:
// half(x * f * 2^e) with the RMSNorm factor f, as f16_act_pack_kernel modes
// 1, 4 and 3 (rowInv[row] = 2^-e for 1 and 2). K % 16 == 0, rows 16-byte
// aligned; chunks past K (up to the 64-value tile) are zero. ROT rotates the
// row first (rotate_row_lds: the down projection's online Hadamard).
template <int MODE, int CPT, bool ROT>
__global__ __launch_bounds__(256) void act_pack_rows_kernel(const float *__restrict__ x, long stride, int K, int kt,
                                                            float eps, const float *__restrict__ signs, int block,
                                                            _Float16 *__restrict__ act, float *__restrict__ rowInv,
                                                            int rows) {
    __shared__ float sss[4], smx[4];
    // The 4 rows whose 32-byte slots share a 128-byte line of the tiles go to
    // blocks b, b + 8, b + 16, b + 24, which the dispatcher places on one XCD
    // (round robin over 8), so each line is completed in one L2.
    const int bx = blockIdx.x, row = (bx & ~31) + 4 * (bx & 7) + ((bx >> 3) & 3);
    if (row >= rows) return;
    const float *xr = x + (size_t)row * stride;
    const int chunks = kt * 4;
    float4 v[CPT][4];
    float ss = 0.0f, mx = 0.0f;
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
            ss += v[c][q].x * v[c][q].x + v[c][q].y * v[c][q].y + v[c][q].z * v[c][q].z + v[c][q].w * v[c][q].w;
            mx = fmaxf(fmaxf(fmaxf(mx, fabsf(v[c][q].x)), fmaxf(fabsf(v[c][q].y), fabsf(v[c][q].z))), fabsf(v[c][q].w));
        }
    }
    float scale = 1.0f;
    if constexpr (MODE != 0) {
        ss = wave_sum(ss);
        for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
        if ((threadIdx.x & 63) == 0) {
            sss[threadIdx.x >> 6] = ss;
            smx[threadIdx.x >> 6] = mx;
        }
        __syncthreads();
        const float f = MODE == 2 ? 1.0f / sqrtf(((sss[0] + sss[1]) + (sss[2] + sss[3])) / (float)K + eps) : 1.0f;
        float rs, inv;
        f16_row_scale(fmaxf(fmaxf(smx[0], smx[1]), fmaxf(smx[2], smx[3])) * f, rs, inv);
        scale = f * rs;
        if (threadIdx.x == 0) rowInv[row] = inv;
    }
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int ch = (int)threadIdx.x + 256 * c;
        if (ch >= chunks) continue;
        f16x8 h[2];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            h[q >> 1][4 * (q & 1) + 0] = (_Float16)__fmul_rn(v[c][q].x, scale);
            h[q >> 1][4 * (q & 1) + 1] = (_Float16)__fmul_rn(v[c][q].y, scale);
            h[q >> 1][4 * (q & 1) + 2] = (_Float16)__fmul_rn(v[c][q].z, scale);
            h[q >> 1][4 * (q & 1) + 3] = (_Float16)__fmul_rn(v[c][q].w, scale);
        }
        const size_t off = ((size_t)(row >> 4) * kt + (ch >> 2)) * 1024 + (size_t)((ch & 3) * 16 + (row & 15)) * 16;
        *(f16x8 *)(act + off) = h[0];
        *(f16x8 *)(act + off + 8) = h[1];
    }
}

template <int MODE, bool ROT = false>
static int launch_act_pack_rows(const float *x, long stride, int rows, int K, float eps, _Float16 *act,
                                float *rowInv, hipStream_t stream, const float *signs = nullptr, int block = 0) {
    const int kt = (K + 63) / 64, chunks = kt * 4;
    // A rotated row takes rot_lds_bytes(K) of dynamic LDS (one 4096-value segment at a time, 16.6 KB).
    const size_t lds = ROT ? rot_lds_bytes(K) : 0;
#define GPHQ_ACTPACK(CPT)                                                                                              \
    do {                                                                                                               \
        if (lds > 65536)                                                                                               \
            (void)hipFuncSetAttribute((const void *)act_pack_rows_kernel<MODE, CPT, ROT>,                              \
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);                           \
        hipLaunchKernelGGL((act_pack_rows_kernel<MODE, CPT, ROT>), dim3((unsigned)((rows + 31) & ~31)), dim3(256), lds,\
                           stream, x, stride, K, kt, eps, signs, block, act, rowInv, rows);                            \
    } while (0)
    if (chunks <= 256)
        GPHQ_ACTPACK(1);
    else if (chunks <= 512)
        GPHQ_ACTPACK(2);
    else if (chunks <= 768)
        GPHQ_ACTPACK(3);
    else
        GPHQ_ACTPACK(4);
#undef GPHQ_ACTPACK
    return launch_status();
}

// The qwen3lm batched pass's activation tiles, half(x * f * 2^e) with f the
// RMSNorm factor (norm true) or 1, and rowInv[r] = 2^-e per row. x rows are
// `stride` floats apart, 16-byte aligned, K % 16 == 0, K <= 16384. signs
// (device, K values with the rotation's scale folded in) rotate each row
// first, in blocks of `block`; null for none.
int lm_act_pack(const float *x, long stride, int rows, int K, bool norm, float eps, const float *signs, int block,
                _Float16 *act, float *rowInv, hipStream_t stream) {
    if (rows == 0) return GPHQ_OK;
    if (signs) {
        if (norm) return GPHQ_ERR_UNSUPPORTED;  // no pass normalizes a rotated input
        return launch_act_pack_rows<1, true>(x, stride, rows, K, eps, act, rowInv, stream, signs, block);
    }
    if (norm) return launch_act_pack_rows<2>(x, stride, rows, K, eps, act, rowInv, stream);
    return launch_act_pack_rows<1>(x, stride, rows, K, eps, act, rowInv, stream);
}

// qwen3lm mm activations, half(x), through the register kernel when rows are
// 16-byte aligned and K <= 16384, else the general one.
int f16_act_pack_plain(const float *x, long stride, int rows, int K, _Float16 *act, hipStream_t stream) {
    if (rows == 0) return GPHQ_OK;
    if ((uintptr_t)x % 16 == 0 && stride % 4 == 0 && K % 16 == 0 && K <= 16384)
        return launch_act_pack_rows<0>(x, stride, rows, K, 0.0f, act, nullptr, stream);
    return f16_act_pack(x, stride, rows, K, (K + 63) / 64, 1, 0, K, act, nullptr, nullptr, stream);
}

// One projection of the qwen3lm batched pass over M activation rows packed
// by lm_act_pack (row sums scaled by rowInv): epi 0 stores y[M][N], 1 adds
// into y, 2 stores the SwiGLU of interleaved gate/up columns into y[M][N/2];
// y rows are y_stride floats apart. fmt is a GPHQ_FMT_* layer format.
// Arguments were validated.
int lm_mm_launch(int fmt, int epi, const void *codes, const void *scales, const _Float16 *act, const float *rowInv,
                 float *y, long y_stride, int M, int K, int N, hipStream_t stream) {
    F16GemmArgs a{};
    int wf;
    switch (fmt) {
    case GPHQ_FMT_Q8: wf = W_Q8_ROW; break;
    case GPHQ_FMT_Q8B: wf = W_Q8B_ROW; break;
    case GPHQ_FMT_Q8B_F32: wf = W_Q8BF_ROW; break;
    case GPHQ_FMT_Q4: wf = W_Q4_ROW; break;
    default: return GPHQ_ERR_UNSUPPORTED;
    }
    const bool q8 = fmt == GPHQ_FMT_Q8;
    int e;
    if (epi == 0)
        e = q8 ? EPI_ROWSCALE : EPI_PLAIN;
    else
        e = epi == 1 ? EPI_ADD : EPI_SWIGLU;
    a.A = act;
    a.B = codes;
    a.bScale = scales;
    a.colScale = q8 ? (const float *)scales : nullptr;
    a.rowInv = rowInv;
    a.dst = y;
    a.stride = y_stride;
    a.M = M;
    a.N = N;
    a.K = K;
    a.KT = (K + 63) / 64;
    a.c0 = 0;
    a.c1 = N;
    return f16gemm_launch(wf, e, a, stream);
}

// PackBF16Rows arithmetic (q8gemm/packed.go:148-174) for rows already known to
// be finite: per row, e = clamp(15 - exp(max|v|), -100, 100), values
// f16(v * 2^e) (round to nearest even), stored row scale 2^-e, and a count of
// values that did not convert exactly. One block per row; output row-major.
__global__ __launch_bounds__(256) void bf16_rows_to_f16_kernel(const uint16_t *__restrict__ src, int K,
                                                               uint16_t *__restrict__ dst, float *__restrict__ rowScale,
                                                               unsigned long long *__restrict__ rounded) {
    __shared__ float smax[4];
    __shared__ unsigned long long scount[4];
    const int row = blockIdx.x;
    const uint16_t *s = src + (size_t)row * K;
    float m = 0.0f;
    for (int k = threadIdx.x; k < K; k += blockDim.x)
        m = fmaxf(m, fabsf(__builtin_bit_cast(float, (uint32_t)s[k] << 16)));
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if ((threadIdx.x & 63) == 0) smax[threadIdx.x >> 6] = m;
    __syncthreads();
    float mm = 0.0f;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) mm = fmaxf(mm, smax[i]);
    int e = 0;
    if (mm > 0.0f) {
        int ex;
        (void)frexpf(mm, &ex);
        e = min(max(15 - ex, -100), 100);
    }
    const float scale = ldexpf(1.0f, e);
    if (threadIdx.x == 0) rowScale[row] = ldexpf(1.0f, -e);
    unsigned long long cnt = 0;
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
        const float v = __fmul_rn(__builtin_bit_cast(float, (uint32_t)s[k] << 16), scale);
        const _Float16 h = (_Float16)v;
        cnt += ((float)h != v);
        dst[(size_t)row * K + k] = __builtin_bit_cast(uint16_t, h);
    }
    for (int off = 32; off > 0; off >>= 1) cnt += __shfl_xor(cnt, off);
    if ((threadIdx.x & 63) == 0) scount[threadIdx.x >> 6] = cnt;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long t = 0;
        for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t += scount[i];
        atomicAdd(rounded, t);
    }
}

int bf16_rows_to_f16(const uint16_t *src, int rows, int K, uint16_t *dst, float *rowScale, unsigned long long *rounded,
                     hipStream_t stream) {
    if (rows == 0) return GPHQ_OK;
    hipLaunchKernelGGL(bf16_rows_to_f16_kernel, dim3(rows), dim3(256), 0, stream, src, K, dst, rowScale, rounded);
    return launch_status();
}

// FP16 weights (raw bits, row-major [rows][K]) -> FP16 tile layout.
__global__ void f16_pack_tiles_kernel(const uint16_t *__restrict__ src, uint16_t *__restrict__ dst, int rows, int K,
                                      int row0, int rowTiles, int kt) {
    const size_t chunk = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)rowTiles * kt * 64;
    if (chunk >= total) return;
    const int lane = (int)(chunk & 63);
    const size_t g = chunk >> 6;
    const int ktile = (int)(g % kt);
    const int rtile = (int)(g / kt) + (row0 >> 4);
    const int r = rtile * 16 + (lane & 15);
    const int rr = r - row0;
    if (rr < 0 || rr >= rows) return;
    const int kbase = ktile * 64 + (lane >> 4) * 16;
    uint16_t *d = dst + ((size_t)rtile * kt + ktile) * 1024 + (size_t)lane * 16;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int k = kbase + i;
        d[i] = k < K ? src[(size_t)rr * K + k] : (uint16_t)0;
    }
}

// The reference's FP16 panel layout [panel = row/64][K/2][64][2]
// (q8gemm/packed.go:233-239 at()) -> this library's tile layout, rows past n
// and K values past K zero. One thread per tile-layout lane (16 values).
__global__ void f16_ref_panels_to_tiles_kernel(const uint16_t *__restrict__ ref, uint16_t *__restrict__ dst, int n,
                                               int K, long pairs, int nt, int kt) {
    const size_t chunk = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)nt * kt * 64;
    if (chunk >= total) return;
    const int lane = (int)(chunk & 63);
    const size_t g = chunk >> 6;
    const int ktile = (int)(g % kt), rtile = (int)(g / kt);
    const int r = rtile * 16 + (lane & 15);
    const int kbase = ktile * 64 + (lane >> 4) * 16;
    uint16_t *d = dst + g * 1024 + (size_t)lane * 16;
    const uint16_t *panel = ref + (size_t)(r / 64) * pairs * 128 + (size_t)(r % 64) * 2;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int k = kbase + i;
        d[i] = (r < n && k < K) ? panel[(size_t)(k >> 1) * 128 + (k & 1)] : (uint16_t)0;
    }
}

int f16_ref_panels_to_tiles(const uint16_t *ref, uint16_t *dst, int n, int K, int nt, int kt, hipStream_t stream) {
    const size_t chunks = (size_t)nt * kt * 64;
    if (chunks == 0) return GPHQ_OK;
    hipLaunchKernelGGL(f16_ref_panels_to_tiles_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream,
                       ref, dst, n, K, (long)((K + 1) / 2), nt, kt);
    return launch_status();
}

int f16_pack_tiles(const uint16_t *src, uint16_t *dst, int rows, int K, int row0, int kt, hipStream_t stream) {
    if (rows == 0) return GPHQ_OK;
    const int rowTiles = ((row0 + rows + 15) >> 4) - (row0 >> 4);
    const size_t chunks = (size_t)rowTiles * kt * 64;
    hipLaunchKernelGGL(f16_pack_tiles_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream, src, dst,
                       rows, K, row0, rowTiles, kt);
    return launch_status();
}

}  // namespace gphq
