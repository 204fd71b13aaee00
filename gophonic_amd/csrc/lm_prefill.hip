// qwen3lm batched pass on MI355X: HiddenLastExtendInto's GPU path
// (qwen3lm/evaluator.go:146-262 -> gpuWorkspace.batch / batchPacked / pass /
// encodeBatch, gpu_darwin.go:1406-1480, 1574-1657, 1703-1764).
//
// A prefix-owned K/V cache is extended by n tokens in passes of up to the
// workspace's row capacity (the reference's gpuPositions = 2048 rows; here
// the caller picks it, e.g. a whole 4096-token prompt in one pass). A pass
// runs, per layer:
//   * the QKV projection over the RMS-normalized residual rows (the
//     activation tile packer computes each row's norm, gpu.metal:785-796);
//   * lm_qk_rope16_kernel: head RMSNorm and RoPE of every query and key head,
//     queries scaled by 1/sqrt(head_dim) in place, keys and values appended
//     at cache rows base + m (gpu.metal:1027-1056 qkRope);
//   * lm_kv_half_kernel: FP16 copies of the pass's 32-row K/V cache tiles,
//     converted once per layer for every query block of the next kernel;
//   * lm_flash_kernel: causal attention of each row m over cache rows
//     0 .. base + m (gpu.metal:1099-1240 attendFlash);
//   * the O projection added into the residual, the gate/up projection with
//     the norm prologue and the SwiGLU epilogue, the down input's Hadamard
//     (Q8 / Q4), and the down projection added into the residual.
// Projections run on the FP16 MFMA GEMM of gemm_f16.hip (FP16 weight and
// activation tiles, fp32 sums, the reference mm's arithmetic); a one-row pass
// takes the fp32 GEMV instead, as the reference's encodeTokens does
// (gpu_darwin.go:1605-1614). After the last pass the last row's final norm
// gives the caller's hidden state.
#include <math.h>

#include <algorithm>
#include <type_traits>
#include <vector>

#include "common.h"
#include "lm_model.h"

namespace gphq {
int gemv_fused_launch(int fmt, int pro, int epi, const void *codes, const void *scales, const float *x, float *y,
                      int K, int N, float eps, hipStream_t stream);
int lm_act_pack(const float *x, long stride, int rows, int K, bool norm, float eps, const float *signs, int block,
                _Float16 *act, float *rowInv, hipStream_t stream);
int lm_mm_launch(int fmt, int epi, const void *codes, const void *scales, const _Float16 *act, const float *rowInv,
                 float *y, long y_stride, int M, int K, int N, hipStream_t stream);
int lm_i8_act(const float *x, long stride, int rows, int K, bool norm, float eps, const float *signs, int block,
              int8_t *act, float *rowScale, hipStream_t stream);
int lm_i8_mm(int epi, const int8_t *act, const float *a_scale, const int8_t *codes, const float *w_scale, float *y,
             long y_stride, int M, int K, int N, hipStream_t stream);
}  // namespace gphq

using namespace gphq;

struct gphq_prefill {
    const gphq_lm *lm;
    int rows;  // tokens per pass, at most
    float *h, *qkv, *ctx, *act, *hn;
    _Float16 *a16;  // FP16 activation tiles [rows/16][K/64][64][16]
    float *rinv;    // per-row 2^-e of the activation tiles
    int32_t *tok, *nonfinite;
    int32_t *rowpos, *rowstart;  // packed passes: each row's position and its sequence's first row
    float *okc = nullptr, *ovc = nullptr;  // packed passes' own K/V [layers][rows][kv_dim], on first use
    _Float16 *kv16;  // FP16 K and V^T of the pass's 32-row cache tiles, per layer (lm_kv_half_kernel)
    int arith = GPHQ_PASS_FP16;
    int8_t *a8 = nullptr;  // int8 route: activations in 16-row tiles and their row scales, on first use
    float *s8 = nullptr;
    std::vector<void *> allocs;
};

namespace {

constexpr int kHeadDim = kLmHeadDim;
enum { PRO_PLAIN = 0, PRO_NORM = 1 };
enum { EPI_STORE = 0, EPI_ADD = 1, EPI_SWIGLU = 2 };

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct RopeArgs {
    float *qkv;             // [rows][qkvw]
    float *kc, *vc;         // this layer's cache [capacity][kvd]
    const int32_t *rowpos;  // packed pass: row m's position, K/V at cache row m
    const float *qn, *kn;   // head norm weights [128]
    const float *rope;      // cos [positions][64], sin at +sin_off
    float eps, qscale;
    int qkvw, qd, kvd, heads, kvh, base, sin_off;
};

// qkRope (gpu.metal:1027-1056): head RMSNorm and RoPE of every query and
// key head of row m = blockIdx.x, V rows copied to the cache. Row m sits at
// position base + m and cache row base + m, or, in a packed pass, at
// position rowpos[m] and cache row m. The block takes the row's head items
// (query heads, then key heads, then value heads) 16 at a time, four per
// wavefront; lane j of an item holds dims 4j..4j+3 and 64+4j..64+4j+3 as two
// 16-byte loads. Arithmetic of the decode step's attention kernel, so a key
// row written here equals the one a decode step would write: there lane l
// holds the rotary pair (l, l + 64) and the sum of squares is wave_sum's
// (lane pairs l^1, l^2, the 8- and 16-lane mirrors, then (row 0 + row 1) +
// (row 2 + row 3)). Here lane j holds lanes 4j..4j+3 of that layout, so the
// first two rounds happen in registers, the mirrors become the pairs j^1 and
// j^2 (each partial is a sum of the same two values, and fp32 addition
// commutes), and the last round is the pairs j^4 then j^8. Measured on
// MI355X against one wavefront per item (lane l holding l and l + 64, 4-byte
// loads): the same bits on both routes of a 4096-row Qwen3-8B pass, 42 us
// less per two layers on the FP16 route.
__global__ __launch_bounds__(256) void lm_qk_rope16_kernel(const RopeArgs a) {
    const int m = blockIdx.x, lane = threadIdx.x & 63;
    const int j = lane & 15, slot = threadIdx.x >> 4;  // 16 item slots per block
    const int items = a.heads + 2 * a.kvh;
    float *row = a.qkv + (size_t)m * a.qkvw;
    const int pos = a.rowpos ? a.rowpos[m] : a.base + m;
    const size_t cslot = (size_t)(a.rowpos ? m : pos) * a.kvd;
    const float4 c4 = *(const float4 *)(a.rope + (size_t)pos * 64 + 4 * j);
    const float4 s4 = *(const float4 *)(a.rope + a.sin_off + (size_t)pos * 64 + 4 * j);
    const float cs[4] = {c4.x, c4.y, c4.z, c4.w}, sn[4] = {s4.x, s4.y, s4.z, s4.w};
    for (int h0 = 0; h0 < items; h0 += 16) {
        const int h = h0 + slot;
        const bool live = h < items;
        const int hc = live ? h : items - 1;  // every lane takes part in the lane exchanges
        const bool isV = hc >= a.heads + a.kvh;
        const float *src = row + (isV ? a.qd + a.kvd + (size_t)(hc - a.heads - a.kvh) * kHeadDim
                                      : (size_t)hc * kHeadDim);
        const float4 u0 = *(const float4 *)(src + 4 * j), u1 = *(const float4 *)(src + 64 + 4 * j);
        if (isV) {
            if (live) {
                float *d = a.vc + cslot + (size_t)(hc - a.heads - a.kvh) * kHeadDim;
                *(float4 *)(d + 4 * j) = u0;
                *(float4 *)(d + 64 + 4 * j) = u1;
            }
            continue;  // uniform over the item's 16 lanes
        }
        const bool isQ = hc < a.heads;
        float x0[4] = {u0.x, u0.y, u0.z, u0.w}, x1[4] = {u1.x, u1.y, u1.z, u1.w};
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = x0[i] * x0[i] + x1[i] * x1[i];
        float v = (p[0] + p[1]) + (p[2] + p[3]);
        v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
        v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
        v += __shfl_xor(v, 4);
        v += __shfl_xor(v, 8);
        const float ss = v;
        const float inv = 1.0f / sqrtf(ss / (float)kHeadDim + a.eps);
        const float *w = isQ ? a.qn : a.kn;
        const float4 w0 = *(const float4 *)(w + 4 * j), w1 = *(const float4 *)(w + 64 + 4 * j);
        const float wa[4] = {w0.x, w0.y, w0.z, w0.w}, wb[4] = {w1.x, w1.y, w1.z, w1.w};
        float y0[4], y1[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a0 = x0[i] * (inv * wa[i]);
            const float a1 = x1[i] * (inv * wb[i]);
            y0[i] = a0 * cs[i] - a1 * sn[i];
            y1[i] = a1 * cs[i] + a0 * sn[i];
        }
        if (!live) continue;
        if (isQ) {
            float *d = row + (size_t)hc * kHeadDim;
            *(float4 *)(d + 4 * j) = float4{y0[0] * a.qscale, y0[1] * a.qscale, y0[2] * a.qscale, y0[3] * a.qscale};
            *(float4 *)(d + 64 + 4 * j) =
                float4{y1[0] * a.qscale, y1[1] * a.qscale, y1[2] * a.qscale, y1[3] * a.qscale};
        } else {
            float *d = a.kc + cslot + (size_t)(hc - a.heads) * kHeadDim;
            *(float4 *)(d + 4 * j) = float4{y0[0], y0[1], y0[2], y0[3]};
            *(float4 *)(d + 64 + 4 * j) = float4{y1[0], y1[1], y1[2], y1[3]};
        }
    }
}

// FP16 copies of a pass's K/V cache tiles for lm_flash_kernel, made once per
// layer instead of by every query block: absolute 32-row tiles k0 .. of the
// layer's cache (rows from kvEnd on are zero). Per (tile, KV head), K as
// [32 keys][128] and V^T as [128 dims][32 key positions] in the flash
// kernel's LDS key order; the same fp32 -> FP16 rounding the flash kernel
// applies to the fp32 tiles it stages itself, so attention's results do not
// change.
constexpr int kKvHalfTile = 2 * 32 * kHeadDim;  // halves per (tile, KV head): K then V^T
inline int kv16_tiles(int64_t rows) { return (int)((rows + 31) / 32 + 1); }  // any alignment of the pass rows

__global__ __launch_bounds__(256) void lm_kv_half_kernel(const float *__restrict__ kc, const float *__restrict__ vc,
                                                         int kvd, int k0, int kvEnd, _Float16 *__restrict__ out) {
    typedef _Float16 half4 __attribute__((ext_vector_type(4)));
    const int g = blockIdx.y, jb = (k0 + (int)blockIdx.x) * 32;
    _Float16 *kt = out + ((size_t)blockIdx.x * gridDim.y + g) * kKvHalfTile;
    _Float16 *vt = kt + 32 * kHeadDim;
    for (int u = threadIdx.x; u < 32 * kHeadDim / 4; u += 256) {
        const int key = u >> 5, d4 = 4 * (u & 31), j = jb + key;
        const float4 x = j < kvEnd ? *(const float4 *)(kc + (size_t)j * kvd + g * kHeadDim + d4)
                                   : float4{0.f, 0.f, 0.f, 0.f};
        *(half4 *)(kt + key * kHeadDim + d4) = half4{(_Float16)x.x, (_Float16)x.y, (_Float16)x.z, (_Float16)x.w};
    }
    // V: the tile's rows as FP16 into LDS ([key][dim]), then V^T rows of 16
    // bytes: dim d, key positions 8p .. 8p + 7, where position group pg holds
    // key group 4*(pg/4) + {0, 2, 1, 3}[pg % 4] (the map is its own inverse).
    __shared__ _Float16 vs[32][kHeadDim + 8];
    for (int u = threadIdx.x; u < 32 * kHeadDim / 4; u += 256) {
        const int key = u >> 5, d4 = 4 * (u & 31), j = jb + key;
        const float4 x = j < kvEnd ? *(const float4 *)(vc + (size_t)j * kvd + g * kHeadDim + d4)
                                   : float4{0.f, 0.f, 0.f, 0.f};
        *(half4 *)&vs[key][d4] = half4{(_Float16)x.x, (_Float16)x.y, (_Float16)x.z, (_Float16)x.w};
    }
    __syncthreads();
    typedef _Float16 half8v __attribute__((ext_vector_type(8)));
    for (int u = threadIdx.x; u < kHeadDim * 4; u += 256) {
        const int d = u >> 2, p = u & 3;
        half8v h;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int pos = 8 * p + i, pg = pos >> 2, r = pg & 3;
            const int kg = (pg & ~3) + ((r == 1) ? 2 : (r == 2) ? 1 : r);
            h[i] = vs[4 * kg + (pos & 3)][d];
        }
        *(half8v *)(vt + d * 32 + 8 * p) = h;
    }
}

struct FlashArgs {
    const float *qkv;        // [rows][qkvw], queries prepared by lm_qk_rope16_kernel
    const float *kc, *vc;    // this layer's cache [capacity][kvd] holding the pass's rows
    const float *pkc, *pvc;  // a shared prefix's cache rows [0, plen), seen by every row
    const int32_t *rowstart; // packed pass: the cache row where row m's sequence starts
    const _Float16 *kv16;    // FP16 copies of cache tiles k0.. (lm_kv_half_kernel), or null
    float *ctx;              // [rows][qd]
    int qkvw, qd, kvd, rows, base, plen, k0;
};

// Row block and KV head of a flash block. The grid is (row blocks, KV heads)
// and the hardware starts blocks in x-then-y order; numbered over the whole
// grid, the blocks are dealt out longest causal row block first across every
// KV head, so the long blocks of all heads start in the first wave and the
// short ones fill in behind them (4096 rows, Qwen3-8B heads, on MI355X: 288 ->
// 183 us per layer against row blocks dealt out per head).
__device__ __forceinline__ void flash_block(int nmb, int &mb, int &g) {
    const int lin = (int)(blockIdx.x + gridDim.x * blockIdx.y);
    mb = nmb - 1 - lin / (int)gridDim.y;
    g = lin % (int)gridDim.y;
}

// Causal attention of pass rows m0 .. m0 + 32*RH - 1 (m0 = 32*RH * row block)
// for the GROUP query heads of KV head g (flash_block): wavefront w takes
// query head g*GROUP + w % GROUP for rows m0 + 32*(w / GROUP) .. +31, and the
// block's waves share each 32-key tile of K and V, staged through LDS as
// FP16. Keys come in two segments: the shared prefix's rows 0 .. plen-1,
// which every row sees, then the pass's cache, where row m sees rows
// 0 .. base + m or, in a packed pass (attention items of batchPacked,
// gpu_darwin.go:1445-1500), rows rowstart[m] .. m of its own sequence.
//
// Per tile, on v_mfma_f32_32x32x16_f16 with fp32 accumulation:
//   S^T (32 keys x 32 queries) = K . Q^T, so lane l holds query l % 32 and 16
//     of its keys (the other 16 in lane l ^ 32): the online softmax needs one
//     lane exchange per reduction;
//   O^T (128 dims x 32 queries) += V^T . P^T, P^T taken straight from the
//     S^T registers (the MFMA's K index runs over the lane's own keys; V^T is
//     stored in LDS in the matching key order).
// Queries enter as half(q * log2(e)) (q already carries 1/sqrt(head_dim)), so
// the softmax is exp2(s - m) against a reference maximum m that moves only
// when a score exceeds it by more than 8; probabilities and values are FP16.
// The running output is rescaled only when some lane's reference moved.
template <int N, typename F, int I = 0>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, F, I + 1>(static_cast<F &&>(f));
    }
}

template <int GROUP, int RH, int PF>
__global__ __launch_bounds__(64 * RH * GROUP) void lm_flash_kernel(const FlashArgs a) {
    constexpr int NT = 64 * RH * GROUP;
    constexpr int RB = 32 * RH;  // rows per block
    constexpr int KB = 32;             // keys per tile
    constexpr int KS = kHeadDim + 8;   // K tile row stride (halves): conflict-free 16-byte reads
    constexpr int VS = KB + 8;         // V^T row stride (halves)
    constexpr int KITEMS = (KB * kHeadDim / 4 + NT - 1) / NT;  // float4 of K per thread
    constexpr int VITEMS = (KB / 4 * kHeadDim + NT - 1) / NT;  // (dim, 4 keys) of V per thread
    __shared__ _Float16 Ks[KB * KS];
    __shared__ _Float16 Vt[kHeadDim * VS];
    const int nmb = (a.rows + RB - 1) / RB;
    int mb, g;
    flash_block(nmb, mb, g);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int q = lane & 31, hi = lane >> 5;
    const int head = g * GROUP + wave % GROUP;
    const int m0 = mb * RB, mw = m0 + 32 * (wave / GROUP);
    const bool packed = a.rowstart != nullptr;
    const int off = packed ? 0 : a.base;  // cache row of pass row 0
    const int kvEnd = off + a.rows;       // cache rows written by this pass's qk_rope
    // Tiles: tA of the prefix, then the pass cache's from the block's first
    // visible row (rowstart never decreases along the pass) to its last row.
    const int tA = (a.plen + KB - 1) / KB;
    const int tb0 = (packed ? a.rowstart[m0] : 0) / KB;
    const int tiles = tA + (off + min(m0 + RB - 1, a.rows - 1)) / KB + 1 - tb0;
    const int myLast = off + mw + q;  // this lane's query sees pass-cache keys myFirst..myLast
    const int myFirst = packed ? a.rowstart[min(mw + q, a.rows - 1)] : 0;
    const int waveLast = off + mw + 31;  // no key past this is seen by the wave
    const int waveFirst = packed ? a.rowstart[min(mw, a.rows - 1)] : 0;
    const int waveFirstMax = packed ? a.rowstart[min(mw + 31, a.rows - 1)] : 0;
    const float *kbase = a.kc + (size_t)g * kHeadDim;
    const float *vbase = a.vc + (size_t)g * kHeadDim;
    const float *pkbase = a.pkc ? a.pkc + (size_t)g * kHeadDim : nullptr;
    const float *pvbase = a.pvc ? a.pvc + (size_t)g * kHeadDim : nullptr;
    auto tile_key = [&](int t) { return t < tA ? t * KB : (tb0 + t - tA) * KB; };

    half8 qf[8];
    {
        const float *qrow = a.qkv + (size_t)min(mw + q, a.rows - 1) * a.qkvw + (size_t)head * kHeadDim + 8 * hi;
        constexpr float kLog2e = 1.4426950408889634f;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const float4 x0 = *(const float4 *)(qrow + 16 * c), x1 = *(const float4 *)(qrow + 16 * c + 4);
            qf[c] = half8{(_Float16)(x0.x * kLog2e), (_Float16)(x0.y * kLog2e), (_Float16)(x0.z * kLog2e),
                          (_Float16)(x0.w * kLog2e), (_Float16)(x1.x * kLog2e), (_Float16)(x1.y * kLog2e),
                          (_Float16)(x1.z * kLog2e), (_Float16)(x1.w * kLog2e)};
        }
    }

    float4 kr[KITEMS];
    float4 vr[VITEMS];
    // Pass-cache tiles from k0 on come as FP16 copies (16-byte pieces, 512
    // of K and 512 of V^T per tile), loaded PF tiles ahead into PF register
    // sets (tile t in set t % PF); the prefix's and earlier rows' tiles, which
    // come first, are staged from the fp32 cache one tile ahead.
    constexpr int HITEMS = (32 * kHeadDim / 8 + NT - 1) / NT;
    typedef int i32x4v __attribute__((ext_vector_type(4)));
    i32x4v hk[PF][HITEMS], hv[PF][HITEMS];
    auto half_src = [&](int t) -> const _Float16 * {
        if (t < tA || !a.kv16) return nullptr;
        const int k = tb0 + t - tA;
        return k >= a.k0 ? a.kv16 + ((size_t)(k - a.k0) * gridDim.y + g) * kKvHalfTile : nullptr;
    };
    auto load_half = [&](const _Float16 *hs, auto set_c) __attribute__((always_inline)) {
        constexpr int S = decltype(set_c)::value;
#pragma unroll
        for (int i = 0; i < HITEMS; ++i) {
            const int idx = tid + i * NT;
            if (idx < 32 * kHeadDim / 8) {
                hk[S][i] = *(const i32x4v *)(hs + 8 * idx);
                hv[S][i] = *(const i32x4v *)(hs + 32 * kHeadDim + 8 * idx);
            }
        }
    };
    auto load_tile = [&](int t) __attribute__((always_inline)) {
        const bool inA = t < tA;
        const int jb = tile_key(t), end = inA ? a.plen : kvEnd;
        const float *kb = inA ? pkbase : kbase, *vb = inA ? pvbase : vbase;
#pragma unroll
        for (int i = 0; i < KITEMS; ++i) {
            const int idx = tid + i * NT;
            const int j = jb + (idx >> 5);
            kr[i] = (idx < KB * kHeadDim / 4 && j < end) ? *(const float4 *)(kb + (size_t)j * a.kvd + 4 * (idx & 31))
                                                         : float4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int i = 0; i < VITEMS; ++i) {
            const int idx = tid + i * NT;
            const int d = idx & (kHeadDim - 1), j = jb + 4 * (idx >> 7);
            float4 v{0.f, 0.f, 0.f, 0.f};
            if (idx < KB / 4 * kHeadDim) {
                const float *p = vb + (size_t)j * a.kvd + d;
                if (j < end) v.x = p[0];
                if (j + 1 < end) v.y = p[a.kvd];
                if (j + 2 < end) v.z = p[2 * (size_t)a.kvd];
                if (j + 3 < end) v.w = p[3 * (size_t)a.kvd];
            }
            vr[i] = v;
        }
    };
    auto store_tile = [&](int t, auto set_c) __attribute__((always_inline)) {
        constexpr int S = decltype(set_c)::value;
        if (half_src(t)) {
#pragma unroll
            for (int i = 0; i < HITEMS; ++i) {
                const int idx = tid + i * NT;
                if (idx < 32 * kHeadDim / 8) {
                    *(i32x4v *)(Ks + (idx >> 4) * KS + 8 * (idx & 15)) = hk[S][i];
                    *(i32x4v *)(Vt + (idx >> 2) * VS + 8 * (idx & 3)) = hv[S][i];
                }
            }
            return;
        }
        typedef _Float16 half4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int i = 0; i < KITEMS; ++i) {
            const int idx = tid + i * NT;
            if (idx < KB * kHeadDim / 4)
                *(half4 *)(Ks + (idx >> 5) * KS + 4 * (idx & 31)) =
                    half4{(_Float16)kr[i].x, (_Float16)kr[i].y, (_Float16)kr[i].z, (_Float16)kr[i].w};
        }
#pragma unroll
        for (int i = 0; i < VITEMS; ++i) {
            const int idx = tid + i * NT;
            if (idx < KB / 4 * kHeadDim) {
                // Key group kg (keys 4kg..4kg+3) goes to position group
                // 4*(kg/4) + {0, 2, 1, 3}[kg % 4]: in each 16-key half, LDS
                // positions 0..7 hold keys 0-3, 8-11 and positions 8..15 keys
                // 4-7, 12-15, the keys lanes 0-31 and 32-63 hold in S^T.
                const int d = idx & (kHeadDim - 1), kg = idx >> 7;
                const int r = kg & 3;
                const int pg = (kg & ~3) + ((r == 1) ? 2 : (r == 2) ? 1 : r);
                *(half4 *)(Vt + d * VS + 4 * pg) =
                    half4{(_Float16)vr[i].x, (_Float16)vr[i].y, (_Float16)vr[i].z, (_Float16)vr[i].w};
            }
        }
    };

    f32x16 o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = f32x16{};
    float mrun = -INFINITY, lrun = 0.0f;
    // Loads ahead of tile t: the next tile if it is an fp32 one, tile t + PF
    // if it is an FP16 one (into the set tile t has just left).
    auto prefetch = [&](int t, auto set_c) __attribute__((always_inline)) {
        if (t + 1 < tiles && !half_src(t + 1)) load_tile(t + 1);
        if (t + PF < tiles)
            if (const _Float16 *hs = half_src(t + PF)) load_half(hs, set_c);
    };
    if (!half_src(0)) load_tile(0);
    static_for<PF>([&](auto set_c) {
        if (decltype(set_c)::value < tiles)
            if (const _Float16 *hs = half_src(decltype(set_c)::value)) load_half(hs, set_c);
    });
    auto tile_step = [&](int t, auto set_c) __attribute__((always_inline)) {
        const bool inA = t < tA;
        const int jb = tile_key(t);
        __syncthreads();  // the previous tile's LDS reads are done
        store_tile(t, set_c);
        __syncthreads();
        prefetch(t, set_c);
        // Every key of the tile is outside this wave's rows' ranges.
        if (!inA && (jb > waveLast || jb + KB - 1 < waveFirst)) return;
        f32x16 s = f32x16{};
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const half8 kf = *(const half8 *)(Ks + q * KS + 16 * c + 8 * hi);
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[c], s, 0, 0, 0);
        }
        // s[r] is key jb + 8*(r/4) + 4*hi + r%4 of query row mw + q.
        if (inA) {
            if (jb + KB > a.plen) {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (jb + 8 * (r >> 2) + 4 * hi + (r & 3) >= a.plen) s[r] = -INFINITY;
            }
        } else if (jb + KB - 1 > off + mw || jb < waveFirstMax) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = jb + 8 * (r >> 2) + 4 * hi + (r & 3);
                if (key > myLast || key < myFirst) s[r] = -INFINITY;
            }
        }
        float mx = s[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        // The reference maximum moves only when a score passes it by more
        // than 8 (probabilities stay below 2^8, well inside FP16), so most
        // tiles skip the rescale. A query with no visible key yet (packed
        // passes) keeps mrun = -inf and takes its exponentials against 0, so
        // they stay 0, not NaN.
        const bool grew = mx > mrun + 8.0f;
        const float mnew = grew ? mx : mrun;
        const float msafe = mnew == -INFINITY ? 0.0f : mnew;
        const float corr = __builtin_amdgcn_exp2f(mrun - msafe);
        mrun = mnew;
        float p[16], rs = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            p[r] = __builtin_amdgcn_exp2f(s[r] - msafe);
            rs += p[r];
        }
        rs += __shfl_xor(rs, 32);
        lrun = lrun * corr + rs;
        half8 p0, p1;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            p0[i] = (_Float16)p[i];
            p1[i] = (_Float16)p[8 + i];
        }
        if (__any(grew)) {
#pragma unroll
            for (int c = 0; c < 4; ++c) o[c] *= corr;
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const _Float16 *vrow = Vt + (32 * c + q) * VS + 8 * hi;
            o[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(*(const half8 *)vrow, p0, o[c], 0, 0, 0);
            o[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(*(const half8 *)(vrow + 16), p1, o[c], 0, 0, 0);
        }
    };
    for (int t0 = 0; t0 < tiles; t0 += PF)
        static_for<PF>([&](auto set_c) {
            if (t0 + decltype(set_c)::value < tiles) tile_step(t0 + decltype(set_c)::value, set_c);
        });
    const int m = mw + q;
    if (m >= a.rows) return;
    const float inv = 1.0f / lrun;
    float *out = a.ctx + (size_t)m * a.qd + (size_t)head * kHeadDim + 4 * hi;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            *(float4 *)(out + 32 * c + 8 * j) = float4{o[c][4 * j] * inv, o[c][4 * j + 1] * inv,
                                                       o[c][4 * j + 2] * inv, o[c][4 * j + 3] * inv};
}

// lm_flash_kernel for a pass whose every key tile has an FP16 copy (no shared
// prefix, copies from cache tile 0: a first pass, or any packed pass), with
// the same per-tile arithmetic, taking two 32-key tiles per step: one
// barrier and one softmax update (one maximum exchange, one rescale) per 64
// keys, and two independent score MFMA chains. The results equal
// lm_flash_kernel's up to the rounding of the softmax sums and of the
// reference maximum's moves, which now happen per 64 keys: each lane keeps
// the sum over its own keys, and the lane pair (l, l ^ 32), which shares
// every reference maximum, adds its two sums once at the end instead of
// exchanging them per tile. A pair's second tile past the block's last is a
// copy of the last tile, masked out.
//
// What differs most is the load schedule. Every step loads exactly one pair
// (the index clamped to the last tile, so the last steps reload it), so the
// number of loads in flight is the same on every path and the compiler's wait
// before each LDS store covers only that pair's loads; in the general kernel,
// whose loads depend on the tile's source, the wait covered the next tile's
// loads too. Measured on MI355X at 4096 rows, per layer: 325 us before, 260
// with the one-tile version of this schedule, 174 with the longest-first
// block order (flash_block), 169 with two tiles per step. The pairs pass
// through two LDS buffers: pair u is computed from buffer u & 1 while pair
// u + 1 is stored into the other, one barrier per step.
template <int GROUP, int RH>
__global__ __launch_bounds__(64 * RH * GROUP) void lm_flash_half_kernel(const FlashArgs a) {
    constexpr int NT = 64 * RH * GROUP;
    constexpr int RB = 32 * RH;
    constexpr int KB = 32;
    constexpr int KS = kHeadDim + 8;
    constexpr int VS = KB + 8;
    constexpr int PF = 2;
    constexpr int HITEMS = (32 * kHeadDim / 8 + NT - 1) / NT;
    constexpr bool EVEN = (32 * kHeadDim / 8) % NT == 0;
    __shared__ _Float16 Ks2[2][2 * KB * KS];
    __shared__ _Float16 Vt2[2][2][kHeadDim * VS];
    const int nmb = (a.rows + RB - 1) / RB;
    int mb, g;
    flash_block(nmb, mb, g);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int q = lane & 31, hi = lane >> 5;
    const int head = g * GROUP + wave % GROUP;
    const int m0 = mb * RB, mw = m0 + 32 * (wave / GROUP);
    const bool packed = a.rowstart != nullptr;
    const int off = packed ? 0 : a.base;
    const int tb0 = (packed ? a.rowstart[m0] : 0) / KB;
    const int tiles = (off + min(m0 + RB - 1, a.rows - 1)) / KB + 1 - tb0;
    const int pairs = (tiles + 1) / 2;
    const int myLast = off + mw + q;
    const int myFirst = packed ? a.rowstart[min(mw + q, a.rows - 1)] : 0;
    const int waveLast = off + mw + 31;
    const int waveFirst = packed ? a.rowstart[min(mw, a.rows - 1)] : 0;
    const int waveFirstMax = packed ? a.rowstart[min(mw + 31, a.rows - 1)] : 0;
    const size_t tstride = (size_t)gridDim.y * kKvHalfTile;
    const _Float16 *kvh = a.kv16 + (size_t)tb0 * tstride + (size_t)g * kKvHalfTile;

    half8 qf[8];
    {
        const float *qrow = a.qkv + (size_t)min(mw + q, a.rows - 1) * a.qkvw + (size_t)head * kHeadDim + 8 * hi;
        constexpr float kLog2e = 1.4426950408889634f;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const float4 x0 = *(const float4 *)(qrow + 16 * c), x1 = *(const float4 *)(qrow + 16 * c + 4);
            qf[c] = half8{(_Float16)(x0.x * kLog2e), (_Float16)(x0.y * kLog2e), (_Float16)(x0.z * kLog2e),
                          (_Float16)(x0.w * kLog2e), (_Float16)(x1.x * kLog2e), (_Float16)(x1.y * kLog2e),
                          (_Float16)(x1.z * kLog2e), (_Float16)(x1.w * kLog2e)};
        }
    }
    typedef int i32x4v __attribute__((ext_vector_type(4)));
    i32x4v hk[PF][2][HITEMS], hv[PF][2][HITEMS];
    auto load_pair = [&](int u, auto set_c) __attribute__((always_inline)) {
        constexpr int S = decltype(set_c)::value;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const _Float16 *hs = kvh + (size_t)min(2 * u + h, tiles - 1) * tstride;
#pragma unroll
            for (int i = 0; i < HITEMS; ++i) {
                const int idx = tid + i * NT;
                if (EVEN || idx < 32 * kHeadDim / 8) {
                    hk[S][h][i] = *(const i32x4v *)(hs + 8 * idx);
                    hv[S][h][i] = *(const i32x4v *)(hs + 32 * kHeadDim + 8 * idx);
                }
            }
        }
    };
    auto store_pair = [&](auto set_c, int buf) __attribute__((always_inline)) {
        constexpr int S = decltype(set_c)::value;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < HITEMS; ++i) {
                const int idx = tid + i * NT;
                if (EVEN || idx < 32 * kHeadDim / 8) {
                    *(i32x4v *)(Ks2[buf] + (32 * h + (idx >> 4)) * KS + 8 * (idx & 15)) = hk[S][h][i];
                    *(i32x4v *)(Vt2[buf][h] + (idx >> 2) * VS + 8 * (idx & 3)) = hv[S][h][i];
                }
            }
    };

    f32x16 o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = f32x16{};
    float mrun = -INFINITY, lrun = 0.0f;
    auto compute = [&](int u, int buf) __attribute__((always_inline)) {
        const int jb = (tb0 + 2 * u) * KB;  // first key of the pair
        // Every key of the pair is outside this wave's rows' ranges.
        if (jb > waveLast || jb + 2 * KB - 1 < waveFirst) return;
        f32x16 s[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            s[h] = f32x16{};
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const half8 kf = *(const half8 *)(Ks2[buf] + (32 * h + q) * KS + 16 * c + 8 * hi);
                s[h] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[c], s[h], 0, 0, 0);
            }
        }
        // The pair's second tile past the block's last is a copy of the last.
        const int kend = (tb0 + tiles) * KB;
        if (jb + 2 * KB - 1 > off + mw || jb < waveFirstMax || jb + 2 * KB > kend) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = jb + 32 * h + 8 * (r >> 2) + 4 * hi + (r & 3);
                    if (key > myLast || key < myFirst || key >= kend) s[h][r] = -INFINITY;
                }
        }
        float mx = s[0][0];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[h][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const bool grew = mx > mrun + 8.0f;
        const float mnew = grew ? mx : mrun;
        const float msafe = mnew == -INFINITY ? 0.0f : mnew;
        const float corr = __builtin_amdgcn_exp2f(mrun - msafe);
        mrun = mnew;
        float rs = 0.0f;
        half8 p[2][2];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float e = __builtin_amdgcn_exp2f(s[h][r] - msafe);
                rs += e;
                p[h][r >> 3][r & 7] = (_Float16)e;
            }
        lrun = lrun * corr + rs;
        if (__any(grew)) {
#pragma unroll
            for (int c = 0; c < 4; ++c) o[c] *= corr;
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const _Float16 *vrow = Vt2[buf][h] + (32 * c + q) * VS + 8 * hi;
                o[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(*(const half8 *)vrow, p[h][0], o[c], 0, 0, 0);
                o[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(*(const half8 *)(vrow + 16), p[h][1], o[c], 0, 0, 0);
            }
    };
    static_for<PF>([&](auto set_c) { load_pair(decltype(set_c)::value, set_c); });
    store_pair(std::integral_constant<int, 0>{}, 0);
    load_pair(PF, std::integral_constant<int, 0>{});
    __syncthreads();
    for (int u0 = 0; u0 < pairs; u0 += PF)
        static_for<PF>([&](auto set_c) {
            constexpr int SN = (decltype(set_c)::value + 1) % PF;
            const int u = u0 + decltype(set_c)::value;
            if (u < pairs) compute(u, u & 1);
            store_pair(std::integral_constant<int, SN>{}, (u + 1) & 1);
            load_pair(u + 1 + PF, std::integral_constant<int, SN>{});
            __syncthreads();
        });
    lrun += __shfl_xor(lrun, 32);
    const int m = mw + q;
    if (m >= a.rows) return;
    const float inv = 1.0f / lrun;
    float *out = a.ctx + (size_t)m * a.qd + (size_t)head * kHeadDim + 4 * hi;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            *(float4 *)(out + 32 * c + 8 * j) = float4{o[c][4 * j] * inv, o[c][4 * j + 1] * inv,
                                                       o[c][4 * j + 2] * inv, o[c][4 * j + 3] * inv};
}

// Two 32-row halves per block up to four query heads per KV head (at most
// 512 threads, so no wave is limited to 128 registers), one above.
template <int G>
int launch_flash_g(const FlashArgs &a, int kvh, hipStream_t st) {
    constexpr int RH = G <= 4 ? 2 : 1;
    constexpr int PF = 2;  // FP16 tiles in flight (3 and 4 measured the same)
    const dim3 grid((unsigned)((a.rows + 32 * RH - 1) / (32 * RH)), (unsigned)kvh);
    if (a.plen == 0 && a.kv16 && a.k0 == 0)
        hipLaunchKernelGGL((lm_flash_half_kernel<G, RH>), grid, dim3(64 * RH * G), 0, st, a);
    else
        hipLaunchKernelGGL((lm_flash_kernel<G, RH, PF>), grid, dim3(64 * RH * G), 0, st, a);
    return launch_status();
}

int launch_flash(int group, const FlashArgs &a, int kvh, hipStream_t st) {
    switch (group) {
    case 1: return launch_flash_g<1>(a, kvh, st);
    case 2: return launch_flash_g<2>(a, kvh, st);
    case 3: return launch_flash_g<3>(a, kvh, st);
    case 4: return launch_flash_g<4>(a, kvh, st);
    case 5: return launch_flash_g<5>(a, kvh, st);
    case 6: return launch_flash_g<6>(a, kvh, st);
    case 7: return launch_flash_g<7>(a, kvh, st);
    case 8: return launch_flash_g<8>(a, kvh, st);
    }
    return GPHQ_ERR_UNSUPPORTED;
}

// One projection of a pass over R rows. FP16 route: the fp32 GEMV for one
// row, else the activation tiles (normalized for PRO_NORM) and the FP16 MFMA
// GEMM. int8 route (Q8 layers): every row quantized per row, then the exact
// int8 MFMA GEMM with MulPanelsI8's scaling. rot: the input is the down
// projection's, rotated first for Q8/Q4 layers (gpu_darwin.go:209-215) by the
// packer itself (in place, before the GEMV, for one row).
int project(gphq_prefill *ws, int R, int pro, int epi, const uint8_t *buf, int64_t codes, int64_t scales,
            const float *x, int64_t K, float *y, int64_t ystride, int64_t N, hipStream_t st, bool rot = false) {
    const gphq_lm *lm = ws->lm;
    const gphq_lm_config &c = lm->cfg;
    const float eps = (float)c.eps;
    const bool rotate = rot && c.fmt != GPHQ_FMT_Q8B;
    const float *signs = rotate ? lm->isigns : nullptr;
    const int block = rotate ? (int)lm->iblock : 0;
    if (ws->arith == GPHQ_PASS_INT8) {
        GPHQ_TRY(lm_i8_act(x, (long)K, R, (int)K, pro == PRO_NORM, eps, signs, block, ws->a8, ws->s8, st));
        return lm_i8_mm(epi, ws->a8, ws->s8, (const int8_t *)(buf + codes), (const float *)(buf + scales), y,
                        (long)ystride, R, (int)K, (int)N, st);
    }
    if (R == 1) {
        if (rotate) GPHQ_TRY(lm_rotate_launch(lm, const_cast<float *>(x), 1, (long)K, st));
        return gemv_fused_launch(c.fmt, pro, epi, buf + codes, buf + scales, x, y, (int)K, (int)N, eps, st);
    }
    GPHQ_TRY(lm_act_pack(x, (long)K, R, (int)K, pro == PRO_NORM, eps, signs, block, ws->a16, ws->rinv, st));
    return lm_mm_launch(c.fmt, epi, buf + codes, buf + scales, ws->a16, ws->rinv, y, (long)ystride, R, (int)K, (int)N,
                        st);
}

// Where a pass's keys and values live (layer 0; each layer is cap rows further).
struct PassKV {
    float *kc, *vc;          // the cache receiving the pass's rows
    int64_t cap;
    const float *pkc, *pvc;  // a shared, read-only prefix (or null)
    int64_t pcap;
    int plen;
    const int32_t *rowpos, *rowstart;  // packed pass: per-row position and sequence start (device)
};

// One pass: R tokens already in ws->tok, at cache rows base.. of kv.kc (or,
// packed, at rows 0..R-1 with per-row positions).
int encode_pass(gphq_prefill *ws, const PassKV &kv, int base, int R, hipStream_t st, const float *splice = nullptr) {
    const gphq_lm *lm = ws->lm;
    const gphq_lm_config &c = lm->cfg;
    const int64_t H = c.hidden, I = c.intermediate, qd = lm->qd, kvd = lm->kvd, qkvw = qd + 2 * kvd;
    GPHQ_TRY(lm_embed_launch(lm, ws->tok, R, ws->h, st, splice));
    RopeArgs ra{};
    ra.qkv = ws->qkv;
    ra.rope = lm->rope;
    ra.eps = (float)c.eps;
    ra.qscale = (float)(1.0 / sqrt((double)c.head_dim));
    ra.qkvw = (int)qkvw;
    ra.qd = (int)qd;
    ra.kvd = (int)kvd;
    ra.heads = (int)c.heads;
    ra.kvh = (int)c.kv_heads;
    ra.base = base;
    ra.sin_off = (int)(lm->positions * 64);
    ra.rowpos = kv.rowpos;
    FlashArgs fa{};
    fa.qkv = ws->qkv;
    fa.ctx = ws->ctx;
    fa.qkvw = (int)qkvw;
    fa.qd = (int)qd;
    fa.kvd = (int)kvd;
    fa.rows = R;
    fa.base = base;
    fa.plen = kv.plen;
    fa.rowstart = kv.rowstart;
    // The pass's cache rows (from row 0 in a packed pass) as FP16 tiles.
    const int kvOff = kv.rowstart ? 0 : base, kvEnd = kvOff + R;
    fa.kv16 = ws->kv16;
    fa.k0 = kvOff / 32;
    const int kvTiles = (kvEnd + 31) / 32 - fa.k0;
    for (int layer = 0; layer < c.layers; ++layer) {
        const gphq_lm_layer &L = lm->layers[layer];
        const uint8_t *buf = (const uint8_t *)L.buf_dev;
        GPHQ_TRY(project(ws, R, PRO_NORM, EPI_STORE, buf, L.qkv, L.qkv_scale, ws->h, H, ws->qkv, qkvw, qkvw, st));
        const size_t off = (size_t)layer * kv.cap * kvd;
        ra.kc = kv.kc + off;
        ra.vc = kv.vc + off;
        if (kv.plen > 0) {
            fa.pkc = kv.pkc + (size_t)layer * kv.pcap * kvd;
            fa.pvc = kv.pvc + (size_t)layer * kv.pcap * kvd;
        }
        ra.qn = lm->norms + (size_t)layer * 2 * kHeadDim;
        ra.kn = ra.qn + kHeadDim;
        hipLaunchKernelGGL(lm_qk_rope16_kernel, dim3((unsigned)R), dim3(256), 0, st, ra);
        GPHQ_TRY(launch_status());
        fa.kc = ra.kc;
        fa.vc = ra.vc;
        hipLaunchKernelGGL(lm_kv_half_kernel, dim3((unsigned)kvTiles, (unsigned)c.kv_heads), dim3(256), 0, st, fa.kc,
                           fa.vc, (int)kvd, fa.k0, kvEnd, ws->kv16);
        GPHQ_TRY(launch_status());
        GPHQ_TRY(launch_flash((int)lm->group, fa, (int)c.kv_heads, st));
        GPHQ_TRY(project(ws, R, PRO_PLAIN, EPI_ADD, buf, L.o, L.o_scale, ws->ctx, qd, ws->h, H, H, st));
        GPHQ_TRY(project(ws, R, PRO_NORM, EPI_SWIGLU, buf, L.gu, L.gu_scale, ws->h, H, ws->act, I, 2 * I, st));
        GPHQ_TRY(project(ws, R, PRO_PLAIN, EPI_ADD, buf, L.d, L.d_scale, ws->act, I, ws->h, H, H, st, true));
    }
    return GPHQ_OK;
}

void free_prefill(gphq_prefill *ws) {
    for (void *p : ws->allocs) (void)hipFree(p);
    delete ws;
}

}  // namespace

extern "C" {

int gphq_prefill_new(const gphq_lm *lm, int64_t rows, gphq_prefill **out) {
    if (!out) return GPHQ_ERR_DIMENSIONS;
    *out = nullptr;
    if (!lm) return GPHQ_ERR_WORKSPACE;
    if (rows < 1 || rows > GPHQ_PREFILL_MAX_ROWS) return GPHQ_ERR_DIMENSIONS;
    if (!lm_model_ready(lm)) return GPHQ_ERR_MODEL_INCOMPLETE;
    const gphq_lm_config &c = lm->cfg;
    gphq_prefill *ws = new gphq_prefill();
    ws->lm = lm;
    ws->rows = (int)rows;
    const int64_t H = c.hidden, I = c.intermediate, qkvw = lm->qd + 2 * lm->kvd;
    const int64_t kmax = std::max({H, lm->qd, I});
    const int64_t rpad = (rows + 15) / 16 * 16, kpad = (kmax + 63) / 64 * 64;
    struct {
        void **dst;
        size_t bytes;
    } bufs[] = {
        {(void **)&ws->h, (size_t)rows * H * 4},      {(void **)&ws->qkv, (size_t)rows * qkvw * 4},
        {(void **)&ws->ctx, (size_t)rows * lm->qd * 4}, {(void **)&ws->act, (size_t)rows * I * 4},
        {(void **)&ws->hn, (size_t)H * 4},            {(void **)&ws->a16, (size_t)rpad * kpad * 2},
        {(void **)&ws->tok, (size_t)rows * 4},        {(void **)&ws->nonfinite, 4},
        {(void **)&ws->rinv, (size_t)rows * 4},       {(void **)&ws->rowpos, (size_t)rows * 4},
        {(void **)&ws->rowstart, (size_t)rows * 4},
        {(void **)&ws->kv16, (size_t)kv16_tiles(rows) * c.kv_heads * kKvHalfTile * 2},
    };
    for (auto &b : bufs) {
        const hipError_t e = hipMalloc(b.dst, b.bytes);
        if (e != hipSuccess) {
            free_prefill(ws);
            return hip_status(e);
        }
        ws->allocs.push_back(*b.dst);
    }
    const hipError_t e = hipMemset(ws->nonfinite, 0, 4);
    if (e != hipSuccess) {
        free_prefill(ws);
        return hip_status(e);
    }
    *out = ws;
    return GPHQ_OK;
}

void gphq_prefill_free(gphq_prefill *ws) {
    if (ws) free_prefill(ws);
}

int gphq_prefill_rows(const gphq_prefill *ws) { return ws ? ws->rows : 0; }

int gphq_prefill_set_arith(gphq_prefill *ws, int arith) {
    if (!ws) return GPHQ_ERR_WORKSPACE;
    if (arith != GPHQ_PASS_FP16 && arith != GPHQ_PASS_INT8) return GPHQ_ERR_UNSUPPORTED;
    if (arith == GPHQ_PASS_INT8) {
        const gphq_lm *lm = ws->lm;
        if (lm->cfg.fmt != GPHQ_FMT_Q8) return GPHQ_ERR_UNSUPPORTED;
        // The int8 GEMM takes 64-deep K steps of 16-row activation tiles.
        if (lm->cfg.hidden % 64 || lm->qd % 64 || lm->cfg.intermediate % 64) return GPHQ_ERR_UNSUPPORTED;
        if (!ws->a8) {
            const int64_t kmax = std::max({(int64_t)lm->cfg.hidden, lm->qd, (int64_t)lm->cfg.intermediate});
            hipError_t e = hipMalloc((void **)&ws->a8, (size_t)((ws->rows + 15) / 16 * 16) * kmax);
            if (e != hipSuccess) {
                ws->a8 = nullptr;
                return hip_status(e);
            }
            ws->allocs.push_back(ws->a8);
            e = hipMalloc((void **)&ws->s8, (size_t)ws->rows * 4);
            if (e != hipSuccess) {
                ws->s8 = nullptr;
                return hip_status(e);
            }
            ws->allocs.push_back(ws->s8);
        }
    }
    ws->arith = arith;
    return GPHQ_OK;
}

int gphq_prefill_arith(const gphq_prefill *ws) { return ws ? ws->arith : GPHQ_PASS_FP16; }

int gphq_prefill_project(gphq_prefill *ws, int64_t layer, int proj, const float *x_dev, int64_t rows, float *y_dev,
                         void *stream) {
    if (!ws) return GPHQ_ERR_WORKSPACE;
    const gphq_lm *lm = ws->lm;
    const gphq_lm_config &c = lm->cfg;
    if (layer < 0 || layer >= c.layers || proj < 0 || proj > 3) return GPHQ_ERR_DIMENSIONS;
    if (rows < 1 || rows > ws->rows) return GPHQ_ERR_PASS_ROWS;
    if (!x_dev || !y_dev) return GPHQ_ERR_DIMENSIONS;
    const gphq_lm_layer &L = lm->layers[layer];
    const uint8_t *buf = (const uint8_t *)L.buf_dev;
    const int64_t H = c.hidden, I = c.intermediate, qd = lm->qd, qkvw = qd + 2 * lm->kvd;
    hipStream_t st = (hipStream_t)stream;
    const int R = (int)rows;
    switch (proj) {
    case 0: return project(ws, R, PRO_NORM, EPI_STORE, buf, L.qkv, L.qkv_scale, x_dev, H, y_dev, qkvw, qkvw, st);
    case 1: return project(ws, R, PRO_PLAIN, EPI_ADD, buf, L.o, L.o_scale, x_dev, qd, y_dev, H, H, st);
    case 2: return project(ws, R, PRO_NORM, EPI_SWIGLU, buf, L.gu, L.gu_scale, x_dev, H, y_dev, I, 2 * I, st);
    default: return project(ws, R, PRO_PLAIN, EPI_ADD, buf, L.d, L.d_scale, x_dev, I, y_dev, H, H, st, true);
    }
}

int gphq_prefill_extend(gphq_prefill *ws, gphq_prefix *kv, int64_t keep, const int32_t *tokens, int64_t n,
                        float *hidden_dev, int64_t hidden_len, void *stream) {
    // evaluator.go:178-194 then HiddenLastBatchInto's checks (540-560), in order.
    if (!ws || !ws->lm) return GPHQ_ERR_WORKSPACE;
    const gphq_lm *lm = ws->lm;
    if (!kv || kv->lm != lm || !kv->kc) return GPHQ_ERR_FOREIGN_PREFIX;
    if (keep < 0 || keep > kv->capacity) return GPHQ_ERR_KEEP_RANGE;
    if (n < 0 || keep + n > kv->capacity) return GPHQ_ERR_PREFIX_CAPACITY;
    if (n == 0 || !tokens) return GPHQ_ERR_EMPTY_SEQUENCE;
    if (keep + n > lm->cfg.max_positions || keep + n > lm->positions) return GPHQ_ERR_CONTEXT;
    if (!hidden_dev || hidden_len != lm->cfg.hidden) return GPHQ_ERR_DEST_WIDTH;
    for (int64_t i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= lm->cfg.vocab) return GPHQ_ERR_TOKEN_VOCAB;
    hipStream_t st = (hipStream_t)stream;
    const int64_t H = lm->cfg.hidden;
    // gpu_darwin.go:1460-1476: a sequence longer than a pass runs as
    // consecutive passes, each continuing the cache where the last stopped.
    int last = 0;
    for (int64_t off = 0; off < n; off += ws->rows) {
        const int R = (int)std::min<int64_t>(ws->rows, n - off);
        GPHQ_TRY(hip_status(
            hipMemcpyAsync(ws->tok, tokens + off, (size_t)R * sizeof(int32_t), hipMemcpyHostToDevice, st)));
        const PassKV pk{kv->kc, kv->vc, kv->capacity, nullptr, nullptr, 0, 0, nullptr, nullptr};
        GPHQ_TRY(encode_pass(ws, pk, (int)(keep + off), R, st));
        last = R;
    }
    return lm_final_launch(lm, ws->h + (size_t)(last - 1) * H, 1, hidden_dev, ws->hn, ws->nonfinite, st);
}

int gphq_prefill_extend_embed(gphq_prefill *ws, gphq_prefix *kv, int64_t stored, int64_t keep, int64_t reuse,
                              const int32_t *tokens, int64_t n, const gphq_embeds *embeds, float *tail_dev,
                              int64_t tail_len, void *stream) {
    // HiddenTailContinueEmbedInto (evaluator.go:293-310): the tail shape
    // first (a one-row tail is HiddenLast*, whose empty sequence is reported
    // by the batch checks below).
    if (!ws || !ws->lm) return GPHQ_ERR_WORKSPACE;
    const gphq_lm *lm = ws->lm;
    const gphq_lm_config &c = lm->cfg;
    const int64_t H = c.hidden;
    const int64_t k = tail_len / H;
    if (k == 0 || tail_len != k * H || k > GPHQ_TAIL_MAX_ROWS || (k > 1 && k > n)) return GPHQ_ERR_TAIL_SHAPE;
    // hiddenLastContinueEmbedInto (evaluator.go:182-213), in order.
    if (!kv || kv->lm != lm || !kv->kc) return GPHQ_ERR_FOREIGN_PREFIX;
    if (stored < 0 || stored > kv->capacity || keep < 0 || keep > stored) return GPHQ_ERR_KEEP_RANGE;
    if (n < 0 || keep + n > kv->capacity) return GPHQ_ERR_PREFIX_CAPACITY;
    if (reuse < 0 || reuse > stored - keep || reuse > n) return GPHQ_ERR_REUSE;
    // The GPU path recomputes every row (evaluator.go:197-199): a valid reuse
    // changes nothing.
    const bool splicing = embeds && embeds->rows_len != 0;
    if (splicing) {
        int64_t placeholders = 0;
        for (int64_t i = 0; i < n; ++i) placeholders += tokens && tokens[i] == embeds->token;
        if (embeds->rows_len != placeholders * H || !embeds->rows_dev) return GPHQ_ERR_EMBED_ROWS;
    }
    // HiddenLastBatchInto (evaluator.go:540-560) for the one sequence.
    if (n == 0 || !tokens) return GPHQ_ERR_EMPTY_SEQUENCE;
    if (keep + n > c.max_positions || keep + n > lm->positions) return GPHQ_ERR_CONTEXT;
    if (!tail_dev) return GPHQ_ERR_DEST_WIDTH;
    for (int64_t i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= c.vocab) return GPHQ_ERR_TOKEN_VOCAB;
    // The last pass holds the whole tail (gpu_darwin.go:1473-1479), so a
    // pass must have room for it.
    if (k > ws->rows) return GPHQ_ERR_PASS_ROWS;
    hipStream_t st = (hipStream_t)stream;
    // Placeholders become -1-j (row j of the splice table) in the device ids.
    std::vector<int32_t> ids(tokens, tokens + n);
    if (splicing) {
        int32_t j = 0;
        for (int32_t &t : ids)
            if (t == embeds->token) t = -1 - j++;
    }
    int last = 0;
    for (int64_t off = 0; off < n;) {
        int64_t R = std::min<int64_t>(ws->rows, n - off);
        const int64_t rest = n - off - R;
        if (rest > 0 && rest < k) R = n - off - k;
        GPHQ_TRY(hip_status(
            hipMemcpyAsync(ws->tok, ids.data() + off, (size_t)R * sizeof(int32_t), hipMemcpyHostToDevice, st)));
        const PassKV pk{kv->kc, kv->vc, kv->capacity, nullptr, nullptr, 0, 0, nullptr, nullptr};
        GPHQ_TRY(encode_pass(ws, pk, (int)(keep + off), (int)R, st, splicing ? embeds->rows_dev : nullptr));
        // The host ids are read before the next pass rewrites the device copy.
        if (off + R < n) GPHQ_TRY(hip_status(hipStreamSynchronize(st)));
        last = (int)R;
        off += R;
    }
    GPHQ_TRY(lm_final_launch(lm, ws->h + (size_t)(last - k) * H, (int)k, tail_dev, nullptr, ws->nonfinite, st, true));
    // `ids` is freed on return: wait for the last upload to have read it.
    return hip_status(hipStreamSynchronize(st));
}

int gphq_prefill_batch(gphq_prefill *ws, const gphq_prefix *shared, int64_t past, const int32_t *tokens,
                       const int64_t *lens, int64_t count, float *hidden_dev, int64_t hidden_len, void *stream) {
    if (!ws || !ws->lm) return GPHQ_ERR_WORKSPACE;
    const gphq_lm *lm = ws->lm;
    const gphq_lm_config &c = lm->cfg;
    // HiddenLastSharedInto (evaluator.go:413-419): the prefix is the caller's
    // and `past` is its token count.
    if (shared && (shared->lm != lm || !shared->kc)) return GPHQ_ERR_FOREIGN_PREFIX;
    if (past < 0 || past > (shared ? shared->capacity : 0)) return GPHQ_ERR_KEEP_RANGE;
    // HiddenLastBatchInto (evaluator.go:539-561), sequence by sequence.
    if (count < 1 || !lens) return GPHQ_ERR_SEQUENCE_COUNT;
    const int64_t H = c.hidden;
    int64_t total = 0;
    for (int64_t q = 0; q < count; ++q) {
        const int64_t n = lens[q];
        if (n < 1 || !tokens) return GPHQ_ERR_EMPTY_SEQUENCE;
        if (past + n > c.max_positions || past + n > lm->positions) return GPHQ_ERR_CONTEXT;
        if (!hidden_dev || hidden_len != count * H) return GPHQ_ERR_DEST_WIDTH;
        for (int64_t i = 0; i < n; ++i)
            if (tokens[total + i] < 0 || tokens[total + i] >= c.vocab) return GPHQ_ERR_TOKEN_VOCAB;
        total += n;
    }
    // batchPacked (gpu_darwin.go:1488-1496): a sequence must fit one pass.
    for (int64_t q = 0; q < count; ++q)
        if (lens[q] > ws->rows) return GPHQ_ERR_PASS_ROWS;
    hipStream_t st = (hipStream_t)stream;
    const int64_t kvd = lm->kvd;
    if (!ws->okc) {
        const size_t bytes = (size_t)c.layers * ws->rows * kvd * 4;
        float *k = nullptr, *v = nullptr;
        hipError_t e = hipMalloc(&k, bytes);
        if (e == hipSuccess) {
            e = hipMalloc(&v, bytes);
            if (e != hipSuccess) (void)hipFree(k);
        }
        if (e != hipSuccess) return hip_status(e);
        ws->okc = k;
        ws->ovc = v;
        ws->allocs.push_back(k);
        ws->allocs.push_back(v);
    }
    const PassKV pk{ws->okc,
                    ws->ovc,
                    ws->rows,
                    shared ? shared->kc : nullptr,
                    shared ? shared->vc : nullptr,
                    shared ? shared->capacity : 0,
                    (int)past,
                    ws->rowpos,
                    ws->rowstart};
    std::vector<int32_t> tok, pos, start;
    int64_t q0 = 0, t0 = 0;
    while (q0 < count) {
        // Sequences in order until the next would overflow the pass.
        int64_t q1 = q0, R = 0;
        while (q1 < count && R + lens[q1] <= ws->rows) R += lens[q1++];
        tok.assign(tokens + t0, tokens + t0 + R);
        pos.resize(R);
        start.resize(R);
        for (int64_t q = q0, r = 0; q < q1; ++q)
            for (int64_t i = 0; i < lens[q]; ++i, ++r) {
                pos[r] = (int32_t)(past + i);
                start[r] = (int32_t)(r - i);
            }
        GPHQ_TRY(hip_status(hipMemcpyAsync(ws->tok, tok.data(), R * 4, hipMemcpyHostToDevice, st)));
        GPHQ_TRY(hip_status(hipMemcpyAsync(ws->rowpos, pos.data(), R * 4, hipMemcpyHostToDevice, st)));
        GPHQ_TRY(hip_status(hipMemcpyAsync(ws->rowstart, start.data(), R * 4, hipMemcpyHostToDevice, st)));
        GPHQ_TRY(encode_pass(ws, pk, 0, (int)R, st));
        for (int64_t q = q0, r = 0; q < q1; ++q) {
            r += lens[q];
            GPHQ_TRY(lm_final_launch(lm, ws->h + (size_t)(r - 1) * H, 1, hidden_dev + q * H, ws->hn, ws->nonfinite,
                                     st));
        }
        // The host arrays are read before the next pass rewrites them.
        GPHQ_TRY(hip_status(hipStreamSynchronize(st)));
        t0 += R;
        q0 = q1;
    }
    return GPHQ_OK;
}

int gphq_prefill_check(gphq_prefill *ws, void *stream) {
    if (!ws) return GPHQ_ERR_WORKSPACE;
    hipStream_t st = (hipStream_t)stream;
    GPHQ_TRY(hip_status(hipStreamSynchronize(st)));
    int32_t bad = 0;
    GPHQ_TRY(hip_status(hipMemcpy(&bad, ws->nonfinite, 4, hipMemcpyDeviceToHost)));
    if (!bad) return GPHQ_OK;
    GPHQ_TRY(hip_status(hipMemset(ws->nonfinite, 0, 4)));
    return GPHQ_ERR_NON_FINITE_STATE;
}

}  // extern "C"
