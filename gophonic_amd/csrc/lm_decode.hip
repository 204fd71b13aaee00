// qwen3lm GPU decode provider on MI355X: the lane API of the reference's Metal
// backend (gpuModel / gpuPrefix / gpuDecodeBatchWorkspace,
// qwen3lm/gpu_darwin.go:62-102, 800-893, 731-759, 1046-1281) rebuilt for one
// gfx950 GPU.
//
// A step keeps everything on the device. The reference embeds tokens, applies
// the final norm and rotates on the host between two command buffers per step
// (gpu_darwin.go:1168-1258). Here:
//   * tokens and positions live in device memory. A "seed" kernel sets them
//     from the host arguments, and the argmax kernel writes each lane's next
//     token and advances its position. So one step's launch sequence is
//     identical from step to step, and a run of greedy steps needs no host
//     round trip (it can be replayed as a HIP graph);
//   * embedding gather + hidden rotation, final norm + rotations and the
//     argmax are kernels;
//   * per layer: QKV GEMV with the input RMSNorm fused (PRO_NORM),
//     attention, O GEMV added into the residual, gate/up GEMV with norm and
//     SwiGLU, the down input's Hadamard for Q8/Q4 weights, and the down GEMV
//     added into the residual (gpu.metal:1-14 describes the same six
//     dispatches);
//   * attention splits each lane's context 0..pos over up to `splits` blocks
//     per KV head (one launch fills the chip even at one lane). Each block
//     runs a streaming softmax over its keys for all query heads of the KV
//     head and writes a partial (max, sum, weighted V); a second small kernel
//     merges the partials of each query head in split order. (Merging in the
//     last block to finish needs device-scope fences and atomics, which cost
//     more on MI355X's per-XCD L2 caches than the extra launch.)
// Single-lane steps use the fp32 register GEMV (gemv.hip); steps with two or
// more lanes use the multi-vector MFMA GEMV (gemv_vec.hip), which reads each
// weight once for all lanes.
#include <math.h>

#include <algorithm>
#include <vector>

#include "common.h"
#include "lm_model.h"

namespace gphq {
int gemv_fused_launch(int fmt, int pro, int epi, const void *codes, const void *scales, const float *x, float *y,
                      int K, int N, float eps, hipStream_t stream);
int gemv_vec_fused_launch(int fmt, int norm, int epi, const void *codes, const void *scales, const float *x,
                          long xstride, float *y, long ystride, int V, int K, int N, float eps, void *work,
                          hipStream_t stream, float *split, size_t split_bytes, const VecFold &fold, VecFold *defer);
bool gemv_vec_prep_folds(int fmt, int V, int K);
size_t gemv_vec_split_bytes(int V, int K, int N);
size_t gemv_vec_workspace_bytes(int V, int K);
}  // namespace gphq

using namespace gphq;

namespace {

constexpr int kMaxLanes = GPHQ_DECODE_MAX_LANES;
constexpr int kHeadDim = kLmHeadDim;
constexpr int kPart = 2 + kHeadDim;  // one attention partial: max, sum, weighted V
constexpr int kMaxSplits = 32;  // attention blocks per (KV head, lane), at most
// Keys per attention block, at least. Measured on MI355X with 32 blocks per
// KV head: Qwen3-0.6B at contexts 1024-1280 0.714 ms per step with 64, 0.693
// with 80 or 96, 0.705 with 128; Qwen3-8B at 4096 (144 keys per block)
// unchanged.
constexpr int kMinChunk = 80;
constexpr int kMaxRotation = 4096;  // qwen3lm/hadamard.go:11
constexpr int kMaxWidth = 16384;    // hidden and intermediate widths (LDS)

enum { PRO_PLAIN = 0, PRO_NORM = 1 };
enum { EPI_STORE = 0, EPI_ADD = 1, EPI_SWIGLU = 2 };

// Sign*scale per value of newRotation(k) (multiplying by +-1 is exact, so
// x*(sign*scale) == (x*scale)*sign); returns the block.
int rotation_signs(int64_t k, std::vector<float> &out) {
    const int block = rotation_signs_pm1(k, out);
    const float scale = rotation_scale(block);
    for (float &v : out) v *= scale;
    return block;
}

// Bytes of one stored matrix's codes and scales (gpu_darwin.go:251-264).
void matrix_bytes(int fmt, int64_t rows, int64_t k, int64_t *codes, int64_t *scales) {
    *codes = fmt == GPHQ_FMT_Q4 ? rows * k / 2 : rows * k;
    if (fmt == GPHQ_FMT_Q8)
        *scales = 4 * rows;
    else if (fmt == GPHQ_FMT_Q8B_F32)
        *scales = 4 * rows * (k / 32);
    else
        *scales = 2 * rows * (k / 32);
}

int64_t align256(int64_t n) { return (n + 255) & ~(int64_t)255; }

}  // namespace

struct gphq_decode_batch {
    const gphq_lm *lm;
    int capacity;
    float *h, *qkv, *ctx, *act, *hn, *hidden, *logits, *part;
    uint32_t *cand;  // argmax candidates [lanes][parts][key, index]
    int32_t *tok, *pos, *start, *nonfinite;
    // [lanes][128]: cos then sin of the RoPE angles at the lane's current
    // position, written wherever the position is (seed and argmax kernels),
    // so attention loads them without first waiting for the position.
    float *rope_cur;
    void *vec_work;
    size_t vec_bytes;
    float *vec_split;  // partial sums of the K-split multi-vector GEMV
    size_t vec_split_bytes;
    int vec_min_lanes = 2;  // lane count from which GEMVs use the MFMA multi-vector kernel
    std::vector<void *> allocs;
    // One captured greedy step (gphq_decode_greedy_run), valid for the lane
    // prefixes and output pointers it was captured with.
    bool use_graph = true;
    hipStream_t capture = nullptr;
    hipGraphExec_t step_exec = nullptr;
    std::vector<gphq_prefix *> graph_kvs;
    std::vector<uint64_t> graph_kv_gens;  // the prefixes' generations at capture
    std::vector<int> graph_chunks;        // the attention key ranges its first loads expect
    uint64_t graph_lm_gen = 0;            // the model's binding generation at capture
    float *graph_hidden = nullptr;
    int32_t *graph_out = nullptr;
    int graph_vec_min = 0;
};

namespace {

// ---- kernels ---------------------------------------------------------------

// Deterministic block sum (fixed tree over the block's waves).
__device__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}

struct SeedArgs {
    int32_t tok[kMaxLanes];
    int32_t pos[kMaxLanes];
    int lanes;
    int32_t *tok_dev, *pos_dev, *start_dev;
    const float *rope;  // cos [positions][64], then sin at +sin_off
    float *rope_cur;
    int sin_off, positions;
};

__global__ void lm_seed_kernel(const SeedArgs a) {
    const int l = threadIdx.x;
    if (l < a.lanes) {
        a.tok_dev[l] = a.tok[l];
        a.pos_dev[l] = a.pos[l];
        a.start_dev[l] = a.pos[l];
    }
    for (int i = threadIdx.x; i < a.lanes * 128; i += blockDim.x) {
        const int l = i >> 7, t = i & 127, p = a.pos[l];
        if (p < a.positions)
            a.rope_cur[i] = t < 64 ? a.rope[(size_t)p * 64 + t] : a.rope[a.sin_off + (size_t)p * 64 + t - 64];
    }
}

// One block per lane: h = R . float32(bf16 embedding row of the lane's token)
// (weights.go:614-619 embedRow, then rotation.apply, gpu_darwin.go:1172-1174).
// With a splice table, a negative token -1-j takes row j of it (an Embeds
// row: fp32, unrotated, evaluator.go:155-163) in place of an embedding row.
__global__ __launch_bounds__(1024) void lm_embed_kernel(const uint16_t *__restrict__ embed,
                                                        const int32_t *__restrict__ tok, int vocab, int H,
                                                        const float *__restrict__ signs, int block,
                                                        float *__restrict__ h, const float *__restrict__ splice) {
    extern __shared__ float v[];
    const int lane = blockIdx.x;
    const int id = tok[lane];
    if (splice && id < 0) {
        const float *row = splice + (size_t)(-1 - id) * H;
        for (int i = threadIdx.x; i < H; i += blockDim.x) v[i] = row[i] * signs[i];
    } else {
        const int t = min(max(id, 0), vocab - 1);
        const uint16_t *row = embed + (size_t)t * H;
        for (int i = threadIdx.x; i < H; i += blockDim.x)
            v[i] = __builtin_bit_cast(float, (uint32_t)row[i] << 16) * signs[i];
    }
    __syncthreads();
    lds_fwht(v, H, block);
    for (int i = threadIdx.x; i < H; i += blockDim.x) h[(size_t)lane * H + i] = v[i];
}

// The online Hadamard of down's input (gpu.metal:339-367 rotate): grid
// (n/block, lanes); x[lane][b*block ..] = H . (signs*scale . x).
__global__ __launch_bounds__(512) void lm_rotate_kernel(float *__restrict__ x, int stride,
                                                        const float *__restrict__ signs, int block) {
    extern __shared__ float v[];
    float *base = x + (size_t)blockIdx.y * stride + (size_t)blockIdx.x * block;
    const float *sb = signs + (size_t)blockIdx.x * block;
    for (int i = threadIdx.x; i < block; i += blockDim.x) v[i] = base[i] * sb[i];
    __syncthreads();
    lds_fwht(v, block, block);
    for (int i = threadIdx.x; i < block; i += blockDim.x) base[i] = v[i];
}

// One block per lane (gpu_darwin.go:1241-1252): u = R^T h; hidden = u *
// float32(1/sqrt(mean(u^2) + eps)) * w (ops.go:251-254, mean and root in
// float64); hn = R hidden for the head (skipped when hn is null). Flags a
// non-finite hidden value in nonfinite[lane], or in nonfinite[0] for every
// lane when one_flag is set.
__global__ __launch_bounds__(1024) void lm_final_kernel(const float *__restrict__ h, int H,
                                                        const float *__restrict__ signs, int block,
                                                        const float *__restrict__ w, float eps,
                                                        float *__restrict__ hidden, float *__restrict__ hn,
                                                        int32_t *__restrict__ nonfinite, int one_flag) {
    extern __shared__ float v[];
    __shared__ float red[16];
    __shared__ int bad;
    const int lane = blockIdx.x;
    if (threadIdx.x == 0) bad = 0;
    for (int i = threadIdx.x; i < H; i += blockDim.x) v[i] = h[(size_t)lane * H + i];
    __syncthreads();
    lds_fwht(v, H, block);
    float ss = 0.0f;
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        const float u = v[i] * signs[i];
        v[i] = u;
        ss += u * u;
    }
    ss = block_sum(ss, red);
    const float inv = (float)(1.0 / sqrt((double)ss / (double)H + (double)eps));
    int any = 0;
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        const float o = v[i] * inv * w[i];
        any |= !isfinite(o);
        hidden[(size_t)lane * H + i] = o;
        v[i] = o * signs[i];
    }
    if (any) bad = 1;
    __syncthreads();
    if (hn) {
        lds_fwht(v, H, block);
        for (int i = threadIdx.x; i < H; i += blockDim.x) hn[(size_t)lane * H + i] = v[i];
    }
    if (threadIdx.x == 0 && bad) nonfinite[one_flag ? 0 : lane] = 1;
}

// Keys per attention block at a context of n keys: n spread over at most
// `splits` blocks, at least kMinChunk each, a multiple of 16; the blocks in
// use, ceil(n / chunk), are never empty and never more than `splits`. A
// function of n alone, so a step's attention sums in the same order however
// the steps are enqueued (one by one, or replayed from one captured graph).
__host__ __device__ inline int attn_chunk(int64_t n, int splits) {
    const int64_t chunk = (n + splits - 1) / splits;
    return (int)(chunk + 15 < kMinChunk ? kMinChunk : (chunk + 15) & ~15);
}

struct AttnArgs {
    const float *qkv;  // [lanes][qkvw]
    float *kc[kMaxLanes];
    float *vc[kMaxLanes];  // this layer's cache rows per lane, [capacity][kvd]
    const float *qn, *kn;  // this layer's head norms [128]
    const float *rope;     // cos [positions][64], then sin at +sin_off
    const float *rope_cur;  // [lanes][128], the rows of rope at each lane's position
    const int32_t *pos;    // [lanes]
    float *ctx;            // [lanes][qd]
    float *part;           // [lanes][kvh][splits][GROUP][kPart]
    int chunk[kMaxLanes];  // the expected keys per block (attn_chunk of the context the host expects)
    int cap[kMaxLanes];    // the lane's prefix capacity
    float eps, scale;
    int qkvw, qd, kvd, kvh, splits, sin_off;
};

// Merge factor of a base-2 softmax state with max m into one with max mn.
__device__ __forceinline__ float rescale(float m, float mn) { return m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mn); }

// attend1 (gpu.metal:392-466) split over the context: grid (splits, kvh,
// lanes), 4 wavefronts. Each of the block's 16 row groups of 16 lanes takes
// one key at a time; lane li of a group holds dims 4li..4li+3 and
// 64+4li..64+4li+3 of the key and value rows (two 16-byte loads, a group
// reads one 512-byte row). Softmax in base 2 (log2(e) folded into the
// queries). The loads for the norms are issued first, then the first keys',
// so the norms are computed while the keys are in flight; each iteration
// issues the next iteration's loads before its arithmetic. The new key
// (position pos, the last one) is taken from LDS by the block that holds it,
// after its cached keys. Keys stream through a ring of NB register buffers
// of KPI keys each: while one buffer is consumed the next NB-1 are in flight.
template <int GROUP, int KPI, int NB>
__global__ __launch_bounds__(256) void lm_attend_kernel(const AttnArgs a) {
    constexpr int NI = (GROUP + 4) / 4;  // norm items per wavefront, at most
    __shared__ float qs[GROUP][kHeadDim];
    __shared__ float knew[kHeadDim], vnew[kHeadDim];
    __shared__ float wm[4][GROUP], wl[4][GROUP];
    __shared__ float wacc[4][GROUP][kHeadDim];
    const int lid = blockIdx.z, g = blockIdx.y, sp = blockIdx.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int cap = a.cap[lid];
    // The key range follows from the position (attn_chunk); until it has
    // arrived, the keys of the range the host expects are loaded.
    int chunk = a.chunk[lid];
    int j0 = sp * chunk;
    int pos = a.pos[lid];
    const float *qkv = a.qkv + (size_t)lid * a.qkvw;
    float *kc = a.kc[lid] + g * kHeadDim;
    float *vc = a.vc[lid] + g * kHeadDim;
    const int sub = lane >> 4, li = lane & 15;
    const int rowgroup = wave * 4 + sub;  // 0..15
    const int d0 = li * 4, d1 = 64 + li * 4;

    const float rc = a.rope_cur[lid * 128 + lane], rs = a.rope_cur[lid * 128 + 64 + lane];
    // Norm inputs: item GROUP is the new key, the others the query heads.
    float x0[NI], x1[NI], w0[NI], w1[NI];
    float nv0 = 0.0f, nv1 = 0.0f;
#pragma unroll
    for (int ii = 0; ii < NI; ++ii) {
        const int item = wave + 4 * ii;
        x0[ii] = x1[ii] = w0[ii] = w1[ii] = 0.0f;
        if (item <= GROUP) {
            const bool isKey = item == GROUP;
            const float *src = isKey ? qkv + a.qd + g * kHeadDim : qkv + (size_t)(g * GROUP + item) * kHeadDim;
            const float *w = isKey ? a.kn : a.qn;
            x0[ii] = src[lane];
            x1[ii] = src[lane + 64];
            w0[ii] = w[lane];
            w1[ii] = w[lane + 64];
            if (isKey) {
                nv0 = qkv[a.qd + a.kvd + g * kHeadDim + lane];
                nv1 = qkv[a.qd + a.kvd + g * kHeadDim + lane + 64];
            }
        }
    }

    // Keys of step `it`: rows past the block's cached keys (jc, once the
    // position is known; the capacity before) load row 0 instead.
    float kb[NB][KPI][8], vb[NB][KPI][8];
    bool okb[NB][KPI];
    int jc = cap;
    auto load_keys = [&](int it, float (&kd)[KPI][8], float (&vd)[KPI][8], bool (&ok)[KPI]) {
#pragma unroll
        for (int u = 0; u < KPI; ++u) {
            const int j = j0 + (it * KPI + u) * 16 + rowgroup;
            ok[u] = j < jc;
            const int jj = ok[u] ? j : 0;
            const float4 k0 = *(const float4 *)(kc + (size_t)jj * a.kvd + d0);
            const float4 k1 = *(const float4 *)(kc + (size_t)jj * a.kvd + d1);
            const float4 v0 = *(const float4 *)(vc + (size_t)jj * a.kvd + d0);
            const float4 v1 = *(const float4 *)(vc + (size_t)jj * a.kvd + d1);
            kd[u][0] = k0.x, kd[u][1] = k0.y, kd[u][2] = k0.z, kd[u][3] = k0.w;
            kd[u][4] = k1.x, kd[u][5] = k1.y, kd[u][6] = k1.z, kd[u][7] = k1.w;
            vd[u][0] = v0.x, vd[u][1] = v0.y, vd[u][2] = v0.z, vd[u][3] = v0.w;
            vd[u][4] = v1.x, vd[u][5] = v1.y, vd[u][6] = v1.z, vd[u][7] = v1.w;
        }
    };
#pragma unroll
    for (int b = 0; b < NB; ++b) load_keys(b, kb[b], vb[b], okb[b]);
    // The position is used only once every load above has been issued: the
    // compiler otherwise moves its first use (and the wait for it) ahead of
    // the norm and key loads, which then start one memory round trip late.
    asm volatile("" : "+v"(pos));
    const int n = pos + 1;
    const int want = attn_chunk(n, a.splits);
    if (sp * want >= n) return;  // no keys of this lane's context
    if (want != chunk) {         // the expected range was another: load the block's own
        chunk = want;
        j0 = sp * chunk;
#pragma unroll
        for (int b = 0; b < NB; ++b) load_keys(b, kb[b], vb[b], okb[b]);
    }
    const int j1 = min(n, j0 + chunk);
    const bool owner = j1 == n;  // this block holds the new key
    jc = owner ? j1 - 1 : j1;    // cached keys [j0, jc)
    const int iters = (jc - j0 + 16 * KPI - 1) / (16 * KPI);
    // The ring's first rows past jc (loaded before the position arrived) are
    // zeroed, so masked keys never multiply stale cache contents.
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int u = 0; u < KPI; ++u) {
            okb[b][u] = j0 + (b * KPI + u) * 16 + rowgroup < jc;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                kb[b][u][i] = okb[b][u] ? kb[b][u][i] : 0.0f;
                vb[b][u][i] = okb[b][u] ? vb[b][u][i] : 0.0f;
            }
        }

    // Head RMSNorm and RoPE (gpu.metal:380-388 normRopeAt). Lane l holds the
    // rotary pair (l, l+64).
#pragma unroll
    for (int ii = 0; ii < NI; ++ii) {
        const int item = wave + 4 * ii;
        if (item > GROUP) continue;
        const bool isKey = item == GROUP;
        const float ss = wave_sum(x0[ii] * x0[ii] + x1[ii] * x1[ii]);
        const float inv = 1.0f / sqrtf(ss / (float)kHeadDim + a.eps);
        const float y0n = x0[ii] * (inv * w0[ii]), y1n = x1[ii] * (inv * w1[ii]);
        const float y0 = y0n * rc - y1n * rs, y1 = y1n * rc + y0n * rs;
        if (isKey) {
            knew[lane] = y0;
            knew[lane + 64] = y1;
            vnew[lane] = nv0;
            vnew[lane + 64] = nv1;
            if (owner) {  // this block appends the token's K/V row
                float *kd = kc + (size_t)pos * a.kvd, *vd = vc + (size_t)pos * a.kvd;
                kd[lane] = y0;
                kd[lane + 64] = y1;
                vd[lane] = nv0;
                vd[lane + 64] = nv1;
            }
        } else {
            const float qscale = a.scale * 1.4426950408889634f;
            qs[item][lane] = y0 * qscale;
            qs[item][lane + 64] = y1 * qscale;
        }
    }
    __syncthreads();

    float q[GROUP][8];
#pragma unroll
    for (int hh = 0; hh < GROUP; ++hh) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            q[hh][i] = qs[hh][d0 + i];
            q[hh][4 + i] = qs[hh][d1 + i];
        }
    }
    float m[GROUP], l[GROUP], acc[GROUP][8];
#pragma unroll
    for (int hh = 0; hh < GROUP; ++hh) {
        m[hh] = -INFINITY;
        l[hh] = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[hh][i] = 0.0f;
    }
    // One softmax step over KPI keys held by this row group.
    auto step = [&](const float (&kd)[KPI][8], const float (&vd)[KPI][8], const bool (&ok)[KPI]) {
#pragma unroll
        for (int hh = 0; hh < GROUP; ++hh) {
            float s[KPI];
            float bm = -INFINITY;
#pragma unroll
            for (int u = 0; u < KPI; ++u) {
                float p = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) p = fmaf(q[hh][i], kd[u][i], p);
                p = row16_sum(p);
                s[u] = ok[u] ? p : -INFINITY;
                bm = fmaxf(bm, s[u]);
            }
            const float mn = fmaxf(m[hh], bm);
            const float c = rescale(m[hh], mn);
            l[hh] *= c;
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[hh][i] *= c;
#pragma unroll
            for (int u = 0; u < KPI; ++u) {
                const float p = ok[u] ? __builtin_amdgcn_exp2f(s[u] - mn) : 0.0f;
                l[hh] += p;
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[hh][i] = fmaf(p, vd[u][i], acc[hh][i]);
            }
            m[hh] = mn;
        }
    };
    for (int it0 = 0; it0 < iters; it0 += NB) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (it0 + b < iters) step(kb[b], vb[b], okb[b]);
            // Every slot refills, past the block's keys too (rows past jc read
            // row 0 and are masked): with the same loads in flight on every
            // path the compiler waits only for the slot it consumes, where a
            // conditional refill made it wait for all of them (Qwen3-8B step
            // 2.369 -> 2.357 ms).
            load_keys(it0 + b + NB, kb[b], vb[b], okb[b]);
        }
    }
    if (owner) {  // the new key, on row group 0
#pragma unroll
        for (int u = 0; u < KPI; ++u) {
            okb[0][u] = u == 0 && rowgroup == 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                kb[0][u][i] = knew[d0 + i], kb[0][u][4 + i] = knew[d1 + i];
                vb[0][u][i] = vnew[d0 + i], vb[0][u][4 + i] = vnew[d1 + i];
            }
        }
        step(kb[0], vb[0], okb[0]);
    }
    // Merge the wave's four row groups (lanes l, l^16, l^32, l^48 hold the
    // same dims): xor 16, then xor 32.
#pragma unroll
    for (int off = 16; off <= 32; off <<= 1) {
#pragma unroll
        for (int hh = 0; hh < GROUP; ++hh) {
            const float mo = __shfl_xor(m[hh], off), lo = __shfl_xor(l[hh], off);
            const float mn = fmaxf(m[hh], mo);
            const float c = rescale(m[hh], mn), co = rescale(mo, mn);
            l[hh] = l[hh] * c + lo * co;
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[hh][i] = acc[hh][i] * c + __shfl_xor(acc[hh][i], off) * co;
            m[hh] = mn;
        }
    }
    if (sub == 0) {
#pragma unroll
        for (int hh = 0; hh < GROUP; ++hh) {
            if (li == 0) {
                wm[wave][hh] = m[hh];
                wl[wave][hh] = l[hh];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                wacc[wave][hh][d0 + i] = acc[hh][i];
                wacc[wave][hh][d1 + i] = acc[hh][4 + i];
            }
        }
    }
    __syncthreads();
    // The block's partial per query head, merged over its four waves.
    float *bp = a.part + ((((size_t)lid * a.kvh + g) * a.splits + sp) * GROUP) * kPart;
    for (int t = threadIdx.x; t < GROUP * kHeadDim; t += blockDim.x) {
        const int hh = t / kHeadDim, d = t % kHeadDim;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, wm[w][hh]);
        float L = 0.0f, A = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float c = rescale(wm[w][hh], M);
            L += wl[w][hh] * c;
            A += wacc[w][hh][d] * c;
        }
        bp[hh * kPart + 2 + d] = A;
        if (d == 0) {
            bp[hh * kPart] = M;
            bp[hh * kPart + 1] = L;
        }
    }
}

// The merge of attention's split partials (grid: q_heads, lanes; 128
// threads, thread d owns dim d): weights 2^(m_s - max) per split, then
// ctx = sum_s w_s A_s / sum_s w_s l_s, splits in order. Every load is issued
// up front (thread d reads dim d of all kMaxSplits slots, thread t the
// maximum and sum of slot t % kMaxSplits; the partial buffer holds
// kMaxSplits slots per head, so these stay inside it), and the position
// selects the splits in use afterwards, so the kernel waits for memory once.
__global__ __launch_bounds__(128) void lm_attn_merge_kernel(const AttnArgs a, int group) {
    __shared__ float cw[kMaxSplits];
    __shared__ float linv;
    const int h = blockIdx.x, lid = blockIdx.y;
    const int g = h / group, hh = h - g * group;
    int pos = a.pos[lid];
    const float *lp = a.part + (((size_t)lid * a.kvh + g) * a.splits * group + hh) * kPart;
    const size_t stride = (size_t)group * kPart;
    const int d = threadIdx.x;
    // Every slot is loaded with the position; the splits in use are
    // selected once it has arrived (the other slots hold stale values).
    float v[kMaxSplits];
#pragma unroll
    for (int s = 0; s < kMaxSplits; ++s) v[s] = lp[(size_t)s * stride + 2 + d];
    const int ts = threadIdx.x & (kMaxSplits - 1);
    float ms = lp[ts * stride], ls = lp[ts * stride + 1];
    asm volatile("" : "+v"(pos));  // first use after the loads (see lm_attend_kernel)
    const int chunk = attn_chunk(pos + 1, a.splits);
    const int used = (pos + 1 + chunk - 1) / chunk;
#pragma unroll
    for (int s = 0; s < kMaxSplits; ++s) v[s] = s < used ? v[s] : 0.0f;
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        const bool has = lane < used;
        ms = has ? ms : -INFINITY;
        ls = has ? ls : 0.0f;
        float M = ms;
        for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
        const float c = has ? rescale(ms, M) : 0.0f;
        const float L = wave_sum(ls * c);
        if (lane < kMaxSplits) cw[lane] = c;
        if (lane == 0) linv = 1.0f / L;
    }
    __syncthreads();
    float A = 0.0f;
#pragma unroll
    for (int s = 0; s < kMaxSplits; ++s) A = fmaf(cw[s], v[s], A);
    a.ctx[(size_t)lid * a.qd + (size_t)h * kHeadDim + d] = A * linv;
}

struct ArgmaxArgs {
    const float *logits;  // [lanes][stride], stride a multiple of 4
    int stride, vocab, lanes;
    int32_t *tok, *pos;
    const int32_t *start;
    int32_t *next;  // optional [lanes]
    int32_t *run;   // optional [steps][lanes], indexed by pos - start
    const float *rope;  // the RoPE table and the rows at the lanes' positions (SeedArgs)
    float *rope_cur;
    int sin_off, positions;
};

constexpr uint32_t kNone = 0xFFFFFFFFu;

// Orders candidates as greedy_argmax_rows does (gpu.metal:192-237): larger
// key first, then the smaller index; kNone never wins.
__device__ __forceinline__ bool better(uint32_t k, uint32_t i, uint32_t bk, uint32_t bi) {
    return i != kNone && (bi == kNone || k > bk || (k == bk && i < bi));
}

__device__ __forceinline__ void consider(float v, int i, uint32_t &bk, uint32_t &bi) {
    const uint32_t bits = __builtin_bit_cast(uint32_t, v);
    const uint32_t mag = bits & 0x7FFFFFFFu;
    if (mag <= 0x7F800000u) {  // NaNs never win; signed zeros tie
        const uint32_t key = mag == 0 ? 0x80000000u : ((bits & 0x80000000u) ? ~bits : bits ^ 0x80000000u);
        if (better(key, (uint32_t)i, bk, bi)) bk = key, bi = (uint32_t)i;
    }
}

// Best (key, index) over the wavefront's lanes, then over the block's
// wavefronts through LDS; the result lands in thread 0.
template <int NW>
__device__ __forceinline__ void block_best(uint32_t &bk, uint32_t &bi, uint32_t *sk, uint32_t *si) {
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t ko = __shfl_xor(bk, off), io = __shfl_xor(bi, off);
        if (better(ko, io, bk, bi)) bk = ko, bi = io;
    }
    if ((threadIdx.x & 63) == 0) {
        sk[threadIdx.x >> 6] = bk;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x != 0) return;
    bk = sk[0];
    bi = si[0];
#pragma unroll
    for (int w = 1; w < NW; ++w)
        if (better(sk[w], si[w], bk, bi)) bk = sk[w], bi = si[w];
}

// First-maximum argmax of each lane's logits (decode_batch.go:182-191
// greedyArgmax; a NaN at index 0 keeps index 0), in two launches: the
// logits of a lane are split over kArgParts blocks, each writing its best
// (key, index) to cand[lane][part]; then one block per lane takes the best
// candidate (the order is total: key, then index, so the split does not
// change the winner), writes the next token, feeds it back as the lane's
// current token and advances the lane's position.
constexpr int kArgParts = 128;

__global__ __launch_bounds__(256) void lm_argmax_part_kernel(const ArgmaxArgs a, uint32_t *cand) {
    __shared__ uint32_t sk[4], si[4];
    const int part = blockIdx.x, lane = blockIdx.y;
    const float *x = a.logits + (size_t)lane * a.stride;
    const int n4 = a.vocab >> 2, per = (n4 + kArgParts - 1) / kArgParts;
    const int u0 = part * per, u1 = min(n4, u0 + per);
    uint32_t bk = 0, bi = kNone;
    for (int u = u0 + threadIdx.x; u < u1; u += blockDim.x) {
        const float4 v = *((const float4 *)x + u);
        consider(v.x, 4 * u, bk, bi);
        consider(v.y, 4 * u + 1, bk, bi);
        consider(v.z, 4 * u + 2, bk, bi);
        consider(v.w, 4 * u + 3, bk, bi);
    }
    if (part == kArgParts - 1)
        for (int i = 4 * n4 + threadIdx.x; i < a.vocab; i += blockDim.x) consider(x[i], i, bk, bi);
    block_best<4>(bk, bi, sk, si);
    if (threadIdx.x == 0) {
        cand[((size_t)lane * kArgParts + part) * 2] = bk;
        cand[((size_t)lane * kArgParts + part) * 2 + 1] = bi;
    }
}

__global__ __launch_bounds__(128) void lm_argmax_kernel(const ArgmaxArgs a, const uint32_t *cand) {
    __shared__ uint32_t sk[2], si[2];
    const int lane = blockIdx.x;
    uint32_t bk = cand[((size_t)lane * kArgParts + threadIdx.x) * 2];
    uint32_t bi = cand[((size_t)lane * kArgParts + threadIdx.x) * 2 + 1];
    const uint32_t first = __builtin_bit_cast(uint32_t, a.logits[(size_t)lane * a.stride]) & 0x7FFFFFFFu;
    // The RoPE row of the next position (read by every thread before thread
    // 0 advances the position below, past block_best's barriers).
    static_assert(kArgParts == 128, "one thread per RoPE value of the row");
    const int32_t pn = a.pos[lane] + 1;
    if (pn < a.positions) {
        const int t = threadIdx.x;
        a.rope_cur[lane * 128 + t] = t < 64 ? a.rope[(size_t)pn * 64 + t] : a.rope[a.sin_off + (size_t)pn * 64 + t - 64];
    }
    block_best<2>(bk, bi, sk, si);
    if (threadIdx.x != 0) return;
    const int32_t token = (first > 0x7F800000u || bi == kNone) ? 0 : (int32_t)bi;
    const int32_t p = a.pos[lane];
    if (a.run) a.run[(size_t)(p - a.start[lane]) * a.lanes + lane] = token;
    if (a.next) a.next[lane] = token;
    a.tok[lane] = token;
    a.pos[lane] = p + 1;
}

// ---- host orchestration ----------------------------------------------------

template <int G>
int launch_attend_g(const AttnArgs &a, int lanes, hipStream_t st) {
    constexpr int KPI = G <= 4 ? 2 : 1;
    hipLaunchKernelGGL((lm_attend_kernel<G, KPI, 3>), dim3(a.splits, a.kvh, lanes), dim3(256), 0, st, a);
    return launch_status();
}

int launch_attend(int group, const AttnArgs &a, int lanes, hipStream_t st) {
    switch (group) {
    case 1: return launch_attend_g<1>(a, lanes, st);
    case 2: return launch_attend_g<2>(a, lanes, st);
    case 3: return launch_attend_g<3>(a, lanes, st);
    case 4: return launch_attend_g<4>(a, lanes, st);
    case 5: return launch_attend_g<5>(a, lanes, st);
    case 6: return launch_attend_g<6>(a, lanes, st);
    case 7: return launch_attend_g<7>(a, lanes, st);
    case 8: return launch_attend_g<8>(a, lanes, st);
    }
    return GPHQ_ERR_UNSUPPORTED;
}

// Attention blocks per (KV head, lane): about 256 blocks in all, at most
// kMaxSplits per head (measured on MI355X at contexts 512-4096 for 1, 4 and
// 16 lanes: more splits add merge work faster than they add bandwidth).
int attention_splits(const gphq_lm *lm, int lanes) {
    const int64_t work = lm->cfg.kv_heads * (int64_t)lanes;
    return (int)std::max<int64_t>(1, std::min<int64_t>(kMaxSplits, 256 / work));
}

// One projection GEMV of the step, single- or multi-lane. Multi-lane only:
// fold is a residual add left pending by the previous call (added to x by
// this call's preparation), and a K-split residual add given defer leaves
// its own finish to the next call (*defer).
int gemv(gphq_decode_batch *ws, int lanes, int fmt, int pro, int epi, const uint8_t *buf, int64_t codes,
         int64_t scales, const float *x, int64_t xs, float *y, int64_t ys, int64_t K, int64_t N, hipStream_t st,
         const VecFold &fold = VecFold{}, VecFold *defer = nullptr) {
    const float eps = (float)ws->lm->cfg.eps;
    if (defer) *defer = VecFold{};
    if (lanes < ws->vec_min_lanes) {
        if (fold.parts) return GPHQ_ERR_UNSUPPORTED;
        for (int l = 0; l < lanes; ++l)
            GPHQ_TRY(gemv_fused_launch(fmt, pro, epi, buf + codes, buf + scales, x + (size_t)l * xs,
                                       y + (size_t)l * ys, (int)K, (int)N, eps, st));
        return GPHQ_OK;
    }
    return gemv_vec_fused_launch(fmt, pro == PRO_NORM, epi, buf + codes, buf + scales, x, (long)xs, y, (long)ys, lanes,
                                 (int)K, (int)N, eps, ws->vec_work, st, ws->vec_split, ws->vec_split_bytes, fold,
                                 defer);
}

// Enqueues one decode step for `lanes` lanes whose tokens and positions are
// already in ws->tok / ws->pos. keys[l]: the context (position + 1) the host
// expects lane l's step to have, which sizes the attention blocks' first key
// loads; the blocks take their ranges from the device-side position. head:
// run the final norm, head and argmax; hidden_out receives each lane's
// post-final-norm state.
int encode_step(gphq_decode_batch *ws, gphq_prefix *const *kvs, int lanes, const int64_t *keys, bool head,
                float *hidden_out, int32_t *next_out, int32_t *run_out, hipStream_t st) {
    const gphq_lm *lm = ws->lm;
    const gphq_lm_config &c = lm->cfg;
    const int64_t H = c.hidden, I = c.intermediate, qkvw = lm->qd + 2 * lm->kvd;
    const int fmt = c.fmt;
    hipLaunchKernelGGL(lm_embed_kernel, dim3(lanes), dim3(1024), H * sizeof(float), st, lm->embed, ws->tok,
                       (int)c.vocab, (int)H, lm->hsigns, (int)lm->hblock, ws->h, (const float *)nullptr);
    GPHQ_TRY(launch_status());
    AttnArgs aa{};
    aa.qkv = ws->qkv;
    aa.rope = lm->rope;
    aa.rope_cur = ws->rope_cur;
    aa.pos = ws->pos;
    aa.ctx = ws->ctx;
    aa.part = ws->part;
    aa.eps = (float)c.eps;
    aa.scale = (float)(1.0 / sqrt((double)c.head_dim));
    aa.qkvw = (int)qkvw;
    aa.qd = (int)lm->qd;
    aa.kvd = (int)lm->kvd;
    aa.kvh = (int)c.kv_heads;
    aa.splits = attention_splits(lm, lanes);
    aa.sin_off = (int)(lm->positions * 64);
    // Multi-lane steps leave the K-split down projection's residual add to the
    // next layer's QKV preparation (one launch fewer per layer). Its partial
    // sums and scales stay in the workspace: the QKV preparation's own
    // fragments and scales (hidden-wide) end before the down projection's
    // scales (intermediate-wide) start.
    const bool fold_down = lanes >= ws->vec_min_lanes && H < I && gemv_vec_prep_folds(fmt, lanes, (int)H);
    VecFold pending{};
    for (int layer = 0; layer < c.layers; ++layer) {
        const gphq_lm_layer &L = lm->layers[layer];
        const uint8_t *buf = (const uint8_t *)L.buf_dev;
        GPHQ_TRY(gemv(ws, lanes, fmt, PRO_NORM, EPI_STORE, buf, L.qkv, L.qkv_scale, ws->h, H, ws->qkv, qkvw, H, qkvw,
                      st, pending));
        pending = VecFold{};
        for (int l = 0; l < lanes; ++l) {
            const size_t off = (size_t)layer * kvs[l]->capacity * lm->kvd;
            aa.kc[l] = kvs[l]->kc + off;
            aa.vc[l] = kvs[l]->vc + off;
            aa.chunk[l] = attn_chunk(keys[l], aa.splits);
            aa.cap[l] = (int)kvs[l]->capacity;
        }
        aa.qn = lm->norms + (size_t)layer * 2 * kHeadDim;
        aa.kn = aa.qn + kHeadDim;
        GPHQ_TRY(launch_attend((int)lm->group, aa, lanes, st));
        hipLaunchKernelGGL(lm_attn_merge_kernel, dim3((unsigned)c.heads, lanes), dim3(kHeadDim), 0, st, aa,
                           (int)lm->group);
        GPHQ_TRY(launch_status());
        GPHQ_TRY(gemv(ws, lanes, fmt, PRO_PLAIN, EPI_ADD, buf, L.o, L.o_scale, ws->ctx, lm->qd, ws->h, H, lm->qd, H,
                      st));
        GPHQ_TRY(gemv(ws, lanes, fmt, PRO_NORM, EPI_SWIGLU, buf, L.gu, L.gu_scale, ws->h, H, ws->act, I, H, 2 * I,
                      st));
        if (fmt != GPHQ_FMT_Q8B) {  // gpu_darwin.go:209-215: Q8B skips down's input rotation
            hipLaunchKernelGGL(lm_rotate_kernel, dim3((unsigned)(I / lm->iblock), lanes), dim3(512),
                               lm->iblock * sizeof(float), st, ws->act, (int)I, lm->isigns, (int)lm->iblock);
            GPHQ_TRY(launch_status());
        }
        const bool defer = fold_down && layer + 1 < c.layers;
        GPHQ_TRY(gemv(ws, lanes, fmt, PRO_PLAIN, EPI_ADD, buf, L.d, L.d_scale, ws->act, I, ws->h, H, I, H, st,
                      VecFold{}, defer ? &pending : nullptr));
    }
    if (!head) return GPHQ_OK;
    hipLaunchKernelGGL(lm_final_kernel, dim3(lanes), dim3(1024), H * sizeof(float), st, ws->h, (int)H, lm->hsigns,
                       (int)lm->hblock, lm->final_norm, (float)c.eps, hidden_out, ws->hn, ws->nonfinite, 0);
    GPHQ_TRY(launch_status());
    GPHQ_TRY(gemv(ws, lanes, GPHQ_FMT_Q8B, PRO_PLAIN, EPI_STORE, lm->head, 0, lm->head_scale, ws->hn, H, ws->logits,
                  lm->head_rows, H, lm->head_rows, st));
    ArgmaxArgs ga{ws->logits, (int)lm->head_rows, (int)c.vocab, lanes, ws->tok, ws->pos, ws->start, next_out, run_out,
                  lm->rope, ws->rope_cur, (int)(lm->positions * 64), (int)lm->positions};
    hipLaunchKernelGGL(lm_argmax_part_kernel, dim3(kArgParts, lanes), dim3(256), 0, st, ga, ws->cand);
    GPHQ_TRY(launch_status());
    hipLaunchKernelGGL(lm_argmax_kernel, dim3(lanes), dim3(kArgParts), 0, st, ga, (const uint32_t *)ws->cand);
    return launch_status();
}

int seed(gphq_decode_batch *ws, int lanes, const int64_t *positions, const int32_t *tokens, int64_t advance,
         hipStream_t st) {
    SeedArgs s{};
    for (int l = 0; l < lanes; ++l) {
        s.tok[l] = tokens[l];
        s.pos[l] = (int32_t)(positions[l] + advance);
    }
    s.lanes = lanes;
    s.tok_dev = ws->tok;
    s.pos_dev = ws->pos;
    s.start_dev = ws->start;
    s.rope = ws->lm->rope;
    s.rope_cur = ws->rope_cur;
    s.sin_off = (int)(ws->lm->positions * 64);
    s.positions = (int)ws->lm->positions;
    hipLaunchKernelGGL(lm_seed_kernel, dim3(1), dim3(64), 0, st, s);
    return launch_status();
}

bool overlaps(const void *a, int64_t an, const void *b, int64_t bn) {
    if (!a || !b || an <= 0 || bn <= 0) return false;
    const uintptr_t a0 = (uintptr_t)a, b0 = (uintptr_t)b;
    return a0 < b0 + (uintptr_t)bn && b0 < a0 + (uintptr_t)an;
}

// decode_batch.go:80-146 validateDecodeBatch, in the same order, for
// `steps` consecutive tokens per lane.
int validate(const gphq_decode_batch *ws, gphq_prefix *const *kvs, int64_t lanes, const int64_t *positions,
             const int32_t *tokens, int64_t steps, const float *hidden, int64_t hidden_len, const float *logits,
             const int32_t *next, bool need_head) {
    if (!ws || !ws->lm) return GPHQ_ERR_FOREIGN_WORKSPACE;
    const gphq_lm *lm = ws->lm;
    if (lanes < 1 || !kvs || !positions || !tokens || (need_head && (logits == nullptr) == (next == nullptr)))
        return GPHQ_ERR_BATCH_SHAPE;
    if (lanes > ws->capacity) return GPHQ_ERR_LANE_CAPACITY;
    for (int64_t l = 0; l < lanes; ++l) {
        const gphq_prefix *kv = kvs[l];
        if (!kv || kv->lm != lm || !kv->kc || kv->capacity < 1) return GPHQ_ERR_FOREIGN_PREFIX;
        for (int64_t p = 0; p < l; ++p)
            if (kvs[p] == kv) return GPHQ_ERR_DUPLICATE_PREFIX;
        if (positions[l] < 0 || positions[l] + steps > kv->capacity || positions[l] + steps > lm->positions)
            return GPHQ_ERR_PREFIX_FULL;
    }
    for (int64_t t = 0; t < steps; ++t)
        for (int64_t l = 0; l < lanes; ++l)
            if (tokens[t * lanes + l] < 0 || tokens[t * lanes + l] >= lm->cfg.vocab) return GPHQ_ERR_TOKEN_RANGE;
    const int64_t hb = lanes * lm->cfg.hidden * 4, lb = lanes * lm->cfg.vocab * 4, nb = lanes * 4;
    if (hidden && hidden_len < lanes * lm->cfg.hidden) return GPHQ_ERR_BATCH_SHAPE;
    if (overlaps(next, nb, hidden, hb) || overlaps(hidden, hb, logits, lb)) return GPHQ_ERR_OVERLAP;
    return GPHQ_OK;
}

bool model_ready(const gphq_lm *lm) {
    if (!lm->embed || !lm->head || !lm->final_norm) return false;
    for (char b : lm->bound)
        if (!b) return false;
    return true;
}

void drop_graph(gphq_decode_batch *ws) {
    if (ws->step_exec) (void)hipGraphExecDestroy(ws->step_exec);
    ws->step_exec = nullptr;
    ws->graph_kvs.clear();
    ws->graph_kv_gens.clear();
    ws->graph_chunks.clear();
}

void free_batch(gphq_decode_batch *ws) {
    drop_graph(ws);
    if (ws->capture) (void)hipStreamDestroy(ws->capture);
    for (void *p : ws->allocs) (void)hipFree(p);
    delete ws;
}

// Captures one chained greedy step (embed .. argmax) on the workspace's own
// stream into an executable graph, unless the cached one matches. Capture
// records the launches without running them.
// The cache key is the model's binding generation and each lane's prefix
// generation (a freed prefix's host address may come back from
// gphq_prefix_new with other K/V buffers; its generation does not), plus the
// output pointers and the GEMV mode.
bool graph_matches(const gphq_decode_batch *ws, gphq_prefix *const *kvs, int lanes, const int64_t *keys,
                   const float *hidden, const int32_t *out) {
    if (!ws->step_exec || (int)ws->graph_kvs.size() != lanes || ws->graph_hidden != hidden || ws->graph_out != out ||
        ws->graph_vec_min != ws->vec_min_lanes || ws->graph_lm_gen != ws->lm->gen)
        return false;
    for (int l = 0; l < lanes; ++l)
        if (ws->graph_kvs[(size_t)l] != kvs[l] || ws->graph_kv_gens[(size_t)l] != kvs[l]->gen ||
            ws->graph_chunks[(size_t)l] != attn_chunk(keys[l], attention_splits(ws->lm, lanes)))
            return false;
    return true;
}

int step_graph(gphq_decode_batch *ws, gphq_prefix *const *kvs, int lanes, const int64_t *keys, float *hidden,
               int32_t *out) {
    if (graph_matches(ws, kvs, lanes, keys, hidden, out)) return GPHQ_OK;
    drop_graph(ws);
    if (!ws->capture) GPHQ_TRY(hip_status(hipStreamCreateWithFlags(&ws->capture, hipStreamNonBlocking)));
    GPHQ_TRY(hip_status(hipStreamBeginCapture(ws->capture, hipStreamCaptureModeRelaxed)));
    const int st = encode_step(ws, kvs, lanes, keys, true, hidden, nullptr, out, ws->capture);
    hipGraph_t graph = nullptr;
    const hipError_t e = hipStreamEndCapture(ws->capture, &graph);
    if (st != GPHQ_OK || e != hipSuccess) {
        if (graph) (void)hipGraphDestroy(graph);
        return st != GPHQ_OK ? st : hip_status(e);
    }
    const hipError_t ie = hipGraphInstantiate(&ws->step_exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (ie != hipSuccess) {
        ws->step_exec = nullptr;
        return hip_status(ie);
    }
    ws->graph_kvs.assign(kvs, kvs + lanes);
    ws->graph_chunks.resize((size_t)lanes);
    for (int l = 0; l < lanes; ++l) ws->graph_chunks[(size_t)l] = attn_chunk(keys[l], attention_splits(ws->lm, lanes));
    ws->graph_kv_gens.resize((size_t)lanes);
    for (int l = 0; l < lanes; ++l) ws->graph_kv_gens[(size_t)l] = kvs[l]->gen;
    ws->graph_lm_gen = ws->lm->gen;
    ws->graph_hidden = hidden;
    ws->graph_out = out;
    ws->graph_vec_min = ws->vec_min_lanes;
    return GPHQ_OK;
}

}  // namespace

namespace gphq {

bool lm_model_ready(const gphq_lm *lm) { return model_ready(lm); }

int lm_embed_launch(const gphq_lm *lm, const int32_t *tok, int rows, float *h, hipStream_t st, const float *splice) {
    const int H = (int)lm->cfg.hidden;
    hipLaunchKernelGGL(lm_embed_kernel, dim3(rows), dim3(1024), H * sizeof(float), st, lm->embed, tok,
                       (int)lm->cfg.vocab, H, lm->hsigns, (int)lm->hblock, h, splice);
    return launch_status();
}

int lm_rotate_launch(const gphq_lm *lm, float *act, int rows, long stride, hipStream_t st) {
    const int64_t I = lm->cfg.intermediate;
    hipLaunchKernelGGL(lm_rotate_kernel, dim3((unsigned)(I / lm->iblock), rows), dim3(512),
                       lm->iblock * sizeof(float), st, act, (int)stride, lm->isigns, (int)lm->iblock);
    return launch_status();
}

int lm_final_launch(const gphq_lm *lm, const float *h, int rows, float *hidden, float *hn, int32_t *nonfinite,
                    hipStream_t st, bool one_flag) {
    const int H = (int)lm->cfg.hidden;
    hipLaunchKernelGGL(lm_final_kernel, dim3(rows), dim3(1024), H * sizeof(float), st, h, H, lm->hsigns,
                       (int)lm->hblock, lm->final_norm, (float)lm->cfg.eps, hidden, hn, nonfinite, one_flag ? 1 : 0);
    return launch_status();
}

}  // namespace gphq

extern "C" {

int gphq_lm_layer_layout(const gphq_lm_config *cfg, gphq_lm_layer *out, int64_t *bytes) {
    if (!cfg || !out || !bytes) return GPHQ_ERR_DIMENSIONS;
    const int fmt = cfg->fmt;
    if (fmt != GPHQ_FMT_Q8 && fmt != GPHQ_FMT_Q8B && fmt != GPHQ_FMT_Q8B_F32 && fmt != GPHQ_FMT_Q4)
        return GPHQ_ERR_UNSUPPORTED;
    const int64_t h = cfg->hidden, qd = cfg->heads * cfg->head_dim, kvd = cfg->kv_heads * cfg->head_dim,
                  inter = cfg->intermediate;
    if (h <= 0 || qd <= 0 || kvd <= 0 || inter <= 0 || h % 32 || qd % 32 || inter % 32) return GPHQ_ERR_DIMENSIONS;
    // gpu_darwin.go:251-283 place(): codes, then scales, each region 256-byte aligned.
    int64_t at = 0;
    auto place = [&](int64_t rows, int64_t k, int64_t *w, int64_t *s) {
        int64_t cb, sb;
        matrix_bytes(fmt, rows, k, &cb, &sb);
        *w = at;
        at = align256(at + cb);
        *s = at;
        at = align256(at + sb);
    };
    gphq_lm_layer L{};
    place(qd + 2 * kvd, h, &L.qkv, &L.qkv_scale);
    place(h, qd, &L.o, &L.o_scale);
    place(2 * inter, h, &L.gu, &L.gu_scale);
    place(h, inter, &L.d, &L.d_scale);
    L.buf_bytes = at;
    *out = L;
    *bytes = at;
    return GPHQ_OK;
}

int gphq_lm_head_layout(const gphq_lm_config *cfg, int64_t *rows, int64_t *scale_offset, int64_t *bytes) {
    if (!cfg || !rows || !scale_offset || !bytes || cfg->hidden <= 0 || cfg->hidden % 32 || cfg->vocab <= 0)
        return GPHQ_ERR_DIMENSIONS;
    // gpu_darwin.go:340-346 loadHead: rows padded to 16, Q8B codes then FP16 scales.
    const int64_t r = (cfg->vocab + 15) / 16 * 16;
    *rows = r;
    *scale_offset = align256(r * cfg->hidden);
    *bytes = *scale_offset + 2 * r * (cfg->hidden / 32);
    return GPHQ_OK;
}

int gphq_lm_new(const gphq_lm_config *cfg, gphq_lm **out) {
    if (!cfg || !out) return GPHQ_ERR_DIMENSIONS;
    *out = nullptr;
    const gphq_lm_config c = *cfg;
    if (c.fmt != GPHQ_FMT_Q8 && c.fmt != GPHQ_FMT_Q8B && c.fmt != GPHQ_FMT_Q8B_F32 && c.fmt != GPHQ_FMT_Q4)
        return GPHQ_ERR_UNSUPPORTED;
    // weights.go:672-680 readConfig plausibility.
    if (c.hidden <= 0 || c.layers <= 0 || c.heads <= 0 || c.kv_heads <= 0 || c.head_dim <= 0 || c.intermediate <= 0 ||
        c.vocab <= 0 || c.max_positions <= 0 || c.heads % c.kv_heads != 0 || c.head_dim % 2 != 0 || !(c.eps > 0) ||
        !(c.rope_theta > 0))
        return GPHQ_ERR_GEOMETRY;
    // gpu_darwin.go:116-129 gpuGeometry.
    const int64_t qd = c.heads * c.head_dim, kvd = c.kv_heads * c.head_dim, group = c.heads / c.kv_heads;
    int64_t iblock = 1;
    while (iblock < kMaxRotation && c.intermediate % (2 * iblock) == 0) iblock *= 2;
    if (c.head_dim != kHeadDim || group > 8 || c.hidden % 64 || c.intermediate % 64 || (qd + 2 * kvd) % 64 ||
        iblock < 64)
        return GPHQ_ERR_GEOMETRY;
    // Device limits of this implementation: one block holds a hidden vector
    // in LDS; int32 row and column indices.
    if (c.hidden > kMaxWidth || c.intermediate > kMaxWidth || qd > kMaxWidth || c.vocab > (1 << 28) ||
        c.layers > 4096)
        return GPHQ_ERR_GEOMETRY;
    gphq_lm *lm = new gphq_lm();
    lm->cfg = c;
    lm->qd = qd;
    lm->kvd = kvd;
    lm->group = group;
    lm->positions = std::min<int64_t>(c.max_positions, 1 << 16);  // gpu_darwin.go:33-35
    lm->layers.assign(c.layers, gphq_lm_layer{});
    lm->bound.assign(c.layers, 0);
    std::vector<float> hs, is;
    lm->hblock = rotation_signs(c.hidden, hs);
    lm->iblock = rotation_signs(c.intermediate, is);
    // gpu_darwin.go:232-241: float32(cos/sin(pos * invFreq[d])), float64 angles.
    const int64_t half = kHeadDim / 2;
    std::vector<float> rope((size_t)(2 * lm->positions * half));
    for (int64_t d = 0; d < half; ++d) {
        const double inv = 1.0 / pow(c.rope_theta, (double)(2 * d) / (double)c.head_dim);
        for (int64_t p = 0; p < lm->positions; ++p) {
            const double th = (double)p * inv;
            rope[(size_t)(p * half + d)] = (float)cos(th);
            rope[(size_t)(lm->positions * half + p * half + d)] = (float)sin(th);
        }
    }
    auto upload = [](float **dst, const std::vector<float> &src) {
        hipError_t e = hipMalloc(dst, src.size() * sizeof(float));
        if (e == hipSuccess) e = hipMemcpy(*dst, src.data(), src.size() * sizeof(float), hipMemcpyHostToDevice);
        return e;
    };
    hipError_t e = upload(&lm->rope, rope);
    if (e == hipSuccess) e = upload(&lm->hsigns, hs);
    if (e == hipSuccess) e = upload(&lm->isigns, is);
    if (e == hipSuccess) e = hipMalloc(&lm->norms, (size_t)c.layers * 2 * kHeadDim * sizeof(float));
    if (e != hipSuccess) {
        gphq_lm_free(lm);
        return hip_status(e);
    }
    *out = lm;
    return GPHQ_OK;
}

void gphq_lm_free(gphq_lm *lm) {
    if (!lm) return;
    for (float *p : {lm->norms, lm->rope, lm->hsigns, lm->isigns, lm->final_norm})
        if (p) (void)hipFree(p);
    delete lm;
}

int gphq_lm_bind_layer(gphq_lm *lm, int64_t layer, const gphq_lm_layer *desc) {
    if (!lm || !desc || layer < 0 || layer >= lm->cfg.layers || !desc->buf_dev || !desc->q_norm_host ||
        !desc->k_norm_host)
        return GPHQ_ERR_DIMENSIONS;
    const gphq_lm_config &c = lm->cfg;
    const int64_t h = c.hidden, inter = c.intermediate;
    struct Region {
        int64_t w, s, rows, k;
    } regs[4] = {{desc->qkv, desc->qkv_scale, lm->qd + 2 * lm->kvd, h},
                 {desc->o, desc->o_scale, h, lm->qd},
                 {desc->gu, desc->gu_scale, 2 * inter, h},
                 {desc->d, desc->d_scale, h, inter}};
    if ((uintptr_t)desc->buf_dev % 256) return GPHQ_ERR_DIMENSIONS;
    for (const Region &r : regs) {
        int64_t cb, sb;
        matrix_bytes(c.fmt, r.rows, r.k, &cb, &sb);
        if (r.w < 0 || r.s < 0 || r.w % 16 || r.s % 4 || r.w + cb > desc->buf_bytes || r.s + sb > desc->buf_bytes)
            return GPHQ_ERR_DIMENSIONS;
    }
    float norms[2 * kHeadDim];
    for (int i = 0; i < kHeadDim; ++i) {
        norms[i] = desc->q_norm_host[i];
        norms[kHeadDim + i] = desc->k_norm_host[i];
    }
    GPHQ_TRY(hip_status(hipMemcpy(lm->norms + (size_t)layer * 2 * kHeadDim, norms, sizeof(norms),
                                  hipMemcpyHostToDevice)));
    lm->layers[layer] = *desc;
    lm->layers[layer].q_norm_host = nullptr;
    lm->layers[layer].k_norm_host = nullptr;
    lm->bound[layer] = 1;
    lm->gen = next_generation();
    return GPHQ_OK;
}

int gphq_lm_bind_embed(gphq_lm *lm, const uint16_t *embed_dev, int64_t len) {
    if (!lm || !embed_dev || len != lm->cfg.vocab * lm->cfg.hidden) return GPHQ_ERR_DIMENSIONS;
    lm->embed = embed_dev;
    lm->gen = next_generation();
    return GPHQ_OK;
}

int gphq_lm_bind_head(gphq_lm *lm, const void *head_dev, int64_t bytes, const float *final_norm_host) {
    if (!lm || !head_dev || !final_norm_host || (uintptr_t)head_dev % 256) return GPHQ_ERR_DIMENSIONS;
    int64_t rows, so, need;
    GPHQ_TRY(gphq_lm_head_layout(&lm->cfg, &rows, &so, &need));
    if (bytes < need) return GPHQ_ERR_DIMENSIONS;
    if (!lm->final_norm) GPHQ_TRY(hip_status(hipMalloc(&lm->final_norm, lm->cfg.hidden * sizeof(float))));
    GPHQ_TRY(hip_status(
        hipMemcpy(lm->final_norm, final_norm_host, lm->cfg.hidden * sizeof(float), hipMemcpyHostToDevice)));
    lm->head = (const uint8_t *)head_dev;
    lm->head_rows = rows;
    lm->head_scale = so;
    lm->gen = next_generation();
    return GPHQ_OK;
}

int gphq_prefix_new(const gphq_lm *lm, int64_t capacity, gphq_prefix **out) {
    if (!lm || !out || capacity < 1) return GPHQ_ERR_DIMENSIONS;
    *out = nullptr;
    gphq_prefix *p = new gphq_prefix();
    p->lm = lm;
    p->capacity = capacity;
    p->gen = next_generation();
    const size_t n = (size_t)lm->cfg.layers * capacity * lm->kvd * sizeof(float);
    hipError_t e = hipMalloc(&p->kc, n);
    if (e == hipSuccess) e = hipMalloc(&p->vc, n);
    if (e == hipSuccess) e = hipMemset(p->kc, 0, n);
    if (e == hipSuccess) e = hipMemset(p->vc, 0, n);
    if (e != hipSuccess) {
        gphq_prefix_free(p);
        return hip_status(e);
    }
    *out = p;
    return GPHQ_OK;
}

void gphq_prefix_free(gphq_prefix *p) {
    if (!p) return;
    if (p->kc) (void)hipFree(p->kc);
    if (p->vc) (void)hipFree(p->vc);
    delete p;
}

int gphq_prefix_kv(const gphq_prefix *p, float **kc_dev, float **vc_dev, int64_t *capacity) {
    if (!p) return GPHQ_ERR_DIMENSIONS;
    if (kc_dev) *kc_dev = p->kc;
    if (vc_dev) *vc_dev = p->vc;
    if (capacity) *capacity = p->capacity;
    return GPHQ_OK;
}

int gphq_prefix_copy(gphq_prefix *dst, const gphq_prefix *src, int64_t n, void *stream) {
    if (!dst || !src || dst->lm != src->lm || n < 0 || n > dst->capacity || n > src->capacity)
        return GPHQ_ERR_DIMENSIONS;
    // gpu_darwin.go:873-881 copyFrom: the first n rows of each layer.
    const int64_t kvd = dst->lm->kvd, layers = dst->lm->cfg.layers;
    const size_t w = (size_t)n * kvd * sizeof(float);
    if (w == 0) return GPHQ_OK;
    const size_t dpitch = (size_t)dst->capacity * kvd * sizeof(float);
    const size_t spitch = (size_t)src->capacity * kvd * sizeof(float);
    GPHQ_TRY(hip_status(hipMemcpy2DAsync(dst->kc, dpitch, src->kc, spitch, w, (size_t)layers, hipMemcpyDeviceToDevice,
                                         (hipStream_t)stream)));
    return hip_status(hipMemcpy2DAsync(dst->vc, dpitch, src->vc, spitch, w, (size_t)layers, hipMemcpyDeviceToDevice,
                                       (hipStream_t)stream));
}

int gphq_decode_batch_new(const gphq_lm *lm, int64_t capacity, gphq_decode_batch **out) {
    if (!out) return GPHQ_ERR_DIMENSIONS;
    *out = nullptr;
    if (!lm) return GPHQ_ERR_FOREIGN_WORKSPACE;
    if (capacity < 1 || capacity > kMaxLanes) return GPHQ_ERR_LANE_CAPACITY;
    if (!model_ready(lm)) return GPHQ_ERR_MODEL_INCOMPLETE;
    const gphq_lm_config &c = lm->cfg;
    gphq_decode_batch *ws = new gphq_decode_batch();
    ws->lm = lm;
    ws->capacity = (int)capacity;
    const int64_t H = c.hidden, I = c.intermediate, qkvw = lm->qd + 2 * lm->kvd;
    const int64_t kmax = std::max({H, lm->qd, I});
    ws->vec_bytes = gemv_vec_workspace_bytes((int)capacity, (int)kmax);
    // Partial sums of the K-split multi-vector path (down: K = intermediate).
    ws->vec_split_bytes = std::max<size_t>(256, gemv_vec_split_bytes((int)std::min<int64_t>(capacity, 16), (int)I, (int)H));
    const size_t partFloats = (size_t)capacity * c.kv_heads * kMaxSplits * lm->group * kPart;
    struct {
        void **dst;
        size_t bytes;
    } bufs[] = {
        {(void **)&ws->h, (size_t)capacity * H * 4},
        {(void **)&ws->qkv, (size_t)capacity * qkvw * 4},
        {(void **)&ws->ctx, (size_t)capacity * lm->qd * 4},
        {(void **)&ws->act, (size_t)capacity * I * 4},
        {(void **)&ws->hn, (size_t)capacity * H * 4},
        {(void **)&ws->hidden, (size_t)capacity * H * 4},
        {(void **)&ws->logits, (size_t)capacity * lm->head_rows * 4},
        {(void **)&ws->part, partFloats * 4},
        {(void **)&ws->cand, (size_t)capacity * kArgParts * 8},
        {(void **)&ws->tok, (size_t)capacity * 4},
        {(void **)&ws->pos, (size_t)capacity * 4},
        {(void **)&ws->start, (size_t)capacity * 4},
        {(void **)&ws->rope_cur, (size_t)capacity * 128 * 4},
        {(void **)&ws->nonfinite, (size_t)capacity * 4},
        {(void **)&ws->vec_work, ws->vec_bytes},
        {(void **)&ws->vec_split, ws->vec_split_bytes},
    };
    for (auto &b : bufs) {
        hipError_t e = hipMalloc(b.dst, b.bytes);
        if (e == hipSuccess) {
            ws->allocs.push_back(*b.dst);
            e = hipMemset(*b.dst, 0, b.bytes);  // counters start at zero; scratch is defined
        }
        if (e != hipSuccess) {
            free_batch(ws);
            return hip_status(e);
        }
    }
    *out = ws;
    return GPHQ_OK;
}

void gphq_decode_batch_free(gphq_decode_batch *ws) {
    if (ws) free_batch(ws);
}

int gphq_decode_batch_set_vec_min_lanes(gphq_decode_batch *ws, int64_t lanes) {
    if (!ws || lanes < 1) return GPHQ_ERR_DIMENSIONS;
    ws->vec_min_lanes = (int)std::min<int64_t>(lanes, kMaxLanes + 1);
    return GPHQ_OK;
}

int gphq_decode_batch_into(gphq_decode_batch *ws, gphq_prefix *const *kvs, int64_t lanes, const int64_t *positions,
                           const int32_t *tokens, float *hidden_dev, int64_t hidden_len, float *logits_dev,
                           int64_t logits_len, void *stream) {
    GPHQ_TRY(validate(ws, kvs, lanes, positions, tokens, 1, hidden_dev, hidden_len, logits_dev, nullptr, true));
    if (!hidden_dev || logits_len < lanes * ws->lm->cfg.vocab) return GPHQ_ERR_BATCH_SHAPE;
    hipStream_t st = (hipStream_t)stream;
    GPHQ_TRY(seed(ws, (int)lanes, positions, tokens, 0, st));
    int64_t keys[kMaxLanes];
    for (int64_t l = 0; l < lanes; ++l) keys[l] = positions[l] + 1;
    GPHQ_TRY(encode_step(ws, kvs, (int)lanes, keys, true, hidden_dev, nullptr, nullptr, st));
    const gphq_lm *lm = ws->lm;
    return hip_status(hipMemcpy2DAsync(logits_dev, (size_t)lm->cfg.vocab * 4, ws->logits, (size_t)lm->head_rows * 4,
                                       (size_t)lm->cfg.vocab * 4, (size_t)lanes, hipMemcpyDeviceToDevice, st));
}

int gphq_decode_batch_greedy_into(gphq_decode_batch *ws, gphq_prefix *const *kvs, int64_t lanes,
                                  const int64_t *positions, const int32_t *tokens, float *hidden_dev,
                                  int64_t hidden_len, int32_t *next_dev, void *stream) {
    GPHQ_TRY(validate(ws, kvs, lanes, positions, tokens, 1, hidden_dev, hidden_len, nullptr, next_dev, true));
    if (!hidden_dev) return GPHQ_ERR_BATCH_SHAPE;
    hipStream_t st = (hipStream_t)stream;
    GPHQ_TRY(seed(ws, (int)lanes, positions, tokens, 0, st));
    int64_t keys[kMaxLanes];
    for (int64_t l = 0; l < lanes; ++l) keys[l] = positions[l] + 1;
    return encode_step(ws, kvs, (int)lanes, keys, true, hidden_dev, next_dev, nullptr, st);
}

int gphq_decode_greedy_run(gphq_decode_batch *ws, gphq_prefix *const *kvs, int64_t lanes, const int64_t *positions,
                           const int32_t *tokens, int64_t steps, int32_t *tokens_out_dev, int64_t tokens_out_len,
                           float *hidden_dev, int64_t hidden_len, void *stream) {
    if (steps < 1 || !tokens_out_dev || tokens_out_len < steps * lanes) return GPHQ_ERR_BATCH_SHAPE;
    GPHQ_TRY(validate(ws, kvs, lanes, positions, tokens, 1, hidden_dev, hidden_len, nullptr, tokens_out_dev, true));
    // Every step's position must fit the prefixes and the RoPE table.
    for (int64_t l = 0; l < lanes; ++l)
        if (positions[l] + steps > kvs[l]->capacity || positions[l] + steps > ws->lm->positions)
            return GPHQ_ERR_PREFIX_FULL;
    if (overlaps(tokens_out_dev, steps * lanes * 4, hidden_dev, lanes * ws->lm->cfg.hidden * 4))
        return GPHQ_ERR_OVERLAP;
    hipStream_t st = (hipStream_t)stream;
    float *hid = hidden_dev ? hidden_dev : ws->hidden;
    int64_t keys[kMaxLanes];
    for (int64_t l = 0; l < lanes; ++l) keys[l] = positions[l] + steps;  // the last step's context
    if (ws->use_graph) GPHQ_TRY(step_graph(ws, kvs, (int)lanes, keys, hid, tokens_out_dev));
    GPHQ_TRY(seed(ws, (int)lanes, positions, tokens, 0, st));
    for (int64_t t = 0; t < steps; ++t) {
        if (ws->use_graph) {
            GPHQ_TRY(hip_status(hipGraphLaunch(ws->step_exec, st)));
        } else {
            for (int64_t l = 0; l < lanes; ++l) keys[l] = positions[l] + t + 1;
            GPHQ_TRY(encode_step(ws, kvs, (int)lanes, keys, true, hid, nullptr, tokens_out_dev, st));
        }
    }
    return GPHQ_OK;
}

int gphq_decode_batch_set_graph(gphq_decode_batch *ws, int on) {
    if (!ws) return GPHQ_ERR_FOREIGN_WORKSPACE;
    ws->use_graph = on != 0;
    if (!ws->use_graph) drop_graph(ws);
    return GPHQ_OK;
}

int gphq_decode_extend(gphq_decode_batch *ws, gphq_prefix *const *kvs, int64_t lanes, const int64_t *positions,
                       const int32_t *tokens, int64_t steps, void *stream) {
    if (steps < 1) return GPHQ_ERR_BATCH_SHAPE;
    GPHQ_TRY(validate(ws, kvs, lanes, positions, tokens, steps, nullptr, 0, nullptr, nullptr, false));
    hipStream_t st = (hipStream_t)stream;
    int64_t keys[kMaxLanes];
    for (int64_t t = 0; t < steps; ++t) {
        GPHQ_TRY(seed(ws, (int)lanes, positions, tokens + t * lanes, t, st));
        for (int64_t l = 0; l < lanes; ++l) keys[l] = positions[l] + t + 1;
        GPHQ_TRY(encode_step(ws, kvs, (int)lanes, keys, false, nullptr, nullptr, nullptr, st));
    }
    return GPHQ_OK;
}

int gphq_decode_batch_logits(gphq_decode_batch *ws, const float *hidden_dev, int64_t hidden_len, float *logits_dev,
                             int64_t logits_len, void *stream) {
    if (!ws || !ws->lm) return GPHQ_ERR_FOREIGN_WORKSPACE;
    const gphq_lm *lm = ws->lm;
    const int64_t H = lm->cfg.hidden, V = lm->cfg.vocab;
    const int64_t k = hidden_len / H;
    // evaluator.go:325-327: whole states in, whole logit rows out, at most maxTail rows.
    if (k == 0 || hidden_len != k * H || logits_len != k * V || k > GPHQ_LOGITS_MAX_ROWS)
        return GPHQ_ERR_LOGITS_SHAPE;
    if (!hidden_dev || !logits_dev) return GPHQ_ERR_LOGITS_SHAPE;
    if (overlaps(hidden_dev, hidden_len * 4, logits_dev, logits_len * 4)) return GPHQ_ERR_OVERLAP;
    hipStream_t st = (hipStream_t)stream;
    for (int64_t r0 = 0; r0 < k; r0 += ws->capacity) {
        const int lanes = (int)std::min<int64_t>(ws->capacity, k - r0);
        // gpu_darwin.go:1517-1520: hidden.apply to each state, then the head
        // GEMV over the rotated rows (gpu_darwin.go:1530-1532).
        GPHQ_TRY(hip_status(hipMemcpyAsync(ws->hn, hidden_dev + r0 * H, (size_t)lanes * H * 4,
                                           hipMemcpyDeviceToDevice, st)));
        hipLaunchKernelGGL(lm_rotate_kernel, dim3((unsigned)(H / lm->hblock), lanes), dim3(256),
                           lm->hblock * sizeof(float), st, ws->hn, (int)H, lm->hsigns, (int)lm->hblock);
        GPHQ_TRY(launch_status());
        GPHQ_TRY(gemv(ws, lanes, GPHQ_FMT_Q8B, PRO_PLAIN, EPI_STORE, lm->head, 0, lm->head_scale, ws->hn, H,
                      ws->logits, lm->head_rows, H, lm->head_rows, st));
        GPHQ_TRY(hip_status(hipMemcpy2DAsync(logits_dev + r0 * V, (size_t)V * 4, ws->logits,
                                             (size_t)lm->head_rows * 4, (size_t)V * 4, (size_t)lanes,
                                             hipMemcpyDeviceToDevice, st)));
    }
    return GPHQ_OK;
}

int gphq_decode_batch_check(gphq_decode_batch *ws, void *stream) {
    if (!ws) return GPHQ_ERR_FOREIGN_WORKSPACE;
    int32_t flags[kMaxLanes];
    GPHQ_TRY(hip_status(hipMemcpyAsync(flags, ws->nonfinite, ws->capacity * 4, hipMemcpyDeviceToHost,
                                       (hipStream_t)stream)));
    GPHQ_TRY(hip_status(hipStreamSynchronize((hipStream_t)stream)));
    bool bad = false;
    for (int l = 0; l < ws->capacity; ++l) bad |= flags[l] != 0;
    if (!bad) return GPHQ_OK;
    GPHQ_TRY(hip_status(hipMemsetAsync(ws->nonfinite, 0, ws->capacity * 4, (hipStream_t)stream)));
    GPHQ_TRY(hip_status(hipStreamSynchronize((hipStream_t)stream)));
    return GPHQ_ERR_NON_FINITE_HIDDEN;
}

}  // extern "C"
