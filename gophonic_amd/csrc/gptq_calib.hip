// The GPTQ calibration pass on MI355X: qwen3lm's QuantizeGPTQ (gptq.go:191-266)
// and its calibration (newCalibration, calibration.weights / layer /
// attention, normalizedRows, project; gptq.go:330-600), which run the model
// layer by layer in FP32 on calibration text and round each projection with
// GPTQ against the inputs the already rounded layers before it produce.
//
// State (gphq_gptq_calibration): the residual stream of every calibration row
// [rows][hidden] in the GPU backend's basis (the hidden rotation applied to
// each BF16 embedding row), each row's position in its sequence and its
// sequence's first row, and a 256-row RoPE table (gptqMaxSeq).
//
// One layer (gphq_gptq_calibration_layer), all on the device:
//   1. the seven projections in the GPU basis (calibration.weights): BF16 ->
//      float32 -> folded RMSNorm weight -> input rotation -> output rotation,
//      the float32 stage of the weight preparation (prepare_rows_f32), so each
//      matrix is the reference's float32 matrix bit for bit;
//   2. x = the normalized residual rows; GPTQ of q, k, v over x (factor, then
//      rounding in place, codes and scales out); q, k, v = x W^T through the
//      rounded matrices (fp32 products);
//   3. head RMSNorm (q_norm / k_norm) and RoPE at each row's position, causal
//      attention within each sequence (dot products, a softmax scaled by
//      1/sqrt(head_dim), the weighted sum of value rows in key order); GPTQ of
//      o over the context rows; h += ctx W_o^T;
//   4. x = the normalized residual rows; GPTQ of gate and up; g = silu(x W_g^T)
//      * (x W_u^T), then the intermediate rotation; GPTQ of down over those
//      rows; h += g W_d^T.
// GPTQ itself is gphq_gptq_factor / gphq_gptq_round (gptq.hip). Everything
// is fp32 as in the reference; sums run in another order than the reference's
// (wavefront reductions, 64 x 64 product tiles), so results agree to fp32
// rounding, not bit for bit. Multiply-add contraction is off in this file, as
// amd64 Go rounds every product and sum.
#include <math.h>
#include <string.h>

#include <string>
#include <vector>

#include "common.h"
#include "host_io.h"
#include "lm_model.h"

#pragma clang fp contract(off)

namespace gphq {
int prepare_rows_f32(const uint16_t *src, int64_t n, int64_t k, const float *norm_host, gphq_rotation_spec in_rot,
                     gphq_rotation_spec out_rot, float *out, float *tables, hipStream_t st);
int sgemm_abt(int M, int N, int K, const float *a, long lda, const float *b, long ldb, float *c, long ldc,
              bool accumulate, hipStream_t st);
int gptq_format_bits(const char *format, int *bits);
}  // namespace gphq

using namespace gphq;

namespace {

constexpr int kMaxSeq = 256;    // gptqMaxSeq (gptq.go:40): tokens per sequence, rows of the RoPE table
constexpr int kMaxRows = 4096;  // gptqMaxRows (gptq.go:39): calibration tokens
constexpr int kHd = 128;        // head_dim (gphq_lm_new requires it)
constexpr int kHalf = kHd / 2;
constexpr int64_t kRotationUnit = 4096;  // maxRotationBlock (hadamard.go:11)

__device__ __forceinline__ float wave_max(float v) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

// normalizedRows (gptq.go:575-587): x[r] = h[r] * float32(1 / sqrt(ss / width
// + eps)) with ss the row's float32 sum of squares; one block per row.
__global__ __launch_bounds__(256) void cal_norm_rows_kernel(const float *__restrict__ h, float *__restrict__ x,
                                                            int width, double eps) {
    __shared__ float part[4];
    const float *src = h + (size_t)blockIdx.x * width;
    float *dst = x + (size_t)blockIdx.x * width;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < width; i += 256) {
        const float v = src[i];
        ss += v * v;
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (part[0] + part[1]) + (part[2] + part[3]);
    const float inv = (float)(1.0 / sqrt((double)ss / (double)width + eps));
    for (int i = threadIdx.x; i < width; i += 256) dst[i] = src[i] * inv;
}

// calibration.attention's first loop (gptq.go:533-548): every q and k head of
// a row through rmsNorm32 (ops.go:251-254: float32(1 / sqrt(float64(ss) / 128
// + eps)), then x * inv * weight) and rotateHalves at the row's position
// (kernels_scalar.go:73-80). One block per row, one wavefront per head at a
// time; lane l holds dimensions l and l + 64, the pair RoPE rotates together.
__global__ __launch_bounds__(256) void cal_qk_rope_kernel(float *__restrict__ q, float *__restrict__ k,
                                                          const int32_t *__restrict__ pos,
                                                          const float *__restrict__ qn, const float *__restrict__ kn,
                                                          const float *__restrict__ rope, int heads, int kv_heads,
                                                          double eps) {
    const int r = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int p = pos[r];
    const float c = rope[p * kHalf + lane], s = rope[kMaxSeq * kHalf + p * kHalf + lane];
    for (int it = w; it < heads + kv_heads; it += 4) {
        const bool isq = it < heads;
        float *x = isq ? q + ((size_t)r * heads + it) * kHd : k + ((size_t)r * kv_heads + (it - heads)) * kHd;
        const float *wt = isq ? qn : kn;
        float a = x[lane], b = x[lane + kHalf];
        const float ss = wave_sum(a * a + b * b);
        const float inv = (float)(1.0 / sqrt((double)ss / (double)kHd + eps));
        a = a * inv * wt[lane];
        b = b * inv * wt[lane + kHalf];
        x[lane] = a * c - b * s;
        x[lane + kHalf] = b * c + a * s;
    }
}

// calibration.attention's second loop (gptq.go:549-569) for one (head, row):
// scores s_j = dot32(q, k_j) over the keys j of the row's sequence up to the
// row itself (four interleaved chains as dot32, kernels_scalar.go:44-58),
// softmaxScaled (max of the raw scores times the scale, exponentials of
// s * scale - m, their sum, each times 1 / sum; kernels_scalar.go:83-95), then
// ctx = the sum of p_j * v_j in key order (axpy32). One wavefront: lane l
// scores keys l, l + 64, ...; lane l sums output dimensions l and l + 64.
__global__ __launch_bounds__(64) void cal_attend_kernel(const float *__restrict__ q, const float *__restrict__ k,
                                                        const float *__restrict__ v,
                                                        const int32_t *__restrict__ start, float *__restrict__ ctx,
                                                        int heads, int kv_heads, float scale) {
    __shared__ float4 qs[kHd / 4];
    __shared__ float sc[kMaxSeq];
    const int h = blockIdx.x, r = blockIdx.y, lane = threadIdx.x;
    const int g = h / (heads / kv_heads);
    const int s0 = start[r], n = r - s0 + 1;
    const float *qr = q + ((size_t)r * heads + h) * kHd;
    if (lane < kHd / 4) qs[lane] = ((const float4 *)qr)[lane];
    __syncthreads();
    float m = -INFINITY;
    for (int j = lane; j < n; j += 64) {
        const float4 *kr = (const float4 *)(k + ((size_t)(s0 + j) * kv_heads + g) * kHd);
        float d0 = 0.0f, d1 = 0.0f, d2 = 0.0f, d3 = 0.0f;
#pragma unroll 8
        for (int i = 0; i < kHd / 4; ++i) {
            const float4 a = qs[i], b = kr[i];
            d0 += a.x * b.x;
            d1 += a.y * b.y;
            d2 += a.z * b.z;
            d3 += a.w * b.w;
        }
        const float d = (d0 + d1) + (d2 + d3);
        sc[j] = d;
        m = fmaxf(m, d);
    }
    m = wave_max(m) * scale;
    float sum = 0.0f;
    for (int j = lane; j < n; j += 64) {
        const float e = expf(sc[j] * scale - m);
        sc[j] = e;
        sum += e;
    }
    const float inv = 1.0f / wave_sum(sum);
    __syncthreads();
    float o0 = 0.0f, o1 = 0.0f;
    const float *vr = v + ((size_t)s0 * kv_heads + g) * kHd;
    for (int j = 0; j < n; ++j, vr += (size_t)kv_heads * kHd) {
        const float p = sc[j] * inv;
        o0 += p * vr[lane];
        o1 += p * vr[lane + 64];
    }
    float *out = ctx + ((size_t)r * heads + h) * kHd;
    out[lane] = o0;
    out[lane + 64] = o1;
}

// silu32 (ops.go:455-461): x / (1 + e^-x) for x >= 0, x e^x / (1 + e^x) below.
__device__ __forceinline__ float silu32(float x) {
    if (x >= 0.0f) return x / (1.0f + expf(-x));
    const float e = expf(x);
    return x * e / (1.0f + e);
}

// gptq.go:504-512 before the rotation: gate[i] = silu32(gate[i]) * up[i].
__global__ __launch_bounds__(256) void cal_swiglu_kernel(float *__restrict__ gate, const float *__restrict__ up,
                                                         size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        gate[i] = silu32(gate[i]) * up[i];
}

// One projection of a layer: rows, input width, the folded norm (0 input, 1
// post-attention, -1 none) and its rotations (calibration.weights,
// gptq.go:404-417: q/k/v hidden in, v per-head out; o per-head in, hidden
// out; gate/up hidden in; down intermediate in, hidden out).
struct ProjSpec {
    int64_t n, k;
    int norm;
    gphq_rotation_spec in, out;
};

void projection_specs(const gphq_lm_config &c, ProjSpec *s) {
    const int64_t h = c.hidden, qd = c.heads * c.head_dim, kv = c.kv_heads * c.head_dim, I = c.intermediate;
    const gphq_rotation_spec none{0, 0}, hid{h, 0}, head{0, c.head_dim}, inter{I, 0};
    s[0] = {qd, h, 0, hid, none};
    s[1] = {kv, h, 0, hid, none};
    s[2] = {kv, h, 0, hid, head};
    s[3] = {h, qd, -1, head, hid};
    s[4] = {I, h, 1, hid, none};
    s[5] = {I, h, 1, hid, none};
    s[6] = {h, I, -1, inter, hid};
}

}  // namespace

struct gphq_gptq_calibration {
    gphq_lm_config cfg{};
    gphq_lm *lm = nullptr;  // the embedding and the rotations' sign tables
    int64_t rows = 0, qd = 0, kvd = 0, kmax = 0, nmax = 0;
    int32_t *ids = nullptr, *pos = nullptr, *start = nullptr;
    float *rope = nullptr;  // [2][kMaxSeq][64]: cos, then sin
    float *h = nullptr, *xa = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *ctx = nullptr, *xm = nullptr;
    float *gate = nullptr, *up = nullptr;
    float *mats[GPHQ_LAYER_PROJECTIONS] = {};
    float *u = nullptr, *tables = nullptr, *qn = nullptr, *kn = nullptr;
    uint8_t *dead = nullptr;
    void *fwork = nullptr, *rwork = nullptr;
    int64_t fwork_bytes = 0, rwork_bytes = 0;
    std::vector<void *> allocs;

    template <typename T>
    int alloc(T **p, int64_t count) {
        void *d = nullptr;
        GPHQ_TRY(hip_status(hipMalloc(&d, (size_t)std::max<int64_t>(count, 1) * sizeof(T))));
        allocs.push_back(d);
        *p = (T *)d;
        return GPHQ_OK;
    }
    ~gphq_gptq_calibration() {
        for (void *p : allocs) (void)hipFree(p);
        if (lm) gphq_lm_free(lm);
    }
};

namespace {

// quantizeGroup (gptq.go:602-665) on the device: factor over x [rows][k], then
// GPTQ rounding of each listed projection in place, codes and scales out.
int quantize_group(gphq_gptq_calibration *cal, const float *x, int64_t k, const int *ps, int np,
                   const ProjSpec *spec, int bits, void *const *codes, void *const *scales, hipStream_t st) {
    GPHQ_TRY(gphq_gptq_factor(x, cal->rows, k, cal->u, cal->dead, cal->fwork, cal->fwork_bytes, st));
    for (int i = 0; i < np; ++i) {
        const int p = ps[i];
        GPHQ_TRY(gphq_gptq_round(cal->mats[p], spec[p].n, k, cal->u, cal->dead, bits, codes[p], scales[p],
                                 cal->rwork, cal->rwork_bytes, st));
    }
    return GPHQ_OK;
}

// project (gptq.go:589-600): y [rows][n] = x [rows][k] . W^T (or y += it).
int project(gphq_gptq_calibration *cal, const float *x, int64_t k, const float *w, int64_t n, float *y,
            bool accumulate, hipStream_t st) {
    return sgemm_abt((int)cal->rows, (int)n, (int)k, x, (long)k, w, (long)k, y, (long)n, accumulate, st);
}

int norm_rows(gphq_gptq_calibration *cal, float *x, hipStream_t st) {
    hipLaunchKernelGGL(cal_norm_rows_kernel, dim3((unsigned)cal->rows), dim3(256), 0, st, cal->h, x,
                       (int)cal->cfg.hidden, cal->cfg.eps);
    return launch_status();
}

}  // namespace

extern "C" {

int gphq_gptq_calibration_new(const gphq_lm_config *cfg, const int32_t *ids, const int64_t *seq_lens, int64_t nseq,
                              const uint16_t *embed_bf16_dev, int64_t embed_len, gphq_gptq_calibration **out,
                              void *stream) {
    // newCalibration (gptq.go:344-383).
    clear_detail();
    if (!cfg || !out || nseq < 0 || (nseq && (!seq_lens || !ids))) return GPHQ_ERR_DIMENSIONS;
    *out = nullptr;
    int64_t rows = 0;
    for (int64_t s = 0; s < nseq; ++s) {
        if (seq_lens[s] < 1 || seq_lens[s] > kMaxSeq)
            return fail(GPHQ_ERR_CALIBRATION_SHAPE,
                        strf("qwen3: calibration sequence %lld has %lld tokens, want 1 to %d", (long long)s,
                             (long long)seq_lens[s], kMaxSeq));
        rows += seq_lens[s];
        if (rows > kMaxRows)
            return fail(GPHQ_ERR_CALIBRATION_SHAPE, strf("qwen3: more than %d calibration tokens", kMaxRows));
    }
    if (rows == 0) return GPHQ_ERR_CALIBRATION_EMPTY;
    gphq_lm_config c = *cfg;
    c.fmt = GPHQ_FMT_Q8;  // the model object only embeds and rotates; no layer is bound
    gphq_lm *lm = nullptr;
    GPHQ_TRY(gphq_lm_new(&c, &lm));
    auto *cal = new gphq_gptq_calibration();
    cal->lm = lm;
    cal->cfg = *cfg;
    int st_ = gphq_lm_bind_embed(lm, embed_bf16_dev, embed_len);
    for (int64_t r = 0; st_ == GPHQ_OK && r < rows; ++r)
        if (ids[r] < 0 || ids[r] >= c.vocab) st_ = GPHQ_ERR_TOKEN_VOCAB;
    if (st_ != GPHQ_OK) {
        delete cal;
        return st_;
    }
    const int64_t H = c.hidden, qd = c.heads * c.head_dim, kvd = c.kv_heads * c.head_dim, I = c.intermediate;
    cal->rows = rows;
    cal->qd = qd;
    cal->kvd = kvd;
    cal->kmax = std::max(std::max(H, qd), I);
    cal->nmax = std::max(std::max(H, qd), std::max(kvd, I));
    ProjSpec spec[GPHQ_LAYER_PROJECTIONS];
    projection_specs(c, spec);
    int64_t table_floats = 0;
    for (const ProjSpec &p : spec) table_floats = std::max(table_floats, 2 * p.k + p.n);
    cal->fwork_bytes = gphq_gptq_work_bytes(cal->kmax);
    cal->rwork_bytes = gphq_gptq_round_work_bytes(cal->nmax, cal->kmax);
    std::vector<int32_t> pos((size_t)rows), start((size_t)rows);
    for (int64_t s = 0, r = 0; s < nseq; ++s)
        for (int64_t p = 0, first = r; p < seq_lens[s]; ++p, ++r) {
            pos[(size_t)r] = (int32_t)p;
            start[(size_t)r] = (int32_t)first;
        }
    // newCalibration's RoPE table: float32(cos/sin(p * invFreq[d])), float64
    // angles, invFreq[d] = 1 / theta^(2d / head_dim) (weights.go:685-688).
    std::vector<float> rope((size_t)(2 * kMaxSeq * kHalf));
    for (int d = 0; d < kHalf; ++d) {
        const double inv = 1.0 / pow(c.rope_theta, (double)(2 * d) / (double)c.head_dim);
        for (int p = 0; p < kMaxSeq; ++p) {
            rope[(size_t)(p * kHalf + d)] = (float)cos((double)p * inv);
            rope[(size_t)(kMaxSeq * kHalf + p * kHalf + d)] = (float)sin((double)p * inv);
        }
    }
    hipStream_t st = (hipStream_t)stream;
    int e = GPHQ_OK;
    auto step = [&](int s) {
        if (e == GPHQ_OK) e = s;
    };
    step(cal->alloc(&cal->ids, rows));
    step(cal->alloc(&cal->pos, rows));
    step(cal->alloc(&cal->start, rows));
    step(cal->alloc(&cal->rope, (int64_t)rope.size()));
    step(cal->alloc(&cal->h, rows * H));
    step(cal->alloc(&cal->xa, rows * H));
    step(cal->alloc(&cal->xm, rows * H));
    step(cal->alloc(&cal->q, rows * qd));
    step(cal->alloc(&cal->ctx, rows * qd));
    step(cal->alloc(&cal->k, rows * kvd));
    step(cal->alloc(&cal->v, rows * kvd));
    step(cal->alloc(&cal->gate, rows * I));
    step(cal->alloc(&cal->up, rows * I));
    for (int p = 0; p < GPHQ_LAYER_PROJECTIONS; ++p) step(cal->alloc(&cal->mats[p], spec[p].n * spec[p].k));
    step(cal->alloc(&cal->u, cal->kmax * cal->kmax));
    step(cal->alloc(&cal->dead, cal->kmax));
    step(cal->alloc(&cal->tables, table_floats));
    step(cal->alloc(&cal->qn, kHd));
    step(cal->alloc(&cal->kn, kHd));
    step(cal->alloc((uint8_t **)&cal->fwork, cal->fwork_bytes));
    step(cal->alloc((uint8_t **)&cal->rwork, cal->rwork_bytes));
    if (e == GPHQ_OK) step(hip_status(hipMemcpyAsync(cal->ids, ids, rows * 4, hipMemcpyHostToDevice, st)));
    if (e == GPHQ_OK) step(hip_status(hipMemcpyAsync(cal->pos, pos.data(), rows * 4, hipMemcpyHostToDevice, st)));
    if (e == GPHQ_OK)
        step(hip_status(hipMemcpyAsync(cal->start, start.data(), rows * 4, hipMemcpyHostToDevice, st)));
    if (e == GPHQ_OK)
        step(hip_status(hipMemcpyAsync(cal->rope, rope.data(), rope.size() * 4, hipMemcpyHostToDevice, st)));
    // Each row: the BF16 embedding row widened, then hidden.apply.
    if (e == GPHQ_OK) step(lm_embed_launch(lm, cal->ids, (int)rows, cal->h, st));
    if (e == GPHQ_OK) step(hip_status(hipStreamSynchronize(st)));
    if (e != GPHQ_OK) {
        delete cal;
        return e;
    }
    *out = cal;
    return GPHQ_OK;
}

void gphq_gptq_calibration_free(gphq_gptq_calibration *cal) { delete cal; }

int gphq_gptq_calibration_layer(gphq_gptq_calibration *cal, const uint16_t *const *src_bf16_dev,
                                const float *input_norm_host, const float *post_norm_host, const float *q_norm_host,
                                const float *k_norm_host, int bits, void *const *codes_dev, void *const *scales_dev,
                                void *stream) {
    // calibration.layer (gptq.go:437-524).
    if (bits != 8 && bits != 4) return GPHQ_ERR_UNSUPPORTED;
    if (!cal || !src_bf16_dev || !input_norm_host || !post_norm_host || !q_norm_host || !k_norm_host ||
        !codes_dev || !scales_dev)
        return GPHQ_ERR_DIMENSIONS;
    for (int p = 0; p < GPHQ_LAYER_PROJECTIONS; ++p)
        if (!src_bf16_dev[p] || !codes_dev[p] || !scales_dev[p]) return GPHQ_ERR_DIMENSIONS;
    const gphq_lm_config &c = cal->cfg;
    if (bits == 4 && (c.hidden % 32 || cal->qd % 32 || c.intermediate % 32)) return GPHQ_ERR_DIMENSIONS;
    hipStream_t st = (hipStream_t)stream;
    ProjSpec spec[GPHQ_LAYER_PROJECTIONS];
    projection_specs(c, spec);
    // calibration.weights (gptq.go:386-433), each matrix into the GPU basis.
    for (int p = 0; p < GPHQ_LAYER_PROJECTIONS; ++p) {
        const float *norm = spec[p].norm == 0 ? input_norm_host : spec[p].norm == 1 ? post_norm_host : nullptr;
        GPHQ_TRY(prepare_rows_f32(src_bf16_dev[p], spec[p].n, spec[p].k, norm, spec[p].in, spec[p].out,
                                  cal->mats[p], cal->tables, st));
    }
    GPHQ_TRY(hip_status(hipMemcpyAsync(cal->qn, q_norm_host, kHd * 4, hipMemcpyHostToDevice, st)));
    GPHQ_TRY(hip_status(hipMemcpyAsync(cal->kn, k_norm_host, kHd * 4, hipMemcpyHostToDevice, st)));
    GPHQ_TRY(hip_status(hipStreamSynchronize(st)));  // the host norms may go once copied
    const int64_t R = cal->rows, H = c.hidden, qd = cal->qd, kvd = cal->kvd, I = c.intermediate;
    // Attention: inputs are the normalized residual rows.
    GPHQ_TRY(norm_rows(cal, cal->xa, st));
    static const int kQKV[] = {0, 1, 2}, kO[] = {3}, kGU[] = {4, 5}, kD[] = {6};
    GPHQ_TRY(quantize_group(cal, cal->xa, H, kQKV, 3, spec, bits, codes_dev, scales_dev, st));
    GPHQ_TRY(project(cal, cal->xa, H, cal->mats[0], qd, cal->q, false, st));
    GPHQ_TRY(project(cal, cal->xa, H, cal->mats[1], kvd, cal->k, false, st));
    GPHQ_TRY(project(cal, cal->xa, H, cal->mats[2], kvd, cal->v, false, st));
    hipLaunchKernelGGL(cal_qk_rope_kernel, dim3((unsigned)R), dim3(256), 0, st, cal->q, cal->k, cal->pos, cal->qn,
                       cal->kn, cal->rope, (int)c.heads, (int)c.kv_heads, c.eps);
    GPHQ_TRY(launch_status());
    hipLaunchKernelGGL(cal_attend_kernel, dim3((unsigned)c.heads, (unsigned)R), dim3(64), 0, st, cal->q, cal->k,
                       cal->v, cal->start, cal->ctx, (int)c.heads, (int)c.kv_heads,
                       (float)(1.0 / sqrt((double)c.head_dim)));
    GPHQ_TRY(launch_status());
    GPHQ_TRY(quantize_group(cal, cal->ctx, qd, kO, 1, spec, bits, codes_dev, scales_dev, st));
    GPHQ_TRY(project(cal, cal->ctx, qd, cal->mats[3], H, cal->h, true, st));
    // MLP.
    GPHQ_TRY(norm_rows(cal, cal->xm, st));
    GPHQ_TRY(quantize_group(cal, cal->xm, H, kGU, 2, spec, bits, codes_dev, scales_dev, st));
    GPHQ_TRY(project(cal, cal->xm, H, cal->mats[4], I, cal->gate, false, st));
    GPHQ_TRY(project(cal, cal->xm, H, cal->mats[5], I, cal->up, false, st));
    const size_t ri = (size_t)(R * I);
    hipLaunchKernelGGL(cal_swiglu_kernel, dim3((unsigned)std::min<size_t>((ri + 255) / 256, 65536)), dim3(256), 0,
                       st, cal->gate, cal->up, ri);
    GPHQ_TRY(launch_status());
    GPHQ_TRY(lm_rotate_launch(cal->lm, cal->gate, (int)R, (long)I, st));  // inter.apply
    GPHQ_TRY(quantize_group(cal, cal->gate, I, kD, 1, spec, bits, codes_dev, scales_dev, st));
    GPHQ_TRY(project(cal, cal->gate, I, cal->mats[6], H, cal->h, true, st));
    return hip_status(hipStreamSynchronize(st));
}

int gphq_gptq_calibration_rows(const gphq_gptq_calibration *cal, int which, float *dst_dev, int64_t dst_len,
                               int64_t *rows, int64_t *width, void *stream) {
    if (!cal) return GPHQ_ERR_DIMENSIONS;
    const float *p = nullptr;
    int64_t w = 0;
    switch (which) {
    case GPHQ_CAL_RESIDUAL: p = cal->h, w = cal->cfg.hidden; break;
    case GPHQ_CAL_ATTN_INPUT: p = cal->xa, w = cal->cfg.hidden; break;
    case GPHQ_CAL_CONTEXT: p = cal->ctx, w = cal->qd; break;
    case GPHQ_CAL_MLP_INPUT: p = cal->xm, w = cal->cfg.hidden; break;
    case GPHQ_CAL_DOWN_INPUT: p = cal->gate, w = cal->cfg.intermediate; break;
    default: return GPHQ_ERR_DIMENSIONS;
    }
    if (rows) *rows = cal->rows;
    if (width) *width = w;
    if (!dst_dev) return GPHQ_OK;
    if (dst_len < cal->rows * w) return GPHQ_ERR_DIMENSIONS;
    return hip_status(hipMemcpyAsync(dst_dev, p, (size_t)(cal->rows * w) * 4, hipMemcpyDeviceToDevice,
                                     (hipStream_t)stream));
}

int gphq_gptq_calibration_sequences(const int64_t *text_lens, int64_t ntexts, int64_t *seq_lens, int64_t max_seqs,
                                    int64_t *nseq) {
    // calibrationSequences' add (gptq.go:275-287) without the tokenizer: each
    // text's token ids cut into sequences of at most gptqMaxSeq tokens until
    // gptqMaxRows tokens are taken. With seq_lens NULL only the count is
    // returned.
    if (ntexts < 0 || (ntexts && !text_lens) || !nseq || max_seqs < 0) return GPHQ_ERR_DIMENSIONS;
    int64_t total = 0, n = 0;
    for (int64_t t = 0; t < ntexts; ++t) {
        if (text_lens[t] < 0) return GPHQ_ERR_DIMENSIONS;
        for (int64_t left = text_lens[t]; left > 0 && total < kMaxRows;) {
            const int64_t take = std::min<int64_t>(std::min<int64_t>(left, kMaxSeq), kMaxRows - total);
            if (seq_lens && n < max_seqs) seq_lens[n] = take;
            ++n;
            total += take;
            left -= take;
        }
    }
    *nseq = n;
    return seq_lens && n > max_seqs ? GPHQ_ERR_DIMENSIONS : GPHQ_OK;
}

int gphq_gptq_quantize(const char *dir, const char *format, const gphq_lm_config *cfg, const int32_t *ids,
                       const int64_t *text_lens, int64_t ntexts, gphq_gptq_progress progress, void *user,
                       void *stream) {
    // QuantizeGPTQ (gptq.go:197-266), the texts already tokenized.
    clear_detail();
    int bits = 0;
    GPHQ_TRY(gptq_format_bits(format, &bits));
    if (!dir || !cfg || ntexts < 0 || (ntexts && !text_lens)) return GPHQ_ERR_DIMENSIONS;
    int64_t tokens = 0;
    for (int64_t t = 0; t < ntexts; ++t) {
        if (text_lens[t] < 0) return GPHQ_ERR_DIMENSIONS;
        tokens += text_lens[t];
    }
    if (tokens && !ids) return GPHQ_ERR_DIMENSIONS;
    const gphq_lm_config &c = *cfg;
    if (c.hidden % kRotationUnit || c.intermediate % kRotationUnit || (c.heads * c.head_dim) % kRotationUnit)
        return GPHQ_ERR_GPTQ_WIDTH;
    int64_t nseq = 0;
    GPHQ_TRY(gphq_gptq_calibration_sequences(text_lens, ntexts, nullptr, 0, &nseq));
    std::vector<int64_t> seqs((size_t)nseq);
    if (nseq == 0) return GPHQ_ERR_CALIBRATION_EMPTY;
    GPHQ_TRY(gphq_gptq_calibration_sequences(text_lens, ntexts, seqs.data(), nseq, &nseq));
    // The sequences are taken from the texts in order, so their ids are the
    // texts' ids with every text's tail past the cut left out.
    std::vector<int32_t> cal_ids;
    {
        int64_t total = 0, off = 0;
        for (int64_t t = 0; t < ntexts; ++t) {
            const int64_t take = std::min<int64_t>(text_lens[t], kMaxRows - total);
            cal_ids.insert(cal_ids.end(), ids + off, ids + off + std::max<int64_t>(take, 0));
            total += std::max<int64_t>(take, 0);
            off += text_lens[t];
        }
    }
    gphq_checkpoint *ck = nullptr;
    GPHQ_TRY(gphq_checkpoint_open(dir, &ck));
    gphq_gptq_writer *w = nullptr;
    int e = gphq_gptq_create(dir, format, &w);
    if (e != GPHQ_OK) {
        gphq_checkpoint_close(ck);
        return e;
    }
    hipStream_t st = (hipStream_t)stream;
    gphq_gptq_calibration *cal = nullptr;
    uint16_t *embed = nullptr, *src[GPHQ_LAYER_PROJECTIONS] = {};
    uint8_t *codes[GPHQ_LAYER_PROJECTIONS] = {}, *scales[GPHQ_LAYER_PROJECTIONS] = {};
    ProjSpec spec[GPHQ_LAYER_PROJECTIONS];
    projection_specs(c, spec);
    std::vector<float> norms[4];
    for (auto &v : norms) v.resize((size_t)std::max<int64_t>(c.hidden, kHd));
    auto step = [&](int s) {
        if (e == GPHQ_OK) e = s;
    };
    const int64_t emb = c.vocab * c.hidden;
    step(hip_status(hipMalloc((void **)&embed, (size_t)emb * 2)));
    for (int p = 0; p < GPHQ_LAYER_PROJECTIONS; ++p) {
        int64_t cb = 0, sb = 0;
        step(gphq_gptq_row_bytes(bits, spec[p].k, &cb, &sb));
        step(hip_status(hipMalloc((void **)&src[p], (size_t)(spec[p].n * spec[p].k * 2))));
        step(hip_status(hipMalloc((void **)&codes[p], (size_t)(spec[p].n * cb))));
        step(hip_status(hipMalloc((void **)&scales[p], (size_t)(spec[p].n * sb))));
    }
    const int64_t embed_shape[2] = {c.vocab, c.hidden};
    if (e == GPHQ_OK) step(gphq_checkpoint_bf16_device(ck, "model.embed_tokens.weight", embed_shape, 2, embed, emb));
    if (e == GPHQ_OK)
        step(gphq_gptq_calibration_new(cfg, cal_ids.data(), seqs.data(), nseq, embed, emb, &cal, stream));
    static const char *kNames[GPHQ_LAYER_PROJECTIONS] = {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                                                         "self_attn.o_proj", "mlp.gate_proj",    "mlp.up_proj",
                                                         "mlp.down_proj"};
    for (int64_t layer = 0; e == GPHQ_OK && layer < c.layers; ++layer) {
        const std::string pre = strf("model.layers.%lld.", (long long)layer);
        const int64_t hshape[1] = {c.hidden}, dshape[1] = {c.head_dim};
        step(gphq_checkpoint_float32(ck, (pre + "input_layernorm.weight").c_str(), hshape, 1, norms[0].data(),
                                     c.hidden));
        if (e == GPHQ_OK)
            step(gphq_checkpoint_float32(ck, (pre + "post_attention_layernorm.weight").c_str(), hshape, 1,
                                         norms[1].data(), c.hidden));
        if (e == GPHQ_OK)
            step(gphq_checkpoint_float32(ck, (pre + "self_attn.q_norm.weight").c_str(), dshape, 1, norms[2].data(),
                                         c.head_dim));
        if (e == GPHQ_OK)
            step(gphq_checkpoint_float32(ck, (pre + "self_attn.k_norm.weight").c_str(), dshape, 1, norms[3].data(),
                                         c.head_dim));
        for (int p = 0; e == GPHQ_OK && p < GPHQ_LAYER_PROJECTIONS; ++p) {
            const int64_t shape[2] = {spec[p].n, spec[p].k};
            step(gphq_checkpoint_bf16_device(ck, (pre + kNames[p] + ".weight").c_str(), shape, 2, src[p],
                                             spec[p].n * spec[p].k));
        }
        if (e == GPHQ_OK)
            step(gphq_gptq_calibration_layer(cal, src, norms[0].data(), norms[1].data(), norms[2].data(),
                                             norms[3].data(), bits, (void *const *)codes, (void *const *)scales,
                                             stream));
        // File order: per projection, every row's codes, then every row's scales.
        for (int p = 0; e == GPHQ_OK && p < GPHQ_LAYER_PROJECTIONS; ++p) {
            int64_t cb = 0, sb = 0;
            gphq_gptq_row_bytes(bits, spec[p].k, &cb, &sb);
            step(gphq_gptq_write_device(w, codes[p], spec[p].n * cb));
            if (e == GPHQ_OK) step(gphq_gptq_write_device(w, scales[p], spec[p].n * sb));
        }
        if (e == GPHQ_OK && progress) progress(layer + 1, c.layers, user);
    }
    if (e == GPHQ_OK) step(hip_status(hipStreamSynchronize(st)));
    gphq_gptq_calibration_free(cal);
    (void)hipFree(embed);
    for (int p = 0; p < GPHQ_LAYER_PROJECTIONS; ++p) {
        (void)hipFree(src[p]);
        (void)hipFree(codes[p]);
        (void)hipFree(scales[p]);
    }
    gphq_checkpoint_close(ck);
    if (e != GPHQ_OK) {
        gphq_gptq_abort(w);
        return e;
    }
    return gphq_gptq_commit(w);
}

}  // extern "C"
