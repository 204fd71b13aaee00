// Weight preparation on the device: one gpuJob of qwen3lm's prepareGPU
// (gpu_darwin.go:392-569), the path from a checkpoint's BF16 projection to the
// stored rows the GEMV, mm and decode kernels read.
//
// For rows of BF16 bits [n][k] the steps are the reference's, in its float32
// operation order, so the stored codes and scales are bit-identical to the
// host path's:
//   1. widen to float32 (exact) and multiply by the folded RMSNorm weight;
//   2. the input rotation, R.row: (x * scale) * sign, then the Walsh-Hadamard
//      butterflies per block (hadamard.go:49-58);
//   3. the output rotation along the rows, R.W: each row times its sign, the
//      butterflies across the rows of each block, then every value times
//      scale (hadamard.go:88-104);
//   4. quantization per row: Q8 (quantizeRow, gpu_darwin.go:582-594), Q8B
//      (quantizeRowQ8B, 599-614) or Q4 (quantizeRowQ4 with its 16-candidate
//      scale search, 616-658), written at the job's offsets into the layer
//      buffer; source row r lands on row row0 + r*step (gate and up rows
//      interleave with step 2).
// Kernels: prep_rows_kernel (steps 1-2 and the output signs, one block per
// row, the row in LDS), prep_cols_fwht_kernel (step 3's butterflies, a tile
// of block rows x a few columns in LDS) and the quantizers (one thread per
// 32-value block; one block per row for Q8's row maximum). Contraction of
// multiplies and adds into FMA is off in this file: the reference rounds
// every product and sum.
#include <math.h>

#include "common.h"

#pragma clang fp contract(off)

namespace gphq {

// qwen3lm/hadamard.go:24-47 newRotation(k): splitmix64 from golden ^ k, the
// low bit of each output picks the sign.
int rotation_signs_pm1(int64_t k, std::vector<float> &signs) {
    int64_t block = 1;
    while (block < 4096 && k % (2 * block) == 0) block *= 2;
    uint64_t state = 0x9e3779b97f4a7c15ull ^ (uint64_t)k;
    signs.resize(k);
    for (int64_t i = 0; i < k; ++i) {
        state += 0x9e3779b97f4a7c15ull;
        uint64_t z = state;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        z ^= z >> 31;
        signs[i] = (z & 1) ? -1.0f : 1.0f;
    }
    return (int)block;
}

}  // namespace gphq

using namespace gphq;

namespace {

constexpr int kMaxPrepWidth = 16384;  // a row in LDS

struct RowsArgs {
    const uint16_t *src;  // [n][k] BF16 bits
    const float *norm;    // [k] or null
    const float *in_signs;  // [k] (+-1) or null
    const float *out_signs;  // [n] (+-1) or null
    float *work;          // [n][k]
    int k, in_block;
    float in_scale;
};

__global__ __launch_bounds__(256) void prep_rows_kernel(const RowsArgs a) {
    extern __shared__ float v[];
    const int r = blockIdx.x;
    const uint16_t *src = a.src + (size_t)r * a.k;
    float *dst = a.work + (size_t)r * a.k;
    for (int i = threadIdx.x; i < a.k; i += blockDim.x) {
        float x = __builtin_bit_cast(float, (uint32_t)src[i] << 16);
        if (a.norm) x = x * a.norm[i];
        if (a.in_signs) x = x * a.in_scale * a.in_signs[i];
        v[i] = x;
    }
    __syncthreads();
    if (a.in_signs) lds_fwht(v, a.k, a.in_block);
    const float os = a.out_signs ? a.out_signs[r] : 1.0f;  // exact: +-1
    for (int i = threadIdx.x; i < a.k; i += blockDim.x) dst[i] = v[i] * os;
}

// Butterflies across the rows of each `block`-row group, then x*scale:
// grid (k / cols, n / block); the tile is block rows x cols columns.
__global__ __launch_bounds__(256) void prep_cols_fwht_kernel(float *work, int k, int block, int cols, float scale) {
    extern __shared__ float v[];  // [block][cols]
    const int c0 = blockIdx.x * cols;
    const size_t r0 = (size_t)blockIdx.y * block;
    for (int idx = threadIdx.x; idx < block * cols; idx += blockDim.x) {
        const int r = idx / cols, c = idx - r * cols;
        v[idx] = work[(r0 + r) * k + c0 + c];
    }
    __syncthreads();
    for (int h = 1; h < block; h <<= 1) {
        for (int idx = threadIdx.x; idx < (block >> 1) * cols; idx += blockDim.x) {
            const int p = idx / cols, c = idx - p * cols;
            const int i = (p / h) * 2 * h + (p % h);
            const float x = v[i * cols + c], y = v[(i + h) * cols + c];
            v[i * cols + c] = x + y;
            v[(i + h) * cols + c] = x - y;
        }
        __syncthreads();
    }
    for (int idx = threadIdx.x; idx < block * cols; idx += blockDim.x) {
        const int r = idx / cols, c = idx - r * cols;
        work[(r0 + r) * k + c0 + c] = v[idx] * scale;
    }
}

struct QuantArgs {
    const float *work;  // [n][k]
    uint8_t *dst;       // the layer buffer
    long base, sc, step, row0;
    int n, k;
    float mul;
};

// The float32 value itself, opaque to the optimizer. A float32 product fed to
// an FP16 conversion is otherwise fused into one v_fma_mix (rounded once, from
// the exact product), which differs from rounding to float32 and then to FP16
// when the float32 product is an FP16 halfway case.
__device__ __forceinline__ float f32_value(float x) {
    asm volatile("" : "+v"(x));
    return x;
}
__device__ __forceinline__ float f16_round(float x) { return (float)(_Float16)f32_value(x); }
__device__ __forceinline__ uint16_t f16_bits(float x) { return __builtin_bit_cast(uint16_t, (_Float16)f32_value(x)); }

// q8gemm.MaxAbs (gemm.go:138-150): the largest |x|; a NaN is returned as is.
__device__ __forceinline__ float max_abs_step(float m, float x) {
    if (m != m) return m;
    if (x != x) return x;
    return fmaxf(m, fabsf(x));
}

__device__ __forceinline__ int8_t q8_code(float x, float d) {
    const float q = rintf(x / d);  // IEEE division, nearest-even
    return (int8_t)(q != q ? 0.0f : fminf(127.0f, fmaxf(-127.0f, q)));
}

// Q8 (quantizeRow): one block per row. s = max|row| / 127, codes nearest-even
// of x/s clamped to +-127, stored scale s * mul.
__global__ __launch_bounds__(256) void prep_q8_kernel(const QuantArgs a) {
    __shared__ float red[4];
    const int r = blockIdx.x;
    const float *row = a.work + (size_t)r * a.k;
    float m = 0.0f;
    for (int i = threadIdx.x; i < a.k; i += blockDim.x) m = max_abs_step(m, row[i]);
    for (int off = 32; off > 0; off >>= 1) m = max_abs_step(m, __shfl_xor(m, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = max_abs_step(max_abs_step(red[0], red[1]), max_abs_step(red[2], red[3]));
    const long d = a.row0 + (long)r * a.step;
    int8_t *q = (int8_t *)(a.dst + a.base + d * a.k);
    const float s = m / 127.0f;
    for (int i = threadIdx.x; i < a.k; i += blockDim.x) q[i] = m == 0.0f ? 0 : q8_code(row[i], s);
    if (threadIdx.x == 0) *(float *)(a.dst + a.sc + d * 4) = m == 0.0f ? 0.0f * a.mul : s * a.mul;
}

// Q8B (quantizeRowQ8B) and its fp32-scale variant: one thread per 32 values.
template <bool F32SCALE>
__global__ __launch_bounds__(256) void prep_q8b_kernel(const QuantArgs a) {
    const int kb = a.k >> 5;
    const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (long)a.n * kb) return;
    const int r = (int)(t / kb), b = (int)(t - (long)r * kb);
    const float *v = a.work + (size_t)r * a.k + b * 32;
    float m = 0.0f;
    for (int i = 0; i < 32; ++i) m = max_abs_step(m, v[i]);
    const long d = a.row0 + (long)r * a.step;
    int8_t *q = (int8_t *)(a.dst + a.base + d * a.k) + b * 32;
    float dd;
    if constexpr (F32SCALE) {
        dd = m / 127.0f;
        ((float *)(a.dst + a.sc + d * kb * 4))[b] = dd * a.mul;
    } else {
        dd = f16_round(m / 127.0f);
        ((uint16_t *)(a.dst + a.sc + d * kb * 2))[b] = f16_bits(dd * a.mul);
    }
    for (int i = 0; i < 32; ++i) q[i] = dd == 0.0f ? 0 : q8_code(v[i], dd);
}

// Q4 (quantizeRowQ4): one thread per 32 values. peak = the value of largest
// magnitude (first on ties); 16 FP16 candidates peak/-8*(1-0.02*step), the
// one with the smallest float32 sum of squared errors (first on ties); codes
// clamp(rne(x/d), -8, 7) + 8, value j in the low nibble of byte j and value
// j+16 in the high nibble; stored scale f16(best * mul).
__global__ __launch_bounds__(256) void prep_q4_kernel(const QuantArgs a) {
    const int kb = a.k >> 5;
    const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (long)a.n * kb) return;
    const int r = (int)(t / kb), b = (int)(t - (long)r * kb);
    const float *v = a.work + (size_t)r * a.k + b * 32;
    float x[32];
    for (int i = 0; i < 32; ++i) x[i] = v[i];
    float peak = 0.0f;
    for (int i = 0; i < 32; ++i)
        if (fabsf(x[i]) > fabsf(peak)) peak = x[i];
    float best = 0.0f, bestErr = INFINITY;
    if (peak != 0.0f) {
        for (int step = 0; step < 16; ++step) {
            const float d = f16_round(peak / -8.0f * (1.0f - 0.02f * (float)step));
            if (d == 0.0f) continue;
            float e = 0.0f;
            for (int i = 0; i < 32; ++i) {
                const float qv = fminf(7.0f, fmaxf(-8.0f, rintf(x[i] / d)));
                const float diff = x[i] - qv * d;
                e += diff * diff;
            }
            if (e < bestErr) {
                best = d;
                bestErr = e;
            }
        }
    }
    const long d = a.row0 + (long)r * a.step;
    uint8_t *out = a.dst + a.base + d * (a.k >> 1) + b * 16;
    for (int j = 0; j < 16; ++j) {
        int lo = 8, hi = 8;
        if (best != 0.0f) {
            lo = (int)fminf(7.0f, fmaxf(-8.0f, rintf(x[j] / best))) + 8;
            hi = (int)fminf(7.0f, fmaxf(-8.0f, rintf(x[j + 16] / best))) + 8;
        }
        out[j] = (uint8_t)(lo | (hi << 4));
    }
    ((uint16_t *)(a.dst + a.sc + d * kb * 2))[b] = f16_bits(best * a.mul);
}

// Signs of a rotation spec: newRotation(width)'s, or newRotation(tile)'s
// repeated every tile values (the per-head rotation, gpu_darwin.go:217-221).
int spec_signs(const gphq_rotation_spec &r, int64_t len, std::vector<float> &signs, float *scale) {
    int block;
    if (r.tile > 0) {
        std::vector<float> t;
        block = rotation_signs_pm1(r.tile, t);
        signs.resize(len);
        for (int64_t i = 0; i < len; ++i) signs[i] = t[i % r.tile];
    } else {
        block = rotation_signs_pm1(r.width, signs);
    }
    *scale = rotation_scale(block);
    return block;
}

bool spec_ok(const gphq_rotation_spec &r, int64_t len) {
    if (r.width == 0 && r.tile == 0) return true;
    if (r.tile < 0 || r.width < 0) return false;
    if (r.tile > 0) return len % r.tile == 0;
    return r.width == len;
}

int64_t region_bytes(int fmt, int64_t rows, int64_t k, bool scales) {
    if (!scales) return fmt == GPHQ_FMT_Q4 ? rows * k / 2 : rows * k;
    if (fmt == GPHQ_FMT_Q8) return rows * 4;
    if (fmt == GPHQ_FMT_Q8B_F32) return rows * (k / 32) * 4;
    return rows * (k / 32) * 2;
}

}  // namespace

namespace gphq {

// The float32 stage of a projection job (steps 1-3 above): BF16 rows [n][k]
// times the folded norm (norm_host, or null), the input rotation along each
// row, the output rotation across the rows, into out [n][k] -- the values the
// quantizers read, which are the reference's float32 matrix bit for bit.
// tables: 2k + n floats of device scratch for the norm and the signs. The
// rotations must fit (spec_ok; n a multiple of the output block). Waits for
// the stream (the host tables are copied from temporaries).
int prepare_rows_f32(const uint16_t *src, int64_t n, int64_t k, const float *norm_host, gphq_rotation_spec in_rot,
                     gphq_rotation_spec out_rot, float *out, float *tables, hipStream_t st) {
    if (n <= 0 || k <= 0 || k > kMaxPrepWidth || n > INT32_MAX || !src || !out || !tables)
        return GPHQ_ERR_DIMENSIONS;
    if (!spec_ok(in_rot, k) || !spec_ok(out_rot, n)) return GPHQ_ERR_DIMENSIONS;
    // The output rotation mixes rows in blocks: the rows must fill whole blocks.
    std::vector<float> in_s, out_s;
    float in_scale = 1.0f, out_scale = 1.0f;
    int in_block = 0, out_block = 0;
    const bool has_in = in_rot.width || in_rot.tile, has_out = out_rot.width || out_rot.tile;
    if (has_in) in_block = spec_signs(in_rot, k, in_s, &in_scale);
    if (has_out) {
        out_block = spec_signs(out_rot, n, out_s, &out_scale);
        if (n % out_block) return GPHQ_ERR_DIMENSIONS;
    }
    float *norm_d = tables, *in_d = norm_d + k, *out_d = in_d + k;
    if (norm_host) GPHQ_TRY(hip_status(hipMemcpyAsync(norm_d, norm_host, k * 4, hipMemcpyHostToDevice, st)));
    if (has_in) GPHQ_TRY(hip_status(hipMemcpyAsync(in_d, in_s.data(), k * 4, hipMemcpyHostToDevice, st)));
    if (has_out) GPHQ_TRY(hip_status(hipMemcpyAsync(out_d, out_s.data(), n * 4, hipMemcpyHostToDevice, st)));
    RowsArgs ra{src, norm_host ? norm_d : nullptr, has_in ? in_d : nullptr, has_out ? out_d : nullptr, out, (int)k,
                in_block, in_scale};
    hipLaunchKernelGGL(prep_rows_kernel, dim3((unsigned)n), dim3(256), k * 4, st, ra);
    GPHQ_TRY(launch_status());
    if (has_out) {
        int cols = std::max(1, std::min<int>(64, kMaxPrepWidth / out_block));
        while (k % cols) cols >>= 1;
        hipLaunchKernelGGL(prep_cols_fwht_kernel, dim3((unsigned)(k / cols), (unsigned)(n / out_block)), dim3(256),
                           (size_t)out_block * cols * 4, st, out, (int)k, out_block, cols, out_scale);
        GPHQ_TRY(launch_status());
    }
    // The host-side signs and norm must outlive their copies.
    return hip_status(hipStreamSynchronize(st));
}

}  // namespace gphq

extern "C" {


int64_t gphq_prepare_work_bytes(int64_t n, int64_t k) {
    if (n <= 0 || k <= 0 || k > kMaxPrepWidth) return GPHQ_ERR_DIMENSIONS;
    return (n * k + 2 * k + n) * 4 + 256;
}

int gphq_prepare_projection(const gphq_prepare_job *j, void *work_dev, int64_t work_bytes, void *stream) {
    if (!j) return GPHQ_ERR_DIMENSIONS;
    const int fmt = j->fmt;
    if (fmt != GPHQ_FMT_Q8 && fmt != GPHQ_FMT_Q8B && fmt != GPHQ_FMT_Q8B_F32 && fmt != GPHQ_FMT_Q4)
        return GPHQ_ERR_UNSUPPORTED;
    const int64_t n = j->n, k = j->k;
    if (n <= 0 || k <= 0 || k % 32 || k > kMaxPrepWidth || n > INT32_MAX || j->step < 1 || j->row0 < 0)
        return GPHQ_ERR_DIMENSIONS;
    if (!spec_ok(j->in_rot, k) || !spec_ok(j->out_rot, n)) return GPHQ_ERR_DIMENSIONS;
    if (!j->src_bf16_dev || !j->dst_dev || !work_dev || (uintptr_t)work_dev % 16) return GPHQ_ERR_DIMENSIONS;
    if (work_bytes < gphq_prepare_work_bytes(n, k)) return GPHQ_ERR_DIMENSIONS;
    const int64_t last = j->row0 + (n - 1) * j->step;  // the last destination row
    if (j->base < 0 || j->sc < 0 || j->base + region_bytes(fmt, last + 1, k, false) > j->dst_bytes ||
        j->sc + region_bytes(fmt, last + 1, k, true) > j->dst_bytes)
        return GPHQ_ERR_DIMENSIONS;
    if ((fmt != GPHQ_FMT_Q8 && j->sc % 2) || ((fmt == GPHQ_FMT_Q8 || fmt == GPHQ_FMT_Q8B_F32) && j->sc % 4))
        return GPHQ_ERR_DIMENSIONS;
    float *work = (float *)work_dev;
    GPHQ_TRY(prepare_rows_f32(j->src_bf16_dev, n, k, j->norm_host, j->in_rot, j->out_rot, work, work + n * k,
                              (hipStream_t)stream));
    hipStream_t st = (hipStream_t)stream;
    QuantArgs qa{work, (uint8_t *)j->dst_dev, (long)j->base, (long)j->sc, (long)j->step, (long)j->row0,
                 (int)n, (int)k, j->scale_mul};
    const unsigned blocks32 = (unsigned)((n * (k / 32) + 255) / 256);
    switch (fmt) {
    case GPHQ_FMT_Q8: hipLaunchKernelGGL(prep_q8_kernel, dim3((unsigned)n), dim3(256), 0, st, qa); break;
    case GPHQ_FMT_Q8B: hipLaunchKernelGGL(prep_q8b_kernel<false>, dim3(blocks32), dim3(256), 0, st, qa); break;
    case GPHQ_FMT_Q8B_F32: hipLaunchKernelGGL(prep_q8b_kernel<true>, dim3(blocks32), dim3(256), 0, st, qa); break;
    case GPHQ_FMT_Q4: hipLaunchKernelGGL(prep_q4_kernel, dim3(blocks32), dim3(256), 0, st, qa); break;
    }
    GPHQ_TRY(launch_status());
    // The host-side signs and norm must outlive their copies.
    return hip_status(hipStreamSynchronize(st));
}

int gphq_prepare_layer_jobs(const gphq_lm_config *cfg, const float *input_norm_host, const float *post_norm_host,
                            void *dst_dev, int64_t dst_bytes, gphq_prepare_job *jobs) {
    // prepareGPU's dense-layer jobs (gpu_darwin.go:400-415), in its order.
    if (!cfg || !jobs || !input_norm_host || !post_norm_host) return GPHQ_ERR_DIMENSIONS;
    gphq_lm_layer L{};
    int64_t bytes = 0;
    GPHQ_TRY(gphq_lm_layer_layout(cfg, &L, &bytes));
    const int64_t h = cfg->hidden, hd = cfg->head_dim, qd = cfg->heads * hd, kv = cfg->kv_heads * hd,
                  inter = cfg->intermediate;
    const int fmt = cfg->fmt;
    const gphq_rotation_spec none{0, 0}, hidden{h, 0}, head{0, hd};
    // Q8B skips the down projection's input rotation (gpu_darwin.go:209-215).
    const gphq_rotation_spec down_in = fmt == GPHQ_FMT_Q8B ? none : gphq_rotation_spec{inter, 0};
    struct {
        int64_t n, k;
        const float *norm;
        gphq_rotation_spec in, out;
        int64_t base, sc, step, row0;
    } spec[GPHQ_LAYER_PROJECTIONS] = {
        {qd, h, input_norm_host, hidden, none, L.qkv, L.qkv_scale, 1, 0},          // q_proj
        {kv, h, input_norm_host, hidden, none, L.qkv, L.qkv_scale, 1, qd},         // k_proj
        {kv, h, input_norm_host, hidden, head, L.qkv, L.qkv_scale, 1, qd + kv},    // v_proj
        {h, qd, nullptr, head, hidden, L.o, L.o_scale, 1, 0},                      // o_proj
        {inter, h, post_norm_host, hidden, none, L.gu, L.gu_scale, 2, 0},          // gate_proj
        {inter, h, post_norm_host, hidden, none, L.gu, L.gu_scale, 2, 1},          // up_proj
        {h, inter, nullptr, down_in, hidden, L.d, L.d_scale, 1, 0},                // down_proj
    };
    for (int i = 0; i < GPHQ_LAYER_PROJECTIONS; ++i) {
        gphq_prepare_job &j = jobs[i];
        j = gphq_prepare_job{};
        j.n = spec[i].n;
        j.k = spec[i].k;
        j.norm_host = spec[i].norm;
        j.in_rot = spec[i].in;
        j.out_rot = spec[i].out;
        j.fmt = fmt;
        j.dst_dev = dst_dev;
        j.dst_bytes = dst_bytes;
        j.base = spec[i].base;
        j.sc = spec[i].sc;
        j.step = spec[i].step;
        j.row0 = spec[i].row0;
        j.scale_mul = 1.0f;
    }
    return GPHQ_OK;
}

int64_t gphq_prepare_head_chunk_rows(const gphq_lm_config *cfg) {
    // gpu_darwin.go:432-436: the head is read in chunks of max(inter, 4096) rows.
    if (!cfg || cfg->intermediate <= 0) return GPHQ_ERR_DIMENSIONS;
    return std::max<int64_t>(cfg->intermediate, 4096);
}

int gphq_prepare_head_job(const gphq_lm_config *cfg, int64_t row0, void *dst_dev, int64_t dst_bytes,
                          gphq_prepare_job *job) {
    // One head chunk (gpu_darwin.go:435): vocabulary rows row0.. of at most
    // one chunk over hidden-rotated rows, Q8B whatever the layers' format.
    if (!cfg || !job || row0 < 0 || row0 >= cfg->vocab) return GPHQ_ERR_DIMENSIONS;
    int64_t rows = 0, sc = 0, bytes = 0;
    GPHQ_TRY(gphq_lm_head_layout(cfg, &rows, &sc, &bytes));
    const int64_t chunk = gphq_prepare_head_chunk_rows(cfg);
    *job = gphq_prepare_job{};
    job->n = std::min(chunk, cfg->vocab - row0);
    job->k = cfg->hidden;
    job->in_rot = gphq_rotation_spec{cfg->hidden, 0};
    job->fmt = GPHQ_FMT_Q8B;
    job->dst_dev = dst_dev;
    job->dst_bytes = dst_bytes;
    job->base = 0;
    job->sc = sc;
    job->step = 1;
    job->row0 = row0;
    job->scale_mul = 1.0f;
    return GPHQ_OK;
}

int64_t gphq_prepare_lm_work_bytes(const gphq_lm_config *cfg) {
    if (!cfg) return GPHQ_ERR_DIMENSIONS;
    gphq_prepare_job jobs[GPHQ_LAYER_PROJECTIONS];
    static const float one = 1.0f;  // placeholders: only the shapes are read
    GPHQ_TRY(gphq_prepare_layer_jobs(cfg, &one, &one, nullptr, 0, jobs));
    int64_t most = 0;
    for (const gphq_prepare_job &j : jobs) {
        const int64_t b = gphq_prepare_work_bytes(j.n, j.k);
        if (b < 0) return b;
        most = std::max(most, b);
    }
    const int64_t head = gphq_prepare_work_bytes(std::min(gphq_prepare_head_chunk_rows(cfg), cfg->vocab), cfg->hidden);
    if (head < 0) return head;
    return std::max(most, head);
}

int gphq_prepare_layer(const gphq_lm_config *cfg, const uint16_t *const *src_bf16_dev, const float *input_norm_host,
                       const float *post_norm_host, void *dst_dev, int64_t dst_bytes, void *work_dev,
                       int64_t work_bytes, void *stream) {
    if (!src_bf16_dev) return GPHQ_ERR_DIMENSIONS;
    gphq_prepare_job jobs[GPHQ_LAYER_PROJECTIONS];
    GPHQ_TRY(gphq_prepare_layer_jobs(cfg, input_norm_host, post_norm_host, dst_dev, dst_bytes, jobs));
    for (int i = 0; i < GPHQ_LAYER_PROJECTIONS; ++i) {
        jobs[i].src_bf16_dev = src_bf16_dev[i];
        GPHQ_TRY(gphq_prepare_projection(&jobs[i], work_dev, work_bytes, stream));
    }
    return GPHQ_OK;
}

int gphq_prepare_head(const gphq_lm_config *cfg, const uint16_t *src_bf16_dev, void *dst_dev, int64_t dst_bytes,
                      void *work_dev, int64_t work_bytes, void *stream) {
    if (!cfg || !src_bf16_dev) return GPHQ_ERR_DIMENSIONS;
    const int64_t chunk = gphq_prepare_head_chunk_rows(cfg);
    if (chunk < 0) return (int)chunk;
    for (int64_t r = 0; r < cfg->vocab; r += chunk) {
        gphq_prepare_job j;
        GPHQ_TRY(gphq_prepare_head_job(cfg, r, dst_dev, dst_bytes, &j));
        j.src_bf16_dev = src_bf16_dev + r * cfg->hidden;
        GPHQ_TRY(gphq_prepare_projection(&j, work_dev, work_bytes, stream));
    }
    return GPHQ_OK;
}

}  // extern "C"
