// Host side of the q8gemm FP16 path (Weights / Workspace / MulPanels /
// MulInto, q8gemm/packed.go and gemm.go) and of the qwen3lm mm entry point,
// behind the C ABI. Argument checks follow the reference in order.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "common.h"
#include "gemm_f16.h"

namespace gphq {
int gemv_gptq_launch(const void *codes, const void *scales, const uint8_t *zeros, const float *x, float *y, int K,
                     int N, hipStream_t stream);
int f16_act_pack_plain(const float *x, long stride, int rows, int K, _Float16 *act, hipStream_t stream);
int f16_act_pack(const float *x, long stride, int rows, int K, int kt, int mode, int k0, int k1, _Float16 *act,
                 float *rowScale, float *rowInv, hipStream_t stream);
int f16_pack_tiles(const uint16_t *src, uint16_t *dst, int rows, int K, int row0, int kt, hipStream_t stream);
int f16_ref_panels_to_tiles(const uint16_t *ref, uint16_t *dst, int n, int K, int nt, int kt, hipStream_t stream);
int i8_pack_tiles(const int8_t *src, int8_t *dst, int rows, int K, int row0, int kt, hipStream_t stream);
int fill_zero_columns(float *dst, long stride, int rows, int c0, int c1, hipStream_t stream);
int bf16_rows_to_f16(const uint16_t *src, int rows, int K, uint16_t *dst, float *rowScale, unsigned long long *rounded,
                     hipStream_t stream);
}  // namespace gphq

using namespace gphq;

static constexpr int64_t kOutputPanel = 64;  // q8gemm/packed.go:17
static int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }


struct gphq_weights {
    int64_t k = 0, n = 0, kt = 0, nt = 0;
    bool f16 = false;
    bool owned = true;     // storage allocated here (false: bound caller buffer)
    void *codes = nullptr;  // int8 tile layout (1 KiB groups) or FP16 tile layout (2 KiB groups)
    float *scales = nullptr;  // [nt * 16]
    size_t code_bytes() const { return (size_t)nt * kt * 1024 * (f16 ? 2 : 1); }
};

struct gphq_workspace {
    int64_t kcap = 0, rowcap = 0;
    int64_t k = 0, rows = 0, kt = 0;
    _Float16 *act = nullptr;
    float *rowScale = nullptr, *rowInv = nullptr;
    std::vector<float> hScale, hInv;
    bool dirty = false;
};

static int alloc_zero(void **p, size_t bytes) {
    *p = nullptr;
    if (!bytes) return GPHQ_OK;
    GPHQ_TRY(hip_status(hipMalloc(p, bytes)));
    return hip_status(hipMemset(*p, 0, bytes));
}

static gphq_weights *make_weights(int64_t k, int64_t n, bool f16) {
    auto *w = new (std::nothrow) gphq_weights();
    if (!w) return nullptr;
    w->k = k;
    w->n = n;
    w->kt = ceil_div(k, 64);
    w->nt = ceil_div(n, 16);
    w->f16 = f16;
    return w;
}

extern "C" {

int gphq_q8gemm_new_weights(int64_t k, int64_t n, gphq_weights **out) {
    // packed.go:43-61 NewWeights (int8 storage).
    if (!out) return GPHQ_ERR_DIMENSIONS;
    *out = nullptr;
    if (k < 0 || n < 0 || k > INT32_MAX - 64 || n > INT32_MAX - 64) return GPHQ_ERR_DIMENSIONS;
    gphq_weights *w = make_weights(k, n, false);
    if (!w) return GPHQ_ERR_DIMENSIONS;
    int st = alloc_zero(&w->codes, w->code_bytes());
    if (st == GPHQ_OK) st = alloc_zero((void **)&w->scales, (size_t)w->nt * 16 * 4);
    if (st != GPHQ_OK) {
        (void)hipFree(w->codes);
        (void)hipFree(w->scales);
        delete w;
        return st;
    }
    *out = w;
    return GPHQ_OK;
}

int gphq_q8gemm_new_weights_f16(int64_t k, int64_t n, gphq_weights **out) {
    // packed.go:63-76 NewWeightsF16.
    if (!out) return GPHQ_ERR_DIMENSIONS;
    *out = nullptr;
    if (k < 0 || n < 0 || k > INT32_MAX - 64 || n > INT32_MAX - 64) return GPHQ_ERR_DIMENSIONS;
    gphq_weights *w = make_weights(k, n, true);
    if (!w) return GPHQ_ERR_DIMENSIONS;
    int st = alloc_zero(&w->codes, w->code_bytes());
    if (st == GPHQ_OK) st = alloc_zero((void **)&w->scales, (size_t)w->nt * 16 * 4);
    if (st != GPHQ_OK) {
        (void)hipFree(w->codes);
        (void)hipFree(w->scales);
        delete w;
        return st;
    }
    *out = w;
    return GPHQ_OK;
}

int64_t gphq_q8gemm_weights_f16_bytes(int64_t k, int64_t n) {
    // packed.go:78-93 WeightsF16Bytes, for this library's layout: FP16 codes in
    // [n/16][k/64][64][16] groups followed by n/16*16 fp32 scales. Returns a
    // negative status for invalid dimensions (the reference's ErrDimensions).
    if (k < 0 || n < 0 || k > INT32_MAX - 64 || n > INT32_MAX - 64) return GPHQ_ERR_DIMENSIONS;
    const int64_t nt = ceil_div(n, 16), kt = ceil_div(k, 64);
    return nt * kt * 2048 + nt * 16 * 4;
}

int gphq_q8gemm_new_weights_f16_buffer(int64_t k, int64_t n, void *data_dev, int64_t data_len, gphq_weights **out) {
    // packed.go:95-121 NewWeightsF16Buffer: binds caller-owned, zeroed,
    // 4-byte-aligned device storage of at least weights_f16_bytes(k, n).
    if (!out) return GPHQ_ERR_DIMENSIONS;
    *out = nullptr;
    const int64_t size = gphq_q8gemm_weights_f16_bytes(k, n);
    if (size < 0 || data_len < size) return GPHQ_ERR_DIMENSIONS;
    if (size > 0 && (!data_dev || (uintptr_t)data_dev % 4 != 0)) return GPHQ_ERR_DIMENSIONS;
    gphq_weights *w = make_weights(k, n, true);
    if (!w) return GPHQ_ERR_DIMENSIONS;
    w->owned = false;
    w->codes = data_dev;
    w->scales = (float *)((char *)data_dev + w->code_bytes());
    *out = w;
    return GPHQ_OK;
}

int64_t gphq_q8gemm_reference_f16_bytes(int64_t k, int64_t n) {
    // packed.go:78-93 WeightsF16Bytes: the reference's own layout, FP16
    // panels [ceil(n/64)][ceil(k/2)][64][2] followed by n fp32 row scales.
    if (k < 0 || n < 0 || k > INT32_MAX - 64 || n > INT32_MAX - 64) return GPHQ_ERR_DIMENSIONS;
    return ceil_div(n, kOutputPanel) * ((k + 1) / 2) * 4 * kOutputPanel + n * 4;
}

int gphq_q8gemm_weights_f16_load_reference(gphq_weights *w, const void *ref_host, int64_t ref_len) {
    // The bytes a reference NewWeightsF16Buffer + PackBF16 leave in the
    // caller's storage (a wcache mapping, qwen3lm/weights.go:362-370; packed.go
    // 95-175), copied from host memory and repacked on the device.
    if (!w || !w->f16) return GPHQ_ERR_DIMENSIONS;
    const int64_t size = gphq_q8gemm_reference_f16_bytes(w->k, w->n);
    if (size < 0 || ref_len < size) return GPHQ_ERR_DIMENSIONS;
    if (size == 0) return GPHQ_OK;
    if (!ref_host) return GPHQ_ERR_DIMENSIONS;
    const int64_t code_bytes = size - 4 * w->n;
    const float *scales = (const float *)((const char *)ref_host + code_bytes);
    for (int64_t r = 0; r < w->n; ++r) {
        float s;
        std::memcpy(&s, scales + r, 4);
        if (!std::isfinite(s)) return GPHQ_ERR_NON_FINITE;
    }
    void *staging = nullptr;
    GPHQ_TRY(hip_status(hipMalloc(&staging, (size_t)size)));
    int st = hip_status(hipMemcpy(staging, ref_host, (size_t)size, hipMemcpyHostToDevice));
    if (st == GPHQ_OK && code_bytes)
        st = f16_ref_panels_to_tiles((const uint16_t *)staging, (uint16_t *)w->codes, (int)w->n, (int)w->k,
                                     (int)w->nt, (int)w->kt, nullptr);
    if (st == GPHQ_OK && w->n)
        st = hip_status(hipMemcpyAsync(w->scales, (const char *)staging + code_bytes, (size_t)w->n * 4,
                                       hipMemcpyDeviceToDevice, nullptr));
    if (st == GPHQ_OK) st = hip_status(hipStreamSynchronize(nullptr));
    (void)hipFree(staging);
    return st;
}

void gphq_q8gemm_weights_free(gphq_weights *w) {
    if (!w) return;
    if (w->owned) {
        (void)hipFree(w->codes);
        (void)hipFree(w->scales);
    }
    delete w;
}

int gphq_q8gemm_weights_pack(gphq_weights *w, const int8_t *q, int64_t q_len, const float *scales,
                             int64_t scales_len) {
    // packed.go:181-204 Pack (int8 weights).
    if (!w || (w->f16 && w->k * w->n != 0) || q_len != w->k * w->n || scales_len != w->n) return GPHQ_ERR_DIMENSIONS;
    for (int64_t i = 0; i < scales_len; ++i)
        if (std::isnan(scales[i]) || std::isinf(scales[i])) return GPHQ_ERR_NON_FINITE;
    if (scales_len) GPHQ_TRY(hip_status(hipMemcpy(w->scales, scales, (size_t)scales_len * 4, hipMemcpyHostToDevice)));
    if (w->code_bytes()) GPHQ_TRY(hip_status(hipMemset(w->codes, 0, w->code_bytes())));
    if (q_len == 0) return GPHQ_OK;
    int8_t *staging = nullptr;
    GPHQ_TRY(hip_status(hipMalloc(&staging, (size_t)q_len)));
    int st = hip_status(hipMemcpy(staging, q, (size_t)q_len, hipMemcpyHostToDevice));
    if (st == GPHQ_OK) st = i8_pack_tiles(staging, (int8_t *)w->codes, (int)w->n, (int)w->k, 0, (int)w->kt, nullptr);
    if (st == GPHQ_OK) st = hip_status(hipStreamSynchronize(nullptr));
    (void)hipFree(staging);
    return st;
}

static bool bf16_finite(uint16_t b) { return (b & 0x7f80) != 0x7f80; }

int gphq_q8gemm_weights_pack_bf16_rows(gphq_weights *w, const uint16_t *bf16, int64_t len, int64_t row0,
                                       int64_t *rounded) {
    // packed.go:127-175 PackBF16Rows: per row, an exact power-of-two shift of
    // the row into [2^14, 2^15), FP16 conversion, count of rounded values.
    if (rounded) *rounded = 0;
    if (!w || !w->f16 || w->k == 0 || len % w->k != 0 || row0 < 0 || row0 + len / w->k > w->n)
        return GPHQ_ERR_DIMENSIONS;
    const int64_t rows = len / w->k;
    // The reference stops at the first row holding a non-finite value, after
    // packing the rows before it; find that row first.
    int64_t good = rows;
    for (int64_t r = 0; r < rows && good == rows; ++r)
        for (int64_t i = 0; i < w->k; ++i)
            if (!bf16_finite(bf16[r * w->k + i])) {
                good = r;
                break;
            }
    int st = GPHQ_OK;
    if (good > 0) {
        const size_t count = (size_t)good * w->k;
        uint16_t *src = nullptr, *conv = nullptr;
        unsigned long long *cnt = nullptr;
        float *dscale = nullptr;
        st = hip_status(hipMalloc(&src, count * 2));
        if (st == GPHQ_OK) st = hip_status(hipMalloc(&conv, count * 2));
        if (st == GPHQ_OK) st = hip_status(hipMalloc(&cnt, sizeof(unsigned long long)));
        if (st == GPHQ_OK) st = hip_status(hipMalloc(&dscale, (size_t)good * 4));
        if (st == GPHQ_OK) st = hip_status(hipMemset(cnt, 0, sizeof(unsigned long long)));
        if (st == GPHQ_OK) st = hip_status(hipMemcpy(src, bf16, count * 2, hipMemcpyHostToDevice));
        if (st == GPHQ_OK) st = bf16_rows_to_f16(src, (int)good, (int)w->k, conv, dscale, cnt, nullptr);
        if (st == GPHQ_OK)
            st = f16_pack_tiles(conv, (uint16_t *)w->codes, (int)good, (int)w->k, (int)row0, (int)w->kt, nullptr);
        if (st == GPHQ_OK)
            st = hip_status(hipMemcpy(w->scales + row0, dscale, (size_t)good * 4, hipMemcpyDeviceToDevice));
        unsigned long long h = 0;
        if (st == GPHQ_OK) st = hip_status(hipMemcpy(&h, cnt, sizeof(h), hipMemcpyDeviceToHost));
        if (st == GPHQ_OK && rounded && good == rows) *rounded = (int64_t)h;
        (void)hipFree(src);
        (void)hipFree(conv);
        (void)hipFree(cnt);
        (void)hipFree(dscale);
    }
    if (st != GPHQ_OK) return st;
    return good == rows ? GPHQ_OK : GPHQ_ERR_NON_FINITE;
}

int gphq_q8gemm_weights_pack_bf16(gphq_weights *w, const uint16_t *bf16, int64_t len, int64_t *rounded) {
    // packed.go:127-146 PackBF16: clear, then every row (k == 0: scales = 1).
    if (rounded) *rounded = 0;
    if (!w || !w->f16 || len != w->k * w->n) return GPHQ_ERR_DIMENSIONS;
    if (w->code_bytes()) GPHQ_TRY(hip_status(hipMemset(w->codes, 0, w->code_bytes())));
    if (w->k == 0) {
        std::vector<float> ones((size_t)w->n, 1.0f);
        if (w->n) GPHQ_TRY(hip_status(hipMemcpy(w->scales, ones.data(), (size_t)w->n * 4, hipMemcpyHostToDevice)));
        return GPHQ_OK;
    }
    return gphq_q8gemm_weights_pack_bf16_rows(w, bf16, len, 0, rounded);
}

int gphq_q8gemm_weights_dims(const gphq_weights *w, int64_t *k, int64_t *n) {
    if (k) *k = w ? w->k : 0;
    if (n) *n = w ? w->n : 0;
    return GPHQ_OK;
}
int64_t gphq_q8gemm_weights_panels(const gphq_weights *w) { return w ? ceil_div(w->n, kOutputPanel) : 0; }
int64_t gphq_q8gemm_weights_bytes(const gphq_weights *w) { return w ? (int64_t)w->code_bytes() + 4 * w->n : 0; }
int gphq_q8gemm_weights_is_f16(const gphq_weights *w) { return w && w->f16 ? 1 : 0; }

int gphq_q8gemm_new_workspace(int64_t k, int64_t max_rows, gphq_workspace **out) {
    // gemm.go:58-69 NewWorkspace with a row capacity.
    if (!out) return GPHQ_ERR_DIMENSIONS;
    *out = nullptr;
    if (k < 0 || max_rows < 0 || k > INT32_MAX - 64 || max_rows > INT32_MAX - 16) return GPHQ_ERR_DIMENSIONS;
    auto *ws = new (std::nothrow) gphq_workspace();
    if (!ws) return GPHQ_ERR_DIMENSIONS;
    ws->kcap = k;
    ws->rowcap = max_rows;
    ws->hScale.assign((size_t)max_rows, 1.0f);
    ws->hInv.assign((size_t)max_rows, 1.0f);
    int st = alloc_zero((void **)&ws->act, (size_t)ceil_div(max_rows, 16) * ceil_div(k, 64) * 2048);
    if (st == GPHQ_OK) st = alloc_zero((void **)&ws->rowScale, (size_t)max_rows * 4);
    if (st == GPHQ_OK) st = alloc_zero((void **)&ws->rowInv, (size_t)max_rows * 4);
    if (st != GPHQ_OK) {
        (void)hipFree(ws->act);
        (void)hipFree(ws->rowScale);
        (void)hipFree(ws->rowInv);
        delete ws;
        return st;
    }
    *out = ws;
    return GPHQ_OK;
}

void gphq_q8gemm_workspace_free(gphq_workspace *ws) {
    if (!ws) return;
    (void)hipFree(ws->act);
    (void)hipFree(ws->rowScale);
    (void)hipFree(ws->rowInv);
    delete ws;
}

int gphq_q8gemm_workspace_prepare(gphq_workspace *ws, int64_t rows, int64_t k) {
    // gemm.go:79-89 Prepare: shape, row scales and inverses reset to 1.
    if (!ws || rows < 0 || rows > ws->rowcap || k < 0 || k > ws->kcap) return GPHQ_ERR_DIMENSIONS;
    ws->k = k;
    ws->rows = rows;
    ws->kt = ceil_div(k, 64);
    std::fill(ws->hScale.begin(), ws->hScale.end(), 1.0f);
    std::fill(ws->hInv.begin(), ws->hInv.end(), 1.0f);
    ws->dirty = true;
    return GPHQ_OK;
}

int gphq_q8gemm_workspace_prepare_row_f16(gphq_workspace *ws, int64_t k) {
    // gemm.go:91-104 PrepareRowF16 needs the SME row kernel; like the
    // reference on any CPU without SME (amd64 included), it is ErrDimensions.
    (void)ws;
    (void)k;
    return GPHQ_ERR_DIMENSIONS;
}

int gphq_q8gemm_workspace_prepare_rows_f16(gphq_workspace *ws, int64_t rows, int64_t k) {
    // gemm.go:106-122 PrepareRowsF16: SME-only, ErrDimensions elsewhere.
    (void)ws;
    (void)rows;
    (void)k;
    return GPHQ_ERR_DIMENSIONS;
}

int gphq_q8gemm_workspace_set_row_scale(gphq_workspace *ws, int64_t row, float max_abs) {
    // gemm.go:127-136 SetRowScale.
    if (!ws || row < 0 || row >= ws->rows) return GPHQ_ERR_DIMENSIONS;
    int e = 0;
    if (max_abs > 0 && !std::isinf(max_abs) && !std::isnan(max_abs)) {
        int ex;
        std::frexp((double)max_abs, &ex);
        e = std::min(std::max(15 - ex, -100), 100);
    }
    ws->hScale[(size_t)row] = (float)std::ldexp(1.0, e);
    ws->hInv[(size_t)row] = (float)std::ldexp(1.0, -e);
    ws->dirty = true;
    return GPHQ_OK;
}

int gphq_q8gemm_workspace_pack_range(gphq_workspace *ws, const float *x, int64_t x_len, int64_t stride, int64_t k0,
                                     int64_t k1, void *stream) {
    // gemm.go:152-226 PackRange. The device pass converts whole rows with the
    // set scales; [k0, k1) must be a legal range, and converting outside it
    // rewrites values that an earlier call produced from the same input.
    if (!ws || k0 < 0 || k1 > ws->k || k0 > k1 || k0 % 2 != 0 || (k1 % 2 != 0 && k1 != ws->k) || stride < ws->k ||
        (ws->rows > 0 && x_len < (ws->rows - 1) * stride + ws->k))
        return GPHQ_ERR_DIMENSIONS;
    if (ws->rows == 0) return GPHQ_OK;
    hipStream_t s = (hipStream_t)stream;
    if (ws->dirty) {
        GPHQ_TRY(hip_status(
            hipMemcpyAsync(ws->rowScale, ws->hScale.data(), (size_t)ws->rows * 4, hipMemcpyHostToDevice, s)));
        GPHQ_TRY(hip_status(hipMemcpyAsync(ws->rowInv, ws->hInv.data(), (size_t)ws->rows * 4, hipMemcpyHostToDevice, s)));
        GPHQ_TRY(hip_status(hipStreamSynchronize(s)));
        ws->dirty = false;
    }
    if (ws->k == 0 || k0 == k1) return GPHQ_OK;
    if (!x) return GPHQ_ERR_DIMENSIONS;
    // mode 2: scales already on the device, columns [k0, k1) only.
    return f16_act_pack(x, (long)stride, (int)ws->rows, (int)ws->k, (int)ws->kt, 2, (int)k0, (int)k1, ws->act,
                        ws->rowScale, ws->rowInv, s);
}

int gphq_q8gemm_workspace_pack(gphq_workspace *ws, const float *x, int64_t x_len, int64_t rows, int64_t k,
                               int64_t stride, void *stream) {
    // gemm.go:71-77 Pack: Prepare, SetRowScale(MaxAbs(row)), PackRange(0, k),
    // fused on the device.
    GPHQ_TRY(gphq_q8gemm_workspace_prepare(ws, rows, k));
    if (stride < k || (rows > 0 && x_len < (rows - 1) * stride + k)) return GPHQ_ERR_DIMENSIONS;
    ws->dirty = false;
    if (rows == 0) return GPHQ_OK;
    if (k == 0) {
        ws->dirty = true;  // scales stay 1 (MaxAbs of an empty row is 0)
        return GPHQ_OK;
    }
    if (!x) return GPHQ_ERR_DIMENSIONS;
    return f16_act_pack(x, (long)stride, (int)rows, (int)k, (int)ws->kt, 0, 0, (int)k, ws->act, ws->rowScale,
                        ws->rowInv, (hipStream_t)stream);
}

int gphq_q8gemm_workspace_row_scales(const gphq_workspace *ws, float *scale_dev, float *inverse_dev, void *stream) {
    if (!ws) return GPHQ_ERR_DIMENSIONS;
    if (ws->rows == 0) return GPHQ_OK;
    hipStream_t s = (hipStream_t)stream;
    if (ws->dirty) {
        if (scale_dev)
            GPHQ_TRY(hip_status(hipMemcpyAsync(scale_dev, ws->hScale.data(), (size_t)ws->rows * 4, hipMemcpyHostToDevice, s)));
        if (inverse_dev)
            GPHQ_TRY(hip_status(hipMemcpyAsync(inverse_dev, ws->hInv.data(), (size_t)ws->rows * 4, hipMemcpyHostToDevice, s)));
        return hip_status(hipStreamSynchronize(s));
    }
    if (scale_dev)
        GPHQ_TRY(hip_status(hipMemcpyAsync(scale_dev, ws->rowScale, (size_t)ws->rows * 4, hipMemcpyDeviceToDevice, s)));
    if (inverse_dev)
        GPHQ_TRY(hip_status(hipMemcpyAsync(inverse_dev, ws->rowInv, (size_t)ws->rows * 4, hipMemcpyDeviceToDevice, s)));
    return GPHQ_OK;
}

int gphq_q8gemm_workspace_activations(const gphq_workspace *ws, uint16_t *act_dev, void *stream) {
    // The prepared rows' packed FP16 values as row-major [rows][k] bits (the
    // values the reference's Workspace.activation holds, in logical order).
    if (!ws || !act_dev) return GPHQ_ERR_DIMENSIONS;
    if (ws->rows == 0 || ws->k == 0) return GPHQ_OK;
    std::vector<uint16_t> tiles((size_t)ceil_div(ws->rows, 16) * ws->kt * 1024);
    hipStream_t s = (hipStream_t)stream;
    GPHQ_TRY(hip_status(hipStreamSynchronize(s)));
    GPHQ_TRY(hip_status(hipMemcpy(tiles.data(), ws->act, tiles.size() * 2, hipMemcpyDeviceToHost)));
    std::vector<uint16_t> out((size_t)ws->rows * ws->k);
    for (int64_t r = 0; r < ws->rows; ++r)
        for (int64_t kk = 0; kk < ws->k; ++kk)
            out[(size_t)(r * ws->k + kk)] = tiles[((size_t)(r >> 4) * ws->kt + (kk >> 6)) * 1024 +
                                                  (size_t)(((kk & 63) >> 4) * 16 + (r & 15)) * 16 + (kk & 15)];
    return hip_status(hipMemcpy(act_dev, out.data(), out.size() * 2, hipMemcpyHostToDevice));
}

int gphq_q8gemm_mul_panels(float *dst, int64_t dst_len, int64_t stride, gphq_workspace *ws,
                           const gphq_weights *w, int64_t p0, int64_t p1, void *stream) {
    // gemm.go:228-272 MulPanels (the portable scratch argument has no
    // counterpart: the device kernel needs none).
    if (!w || !ws || ws->k != w->k || p0 < 0 || p1 > ceil_div(w->n, kOutputPanel) || p0 > p1 || stride < w->n)
        return GPHQ_ERR_DIMENSIONS;
    if (ws->rows == 0 || p0 == p1) return GPHQ_OK;
    if (dst_len < (ws->rows - 1) * stride + w->n || !dst) return GPHQ_ERR_DIMENSIONS;
    hipStream_t s = (hipStream_t)stream;
    const int64_t c0 = p0 * kOutputPanel, c1 = std::min(p1 * kOutputPanel, w->n);
    if (w->k == 0) return fill_zero_columns(dst, (long)stride, (int)ws->rows, (int)c0, (int)c1, s);
    if (ws->dirty) {
        // Row scales set on the host since the last PackRange: upload them.
        GPHQ_TRY(hip_status(hipMemcpyAsync(ws->rowInv, ws->hInv.data(), (size_t)ws->rows * 4, hipMemcpyHostToDevice, s)));
        GPHQ_TRY(hip_status(hipMemcpyAsync(ws->rowScale, ws->hScale.data(), (size_t)ws->rows * 4, hipMemcpyHostToDevice, s)));
        GPHQ_TRY(hip_status(hipStreamSynchronize(s)));
        ws->dirty = false;
    }
    F16GemmArgs a{};
    a.A = ws->act;
    a.B = w->codes;
    a.colScale = w->scales;
    a.rowInv = ws->rowInv;
    a.dst = dst;
    a.stride = (long)stride;
    a.M = (int)ws->rows;
    a.N = (int)w->n;
    a.K = (int)w->k;
    a.KT = (int)w->kt;
    a.c0 = (int)c0;
    a.c1 = (int)c1;
    return f16gemm_launch(w->f16 ? W_F16_TILE : W_I8_TILE, EPI_PANELS, a, s);
}

int gphq_q8gemm_mul_into(float *dst, int64_t dst_len, const float *x, int64_t x_len, int64_t rows,
                         const gphq_weights *w, gphq_workspace *ws, void *stream) {
    // gemm.go:274-286 MulInto: rows of x, packed with ws, times all panels.
    if (!w || !ws || rows < 0 || rows > ws->rowcap || dst_len < rows * w->n || x_len < rows * w->k)
        return GPHQ_ERR_DIMENSIONS;
    if (rows == 0 || w->n == 0) return GPHQ_OK;
    GPHQ_TRY(gphq_q8gemm_workspace_pack(ws, x, rows * w->k, rows, w->k, w->k, stream));
    return gphq_q8gemm_mul_panels(dst, dst_len, w->n, ws, w, 0, ceil_div(w->n, kOutputPanel), stream);
}

// ---- qwen3lm mm ------------------------------------------------------------

int64_t gphq_mm_workspace_bytes(int64_t m, int64_t k) {
    if (m < 0 || k < 0) return GPHQ_ERR_DIMENSIONS;
    return ceil_div(m, 16) * ceil_div(k, 64) * 2048;
}

// Activation tiles, then (256-byte aligned) the split-K partial sums the
// 128 x 128-tile GEMM uses for 64 < m with a grid under 512 blocks.
int64_t gphq_mm_split_workspace_bytes(int64_t m, int64_t k, int64_t n) {
    if (m < 0 || k < 0 || n < 0 || m > INT32_MAX || k > INT32_MAX || n > INT32_MAX) return GPHQ_ERR_DIMENSIONS;
    const int64_t act = (gphq_mm_workspace_bytes(m, k) + 255) / 256 * 256;
    if (m <= 64) return act;
    const int splits = mm_split_count(ceil_div(m, 128) * ceil_div(n, 128), (int)ceil_div(k, 64), m * n);
    return act + (splits > 1 ? (int64_t)splits * m * n * 4 : 0);
}

int gphq_mm(int fmt, const void *codes, const void *scales, const uint8_t *zeros, const float *x, float *y,
            int64_t m, int64_t k, int64_t n, void *work, int64_t work_bytes, void *stream) {
    int wf;
    int epi = EPI_PLAIN;
    switch (fmt) {
    case GPHQ_FMT_Q8:
        wf = W_Q8_ROW;
        epi = EPI_ROWSCALE;
        break;
    case GPHQ_FMT_Q8B:
        wf = W_Q8B_ROW;
        break;
    case GPHQ_FMT_Q8B_F32:
        wf = W_Q8BF_ROW;
        break;
    case GPHQ_FMT_Q4:
        wf = W_Q4_ROW;
        break;
    case GPHQ_FMT_GPTQ4_G128:
        wf = W_GPTQ_ROW;
        break;
    default:
        return GPHQ_ERR_UNSUPPORTED;
    }
    if (m < 0 || k < 0 || n < 0 || m > INT32_MAX || k > INT32_MAX || n > INT32_MAX) return GPHQ_ERR_DIMENSIONS;
    if (k % (fmt == GPHQ_FMT_GPTQ4_G128 ? 128 : 32) != 0) return GPHQ_ERR_DIMENSIONS;
    if (m == 0 || n == 0) return GPHQ_OK;
    if (!y || !scales) return GPHQ_ERR_DIMENSIONS;
    if (work_bytes < gphq_mm_workspace_bytes(m, k)) return GPHQ_ERR_DIMENSIONS;
    hipStream_t s = (hipStream_t)stream;
    if (k == 0) return fill_zero_columns(y, (long)n, (int)m, 0, (int)n, s);
    if (!codes || !x || !work || (uintptr_t)codes % 16 != 0 || (uintptr_t)work % 16 != 0) return GPHQ_ERR_DIMENSIONS;
    if (fmt == GPHQ_FMT_GPTQ4_G128 && !zeros) return GPHQ_ERR_DIMENSIONS;
    if (fmt == GPHQ_FMT_GPTQ4_G128 && m == 1) {
        // One activation row: the GEMV kernel (same arithmetic, fp32 sums).
        const int st = gemv_gptq_launch(codes, scales, zeros, x, y, (int)k, (int)n, s);
        if (st != GPHQ_ERR_UNSUPPORTED) return st;
    }
    const int64_t kt = ceil_div(k, 64);
    GPHQ_TRY(f16_act_pack_plain(x, (long)k, (int)m, (int)k, (_Float16 *)work, s));
    F16GemmArgs a{};
    a.A = (const _Float16 *)work;
    a.B = codes;
    a.bScale = scales;
    a.bZero = zeros;
    a.colScale = (const float *)scales;
    a.dst = y;
    a.stride = (long)n;
    a.M = (int)m;
    a.N = (int)n;
    a.K = (int)k;
    a.KT = (int)kt;
    a.c0 = 0;
    a.c1 = (int)n;
    const int64_t act = (gphq_mm_workspace_bytes(m, k) + 255) / 256 * 256;
    if (m > 64 && work_bytes >= gphq_mm_split_workspace_bytes(m, k, n)) a.part = (float *)((char *)work + act);
    return f16gemm_launch(wf, epi, a, s);
}

}  // extern "C"
