// Host side of the q8gemm int8 x int8 path: device-resident WeightsI8 and
// WorkspaceI8 behind the C ABI. Argument checks follow q8gemm/int8.go in the
// same order and return the same error values.
#include <algorithm>
#include <cmath>
#include <new>
#include <vector>

#include "common.h"

namespace gphq {
int i8gemm_launch(const int8_t *A, const int8_t *B, const float *rowScale, const float *colScale, float *dst,
                  long stride, int M, int N, int KT, int c0, int c1, hipStream_t stream);
int i8_pack_tiles(const int8_t *src, int8_t *dst, int rows, int K, int row0, int kt, hipStream_t stream);
int i8_pack_rows(const float *x, long stride, int rows, int K, int kt, int8_t *act, float *rowScale, float *rowInv,
                 hipStream_t stream);
int i8_pack_range(const float *x, long stride, int rows, int K, int kt, int k0, int k1, int8_t *act,
                  const float *rowInv, hipStream_t stream);
int fill_zero_columns(float *dst, long stride, int rows, int c0, int c1, hipStream_t stream);
int fill_f32(float *dst, size_t n, float v, hipStream_t stream);
}  // namespace gphq

using namespace gphq;

// q8gemm/packed.go:17,19 and int8.go:214-222.
static constexpr int64_t kOutputPanel = 64;
static constexpr int64_t kStripColumns = 16;

struct gphq_weights_i8 {
    int64_t k = 0, n = 0, kt = 0, nt = 0;
    int8_t *q = nullptr;       // tile layout, nt * kt * 1024 bytes
    float *scales = nullptr;   // nt * 16 floats (zero past n)
    size_t qbytes() const { return (size_t)nt * kt * 1024; }
};

struct gphq_workspace_i8 {
    int64_t kcap = 0, rowcap = 0;
    int64_t k = 0, rows = 0, kt = 0;
    int8_t *act = nullptr;      // tile layout for the prepared k
    float *rowScale = nullptr;  // [rowcap]
    float *rowInv = nullptr;    // [rowcap]
    std::vector<float> hScale, hInv;
    // Rows whose host scales are newer than the device copy. The fused Pack
    // computes every row's scales on the device, so it leaves all rows clean;
    // PackRange uploads only the rows SetRowScale or Prepare touched since.
    std::vector<uint8_t> rowDirty;
    bool dirty = false;  // some rowDirty entry is set
};

static int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

extern "C" {

int gphq_q8gemm_new_weights_i8(int64_t k, int64_t n, gphq_weights_i8 **out) {
    // int8.go:20-32 NewWeightsI8.
    if (!out) return GPHQ_ERR_DIMENSIONS;
    *out = nullptr;
    if (k < 0 || n < 0 || k > INT32_MAX - 64 || n > INT32_MAX - 64) return GPHQ_ERR_DIMENSIONS;
    auto *w = new (std::nothrow) gphq_weights_i8();
    if (!w) return GPHQ_ERR_DIMENSIONS;
    w->k = k;
    w->n = n;
    w->kt = ceil_div(k, 64);
    w->nt = ceil_div(n, 16);
    if (w->qbytes()) {
        int st = hip_status(hipMalloc(&w->q, w->qbytes()));
        if (st == GPHQ_OK) st = hip_status(hipMemset(w->q, 0, w->qbytes()));
        if (st != GPHQ_OK) {
            (void)hipFree(w->q);
            delete w;
            return st;
        }
    }
    if (w->nt) {
        int st = hip_status(hipMalloc(&w->scales, (size_t)w->nt * 16 * sizeof(float)));
        if (st == GPHQ_OK) st = hip_status(hipMemset(w->scales, 0, (size_t)w->nt * 16 * sizeof(float)));
        if (st != GPHQ_OK) {
            (void)hipFree(w->q);
            (void)hipFree(w->scales);
            delete w;
            return st;
        }
    }
    *out = w;
    return GPHQ_OK;
}

void gphq_q8gemm_weights_i8_free(gphq_weights_i8 *w) {
    if (!w) return;
    (void)hipFree(w->q);
    (void)hipFree(w->scales);
    delete w;
}

int gphq_q8gemm_weights_i8_pack_rows(gphq_weights_i8 *w, const int8_t *q, int64_t q_len, const float *scales,
                                     int64_t rows, int64_t row0) {
    // int8.go:46-63 PackRows: rows = len(scales).
    if (!w || rows < 0 || q_len != w->k * rows || row0 < 0 || row0 + rows > w->n) return GPHQ_ERR_DIMENSIONS;
    if (rows && !scales) return GPHQ_ERR_DIMENSIONS;
    for (int64_t i = 0; i < rows; ++i)
        if (std::isnan(scales[i]) || std::isinf(scales[i])) return GPHQ_ERR_NON_FINITE;
    if (rows == 0) return GPHQ_OK;
    GPHQ_TRY(hip_status(hipMemcpy(w->scales + row0, scales, (size_t)rows * sizeof(float), hipMemcpyHostToDevice)));
    if (w->k == 0) return GPHQ_OK;
    if (!q) return GPHQ_ERR_DIMENSIONS;
    int8_t *staging = nullptr;
    GPHQ_TRY(hip_status(hipMalloc(&staging, (size_t)q_len)));
    int st = hip_status(hipMemcpy(staging, q, (size_t)q_len, hipMemcpyHostToDevice));
    if (st == GPHQ_OK) st = i8_pack_tiles(staging, w->q, (int)rows, (int)w->k, (int)row0, (int)w->kt, nullptr);
    if (st == GPHQ_OK) st = hip_status(hipStreamSynchronize(nullptr));
    (void)hipFree(staging);
    return st;
}

int gphq_q8gemm_weights_i8_pack(gphq_weights_i8 *w, const int8_t *q, int64_t q_len, const float *scales,
                                int64_t scales_len) {
    // int8.go:35-41 Pack: length checks, clear, then PackRows from row 0.
    if (!w || q_len != w->k * w->n || scales_len != w->n) return GPHQ_ERR_DIMENSIONS;
    if (w->qbytes()) GPHQ_TRY(hip_status(hipMemset(w->q, 0, w->qbytes())));
    return gphq_q8gemm_weights_i8_pack_rows(w, q, q_len, scales, scales_len, 0);
}

int gphq_q8gemm_weights_i8_dims(const gphq_weights_i8 *w, int64_t *k, int64_t *n) {
    if (k) *k = w ? w->k : 0;
    if (n) *n = w ? w->n : 0;
    return GPHQ_OK;
}

int64_t gphq_q8gemm_weights_i8_panels(const gphq_weights_i8 *w) { return w ? ceil_div(w->n, kOutputPanel) : 0; }

int64_t gphq_q8gemm_weights_i8_strips(const gphq_weights_i8 *w) { return w ? ceil_div(w->n, kStripColumns) : 0; }

int64_t gphq_q8gemm_weights_i8_bytes(const gphq_weights_i8 *w) {
    return w ? (int64_t)w->qbytes() + 4 * w->n : 0;
}

int gphq_q8gemm_new_workspace_i8(int64_t k, int64_t max_rows, gphq_workspace_i8 **out) {
    // int8.go:91-97 NewWorkspaceI8, with a row capacity instead of the fixed
    // 16-row tile (the device kernels take any M).
    if (!out) return GPHQ_ERR_DIMENSIONS;
    *out = nullptr;
    if (k < 0 || max_rows < 0 || k > INT32_MAX - 64 || max_rows > INT32_MAX - 16) return GPHQ_ERR_DIMENSIONS;
    auto *ws = new (std::nothrow) gphq_workspace_i8();
    if (!ws) return GPHQ_ERR_DIMENSIONS;
    ws->kcap = k;
    ws->rowcap = max_rows;
    ws->hScale.assign((size_t)max_rows, 0.0f);
    ws->hInv.assign((size_t)max_rows, 0.0f);
    ws->rowDirty.assign((size_t)max_rows, 0);
    const size_t abytes = (size_t)ceil_div(max_rows, 16) * ceil_div(k, 64) * 1024;
    int st = GPHQ_OK;
    if (abytes) {
        st = hip_status(hipMalloc(&ws->act, abytes));
        if (st == GPHQ_OK) st = hip_status(hipMemset(ws->act, 0, abytes));
    }
    if (st == GPHQ_OK && max_rows) {
        st = hip_status(hipMalloc(&ws->rowScale, (size_t)max_rows * sizeof(float)));
        if (st == GPHQ_OK) st = hip_status(hipMalloc(&ws->rowInv, (size_t)max_rows * sizeof(float)));
        if (st == GPHQ_OK) st = hip_status(hipMemset(ws->rowScale, 0, (size_t)max_rows * sizeof(float)));
        if (st == GPHQ_OK) st = hip_status(hipMemset(ws->rowInv, 0, (size_t)max_rows * sizeof(float)));
    }
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

void gphq_q8gemm_workspace_i8_free(gphq_workspace_i8 *ws) {
    if (!ws) return;
    (void)hipFree(ws->act);
    (void)hipFree(ws->rowScale);
    (void)hipFree(ws->rowInv);
    delete ws;
}

int gphq_q8gemm_workspace_i8_prepare(gphq_workspace_i8 *ws, int64_t rows, int64_t k) {
    // int8.go:100-108 Prepare: records the shape and clears the row scales.
    if (!ws || rows < 0 || rows > ws->rowcap || k < 0 || k > ws->kcap) return GPHQ_ERR_DIMENSIONS;
    ws->k = k;
    ws->rows = rows;
    ws->kt = ceil_div(k, 64);
    std::fill(ws->hScale.begin(), ws->hScale.end(), 0.0f);
    std::fill(ws->hInv.begin(), ws->hInv.end(), 0.0f);
    std::fill(ws->rowDirty.begin(), ws->rowDirty.begin() + rows, (uint8_t)1);
    ws->dirty = true;
    return GPHQ_OK;
}

int gphq_q8gemm_workspace_i8_set_row_scale(gphq_workspace_i8 *ws, int64_t row, float max_abs) {
    // int8.go:106-112 SetRowScale.
    if (!ws || row < 0 || row >= ws->rows) return GPHQ_ERR_DIMENSIONS;
    if (max_abs > 0 && !std::isinf(max_abs) && max_abs == max_abs) {
        ws->hScale[(size_t)row] = max_abs / 127.0f;
        ws->hInv[(size_t)row] = 127.0f / max_abs;
    } else {
        ws->hScale[(size_t)row] = 0.0f;
        ws->hInv[(size_t)row] = 0.0f;
    }
    ws->rowDirty[(size_t)row] = 1;
    ws->dirty = true;
    return GPHQ_OK;
}

int gphq_q8gemm_workspace_i8_pack_range(gphq_workspace_i8 *ws, const float *x, int64_t x_len, int64_t stride,
                                        int64_t k0, int64_t k1, void *stream) {
    // int8.go:116-163 PackRange.
    if (!ws || k0 < 0 || k1 > ws->k || k0 > k1 || k0 % 4 != 0 || (k1 % 4 != 0 && k1 != ws->k) || stride < ws->k ||
        (ws->rows > 0 && x_len < (ws->rows - 1) * stride + ws->k))
        return GPHQ_ERR_DIMENSIONS;
    if (ws->rows == 0) return GPHQ_OK;
    hipStream_t s = (hipStream_t)stream;
    if (ws->dirty) {
        // Upload each run of consecutive dirty rows; rows whose scales the
        // device computed (the fused Pack) keep them.
        for (int64_t r = 0; r < ws->rows;) {
            if (!ws->rowDirty[(size_t)r]) {
                ++r;
                continue;
            }
            int64_t e = r;
            while (e < ws->rows && ws->rowDirty[(size_t)e]) ws->rowDirty[(size_t)e++] = 0;
            GPHQ_TRY(hip_status(hipMemcpyAsync(ws->rowScale + r, ws->hScale.data() + r, (size_t)(e - r) * sizeof(float),
                                               hipMemcpyHostToDevice, s)));
            GPHQ_TRY(hip_status(hipMemcpyAsync(ws->rowInv + r, ws->hInv.data() + r, (size_t)(e - r) * sizeof(float),
                                               hipMemcpyHostToDevice, s)));
            r = e;
        }
        // The host arrays may change right after this call returns.
        GPHQ_TRY(hip_status(hipStreamSynchronize(s)));
        ws->dirty = false;
    }
    if (ws->k == 0) return GPHQ_OK;
    if (!x) return GPHQ_ERR_DIMENSIONS;
    return i8_pack_range(x, (long)stride, (int)ws->rows, (int)ws->k, (int)ws->kt, (int)k0, (int)k1, ws->act, ws->rowInv,
                         s);
}

int gphq_q8gemm_workspace_i8_pack(gphq_workspace_i8 *ws, const float *x, int64_t x_len, int64_t rows, int64_t k,
                                  int64_t stride, void *stream) {
    // Prepare(rows, k); SetRowScale(r, MaxAbs(row r)) for every row;
    // PackRange(x, stride, 0, k) (int8_test.go:32-43) -- fused on the device.
    GPHQ_TRY(gphq_q8gemm_workspace_i8_prepare(ws, rows, k));
    if (stride < k || (rows > 0 && x_len < (rows - 1) * stride + k)) return GPHQ_ERR_DIMENSIONS;
    std::fill(ws->rowDirty.begin(), ws->rowDirty.end(), (uint8_t)0);
    ws->dirty = false;
    if (rows == 0) return GPHQ_OK;
    if (k > 0 && !x) return GPHQ_ERR_DIMENSIONS;
    if (k == 0) {
        // MaxAbs of an empty row is 0: both scales are 0.
        GPHQ_TRY(fill_f32(ws->rowScale, (size_t)rows, 0.0f, (hipStream_t)stream));
        return fill_f32(ws->rowInv, (size_t)rows, 0.0f, (hipStream_t)stream);
    }
    return i8_pack_rows(x, (long)stride, (int)rows, (int)k, (int)ws->kt, ws->act, ws->rowScale, ws->rowInv,
                        (hipStream_t)stream);
}

int gphq_q8gemm_workspace_i8_row_scales(const gphq_workspace_i8 *ws, float *scale_dev, float *inverse_dev,
                                        void *stream) {
    // Copies the prepared rows' scales (s = max/127) and inverses out, for
    // inspection (WorkspaceI8.rowScale / rowInverse).
    if (!ws) return GPHQ_ERR_DIMENSIONS;
    if (ws->rows == 0) return GPHQ_OK;
    hipStream_t s = (hipStream_t)stream;
    if (scale_dev)
        GPHQ_TRY(hip_status(hipMemcpyAsync(scale_dev, ws->rowScale, (size_t)ws->rows * 4, hipMemcpyDeviceToDevice, s)));
    if (inverse_dev)
        GPHQ_TRY(hip_status(hipMemcpyAsync(inverse_dev, ws->rowInv, (size_t)ws->rows * 4, hipMemcpyDeviceToDevice, s)));
    return GPHQ_OK;
}

static int mul_columns_i8(float *dst, int64_t dst_len, int64_t stride, const gphq_workspace_i8 *ws,
                          const gphq_weights_i8 *w, int64_t c0, int64_t c1, hipStream_t s) {
    if (ws->rows == 0 || c0 >= c1) return GPHQ_OK;
    if (dst_len < (ws->rows - 1) * stride + w->n) return GPHQ_ERR_DIMENSIONS;
    if (!dst) return GPHQ_ERR_DIMENSIONS;
    if (w->k == 0) return fill_zero_columns(dst, (long)stride, (int)ws->rows, (int)c0, (int)c1, s);
    return i8gemm_launch(ws->act, w->q, ws->rowScale, w->scales, dst, (long)stride, (int)ws->rows, (int)w->n,
                         (int)w->kt, (int)c0, (int)c1, s);
}

int gphq_q8gemm_mul_panels_i8(float *dst, int64_t dst_len, int64_t stride, const gphq_workspace_i8 *ws,
                              const gphq_weights_i8 *w, int64_t p0, int64_t p1, void *stream) {
    // int8.go:174-197 MulPanelsI8.
    if (!w || !ws || ws->k != w->k || p0 < 0 || p1 > ceil_div(w->n, kOutputPanel) || p0 > p1 || stride < w->n)
        return GPHQ_ERR_DIMENSIONS;
    if (ws->rows == 0 || p0 == p1) return GPHQ_OK;
    const int64_t c1 = std::min(p1 * kOutputPanel, w->n);
    return mul_columns_i8(dst, dst_len, stride, ws, w, p0 * kOutputPanel, c1, (hipStream_t)stream);
}

int gphq_q8gemm_mul_strips_i8(float *dst, int64_t dst_len, int64_t stride, const gphq_workspace_i8 *ws,
                              const gphq_weights_i8 *w, int64_t s0, int64_t s1, void *stream) {
    // int8.go:224-241 MulStripsI8.
    if (!w || !ws || ws->k != w->k || s0 < 0 || s1 > ceil_div(w->n, kStripColumns) || s0 > s1 || stride < w->n)
        return GPHQ_ERR_DIMENSIONS;
    if (ws->rows == 0 || s0 == s1) return GPHQ_OK;
    const int64_t c1 = std::min(s1 * kStripColumns, w->n);
    return mul_columns_i8(dst, dst_len, stride, ws, w, s0 * kStripColumns, c1, (hipStream_t)stream);
}

}  // extern "C"
