// extern "C" entry points of libgphq: argument validation in the reference's
// order, then dispatch to the kernels. Declarations and reference citations
// are in include/gphq.h.
#include "common.h"

namespace gphq {
int gemv_launch(int fmt, const void *codes, const void *scales, const float *x, float *y, int K, int N,
                hipStream_t stream);
int gemv_batch_launch(int fmt, const void *const *codes, const void *const *scales, const float *const *x,
                      float *const *y, int count, int K, int N, hipStream_t stream);
size_t gemv_vec_workspace_bytes(int V, int K);
int gemv_vec_launch(int fmt, const void *codes, const void *scales, const float *x, long xstride, float *y,
                    long ystride, int V, int K, int N, void *work, hipStream_t stream);

static thread_local int g_last_hip_error = 0;
void set_hip_error(hipError_t e) { g_last_hip_error = (int)e; }
}  // namespace gphq

using namespace gphq;

extern "C" {

const char *gphq_error_string(int status) {
    switch (status) {
    case GPHQ_OK:
        return "";
    case GPHQ_ERR_INVALID_DIMENSIONS:
        return "q8gemv: invalid dimensions";
    case GPHQ_ERR_INVALID_WEIGHT_LENGTH:
        return "q8gemv: invalid weight length";
    case GPHQ_ERR_DIMENSIONS:
        return "q8gemm: invalid dimensions or buffer length";
    case GPHQ_ERR_NON_FINITE:
        return "q8gemm: non-finite row scale";
    case GPHQ_ERR_HIP:
        return "gphq: HIP runtime error";
    case GPHQ_ERR_UNSUPPORTED:
        return "gphq: unsupported format or mode";
    case GPHQ_ERR_GEOMETRY:
        return "qwen3: the GPU backend needs 128-wide heads, at most 8 query heads per key/value head, and 64-aligned "
               "widths";
    case GPHQ_ERR_FOREIGN_WORKSPACE:
        return "qwen3: nil, closed, or foreign decode batch workspace";
    case GPHQ_ERR_BATCH_SHAPE:
        return "qwen3: decode batch has mismatched prefixes, tokens, hidden rows, logits rows, and next tokens";
    case GPHQ_ERR_LANE_CAPACITY:
        return "qwen3: decode batch lanes outside the workspace capacity";
    case GPHQ_ERR_FOREIGN_PREFIX:
        return "qwen3: decode prefix is nil, closed, or belongs to another evaluator";
    case GPHQ_ERR_DUPLICATE_PREFIX:
        return "qwen3: decode prefix is duplicated";
    case GPHQ_ERR_PREFIX_FULL:
        return "qwen3: decode prefix has no room for another token";
    case GPHQ_ERR_TOKEN_RANGE:
        return "qwen3: token in decode lane is outside vocabulary";
    case GPHQ_ERR_OVERLAP:
        return "qwen3: decode batch destinations overlap inputs";
    case GPHQ_ERR_NON_FINITE_HIDDEN:
        return "qwen3: non-finite batched hidden state";
    case GPHQ_ERR_MODEL_INCOMPLETE:
        return "qwen3: batched token decode requires a loaded language-model head; call LoadHead first";
    case GPHQ_ERR_WORKSPACE:
        return "qwen3: nil or foreign workspace";
    case GPHQ_ERR_KEEP_RANGE:
        return "qwen3: keep outside the stored tokens";
    case GPHQ_ERR_PREFIX_CAPACITY:
        return "qwen3: tokens exceed prefix capacity";
    case GPHQ_ERR_EMPTY_SEQUENCE:
        return "qwen3: empty token sequence";
    case GPHQ_ERR_CONTEXT:
        return "qwen3: tokens exceed the Qwen3 context";
    case GPHQ_ERR_DEST_WIDTH:
        return "qwen3: destination width does not match the hidden size";
    case GPHQ_ERR_TOKEN_VOCAB:
        return "qwen3: token is outside vocabulary";
    case GPHQ_ERR_NON_FINITE_STATE:
        return "qwen3: non-finite hidden state";
    case GPHQ_ERR_NOT_POSITIVE_DEFINITE:
        return "qwen3: GPTQ Hessian is not positive definite";
    case GPHQ_ERR_SEQUENCE_COUNT:
        return "qwen3: destinations do not match sequences";
    case GPHQ_ERR_PASS_ROWS:
        return "qwen3: sequence exceeds the GPU context";
    case GPHQ_ERR_LOGITS_SHAPE:
        return "qwen3: logits of the given values do not fill whole states and vocabulary rows";
    case GPHQ_ERR_SCRATCH_LIMIT:
        return "gphq: the call needs more scratch than the library's static array holds";
    case GPHQ_ERR_TAIL_SHAPE:
        return "qwen3: tail values do not fill whole states, or exceed the tokens or maxTail";
    case GPHQ_ERR_REUSE:
        return "qwen3: cannot reuse the rows at this anchor";
    case GPHQ_ERR_EMBED_ROWS:
        return "qwen3: embedding values do not fill one row per placeholder";
    case GPHQ_ERR_IO:
        return "gphq: file I/O failed";
    case GPHQ_ERR_FORMAT:
        return "safetensors: invalid file or index";
    case GPHQ_ERR_TENSOR_MISSING:
        return "safetensors: checkpoint is missing the tensor";
    case GPHQ_ERR_TENSOR_SHAPE:
        return "safetensors: tensor has another shape";
    case GPHQ_ERR_TENSOR_DTYPE:
        return "safetensors: tensor has another dtype or size";
    case GPHQ_ERR_TENSOR_NON_FINITE:
        return "safetensors: tensor has a non-finite value";
    case GPHQ_ERR_READ_RANGE:
        return "read outside the tensor";
    case GPHQ_ERR_GPTQ_WIDTH:
        return "qwen3: GPTQ needs projection widths that are multiples of 4096";
    case GPHQ_ERR_CALIBRATION_EMPTY:
        return "qwen3: empty calibration set";
    case GPHQ_ERR_CALIBRATION_SHAPE:
        return "qwen3: calibration sequences take 1 to 256 tokens each and 4096 in all";
    }
    return "gphq: unknown status";
}

int gphq_last_hip_error(void) { return g_last_hip_error; }

const char *gphq_version(void) { return "0.1.0"; }

int gphq_q8gemv_mul_into(const float *x, int64_t x_len, const int8_t *q, int64_t q_len, const float *scales,
                         int64_t scales_len, float *dst, int64_t dst_len, int64_t k, int64_t n, void *stream) {
    // q8gemv/q8gemv.go:19-28, same checks in the same order.
    if (k < 0 || n < 0 || x_len != k || scales_len != n || dst_len != n) return GPHQ_ERR_INVALID_DIMENSIONS;
    if (k == 0) {
        if (q_len != 0) return GPHQ_ERR_INVALID_WEIGHT_LENGTH;
    } else if (q_len % k != 0 || q_len / k != n) {
        return GPHQ_ERR_INVALID_WEIGHT_LENGTH;
    }
    // Device limits of this implementation (int row and column indices).
    if (k > INT32_MAX || n > INT32_MAX) return GPHQ_ERR_INVALID_DIMENSIONS;
    if (n == 0) return GPHQ_OK;
    if (!x && k) return GPHQ_ERR_INVALID_DIMENSIONS;
    if (!dst || !scales) return GPHQ_ERR_INVALID_DIMENSIONS;
    return gemv_launch(GPHQ_FMT_Q8, q, scales, x, dst, (int)k, (int)n, (hipStream_t)stream);
}

int gphq_gemv(int fmt, const void *codes, const void *scales, const float *x, float *y, int64_t k, int64_t n,
              void *stream) {
    if (fmt != GPHQ_FMT_Q8 && fmt != GPHQ_FMT_Q8B && fmt != GPHQ_FMT_Q8B_F32 && fmt != GPHQ_FMT_Q4)
        return GPHQ_ERR_UNSUPPORTED;
    if (k < 0 || n < 0 || k > INT32_MAX || n > INT32_MAX) return GPHQ_ERR_DIMENSIONS;
    if (fmt != GPHQ_FMT_Q8 && k % 32 != 0) return GPHQ_ERR_DIMENSIONS;
    if (n == 0) return GPHQ_OK;
    if (!y || !scales || (k && (!codes || !x))) return GPHQ_ERR_DIMENSIONS;
    if (fmt != GPHQ_FMT_Q8 && k && ((uintptr_t)codes % 16 != 0 || (uintptr_t)x % 16 != 0))
        return GPHQ_ERR_DIMENSIONS;
    return gemv_launch(fmt, codes, scales, x, y, (int)k, (int)n, (hipStream_t)stream);
}

int64_t gphq_gemv_vec_workspace_bytes(int64_t lanes, int64_t k) {
    if (lanes < 0 || lanes > GPHQ_GEMV_VEC_MAX_LANES || k < 0 || k > INT32_MAX) return GPHQ_ERR_DIMENSIONS;
    return (int64_t)gemv_vec_workspace_bytes((int)lanes, (int)k);
}

int gphq_gemv_vec(int fmt, const void *codes, const void *scales, const float *x, int64_t x_stride, float *y,
                  int64_t y_stride, int64_t lanes, int64_t k, int64_t n, void *work, int64_t work_bytes,
                  void *stream) {
    if (fmt != GPHQ_FMT_Q8 && fmt != GPHQ_FMT_Q8B && fmt != GPHQ_FMT_Q8B_F32 && fmt != GPHQ_FMT_Q4)
        return GPHQ_ERR_UNSUPPORTED;
    if (lanes < 0 || lanes > GPHQ_GEMV_VEC_MAX_LANES || k < 0 || n < 0 || k > INT32_MAX || n > INT32_MAX)
        return GPHQ_ERR_DIMENSIONS;
    if (k % 32 != 0 || x_stride < k || y_stride < n || x_stride % 4 != 0) return GPHQ_ERR_DIMENSIONS;
    if (lanes == 0 || n == 0) return GPHQ_OK;
    if (k && (uintptr_t)x % 16 != 0) return GPHQ_ERR_DIMENSIONS;
    if (work_bytes < gphq_gemv_vec_workspace_bytes(lanes, k)) return GPHQ_ERR_DIMENSIONS;
    if (!y || !scales || !work || (uintptr_t)work % 16 != 0) return GPHQ_ERR_DIMENSIONS;
    if (k && (!codes || !x || (uintptr_t)codes % 16 != 0)) return GPHQ_ERR_DIMENSIONS;
    return gemv_vec_launch(fmt, codes, scales, x, (long)x_stride, y, (long)y_stride, (int)lanes, (int)k, (int)n, work,
                           (hipStream_t)stream);
}

int gphq_gemv_batch(int fmt, const void *const *codes, const void *const *scales, const float *const *x,
                    float *const *y, int count, int64_t k, int64_t n, void *stream) {
    if (fmt != GPHQ_FMT_Q8 && fmt != GPHQ_FMT_Q8B && fmt != GPHQ_FMT_Q8B_F32 && fmt != GPHQ_FMT_Q4)
        return GPHQ_ERR_UNSUPPORTED;
    if (count < 0 || count > GPHQ_GEMV_MAX_BATCH) return GPHQ_ERR_DIMENSIONS;
    if (k < 0 || n < 0 || k > INT32_MAX || n > INT32_MAX) return GPHQ_ERR_DIMENSIONS;
    if (k % (fmt == GPHQ_FMT_Q8 ? 16 : 32) != 0) return GPHQ_ERR_DIMENSIONS;
    if (n == 0 || count == 0) return GPHQ_OK;
    if (!codes || !scales || !x || !y) return GPHQ_ERR_DIMENSIONS;
    for (int i = 0; i < count; ++i) {
        if (!y[i] || !scales[i] || (k && (!codes[i] || !x[i]))) return GPHQ_ERR_DIMENSIONS;
        if (k && ((uintptr_t)codes[i] % 16 != 0 || (uintptr_t)x[i] % 16 != 0)) return GPHQ_ERR_DIMENSIONS;
    }
    return gemv_batch_launch(fmt, codes, scales, x, y, count, (int)k, (int)n, (hipStream_t)stream);
}

}  // extern "C"
