/*
 * gphq.h — C ABI of libgphq, the MI355X (gfx950) implementation of
 * gophonic's quantized matrix-product hot path.
 *
 * Every entry point takes plain pointers and sizes. Pointers named *_dev are
 * device (HBM) addresses; everything is enqueued on `stream` (a hipStream_t,
 * NULL for the default stream) and is complete when the stream reaches it.
 * Entry points validate all arguments before enqueueing anything, and return
 * GPHQ_OK (0) or a negative GPHQ_ERR_* code; gphq_error_string() gives the
 * reference's own message for each code so a binding can raise the same
 * panic or error value.
 *
 * Reference paths cited below are relative to the gophonic source tree.
 */
#ifndef GPHQ_H
#define GPHQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------- */
#define GPHQ_OK 0
/* q8gemv/q8gemv.go:19-21 panic "q8gemv: invalid dimensions" */
#define GPHQ_ERR_INVALID_DIMENSIONS (-1)
/* q8gemv/q8gemv.go:22-28 panic "q8gemv: invalid weight length" */
#define GPHQ_ERR_INVALID_WEIGHT_LENGTH (-2)
/* q8gemm/packed.go:26 ErrDimensions "q8gemm: invalid dimensions or buffer length" */
#define GPHQ_ERR_DIMENSIONS (-3)
/* q8gemm/packed.go:27 ErrNonFinite "q8gemm: non-finite row scale" */
#define GPHQ_ERR_NON_FINITE (-4)
/* a HIP runtime call failed; gphq_last_hip_error() holds its hipError_t */
#define GPHQ_ERR_HIP (-5)
/* the format / mode argument is not one this library implements */
#define GPHQ_ERR_UNSUPPORTED (-6)
/* qwen3lm/gpu_darwin.go:124-126 "qwen3: the GPU backend needs 128-wide heads, at
 * most 8 query heads per key/value head, and 64-aligned widths" (also the
 * readConfig plausibility checks, weights.go:672-680) */
#define GPHQ_ERR_GEOMETRY (-7)
/* decode_batch.go:81-83 "qwen3: nil, closed, or foreign decode batch workspace" */
#define GPHQ_ERR_FOREIGN_WORKSPACE (-8)
/* decode_batch.go:85-89 "qwen3: decode batch has mismatched prefixes, tokens,
 * hidden rows, logits rows, and next tokens" */
#define GPHQ_ERR_BATCH_SHAPE (-9)
/* decode_batch.go:90-92 (and :31-33 at creation) lanes beyond the workspace capacity */
#define GPHQ_ERR_LANE_CAPACITY (-10)
/* decode_batch.go:95-97 "qwen3: decode prefix is nil, closed, or belongs to another evaluator" */
#define GPHQ_ERR_FOREIGN_PREFIX (-11)
/* decode_batch.go:98-102 "qwen3: decode prefix is duplicated" */
#define GPHQ_ERR_DUPLICATE_PREFIX (-12)
/* decode_batch.go:103-105 "qwen3: decode prefix has no room for another token" */
#define GPHQ_ERR_PREFIX_FULL (-13)
/* decode_batch.go:106-108 "qwen3: token in decode lane is outside vocabulary" */
#define GPHQ_ERR_TOKEN_RANGE (-14)
/* decode_batch.go:112-125 "qwen3: decode batch destinations overlap inputs" */
#define GPHQ_ERR_OVERLAP (-15)
/* gpu_darwin.go:1245-1249 "qwen3: non-finite batched hidden state" */
#define GPHQ_ERR_NON_FINITE_HIDDEN (-16)
/* decode_batch.go / gpu_darwin.go:1048-1069: the model has no head (LoadHead)
 * or a layer / the embedding table is not bound */
#define GPHQ_ERR_MODEL_INCOMPLETE (-17)
/* evaluator.go:191-193 "qwen3: nil or foreign workspace" */
#define GPHQ_ERR_WORKSPACE (-18)
/* evaluator.go:185-187 "qwen3: keep outside the stored tokens" */
#define GPHQ_ERR_KEEP_RANGE (-19)
/* evaluator.go:188-190 "qwen3: tokens exceed prefix capacity" */
#define GPHQ_ERR_PREFIX_CAPACITY (-20)
/* evaluator.go:545-547 "qwen3: empty token sequence" */
#define GPHQ_ERR_EMPTY_SEQUENCE (-21)
/* evaluator.go:548-550 "qwen3: tokens exceed the Qwen3 context" */
#define GPHQ_ERR_CONTEXT (-22)
/* evaluator.go:551-553 "qwen3: destination width does not match the hidden size" */
#define GPHQ_ERR_DEST_WIDTH (-23)
/* evaluator.go:554-558 "qwen3: token is outside vocabulary" */
#define GPHQ_ERR_TOKEN_VOCAB (-24)
/* gpu_darwin.go:1636-1638, 1649-1652 "qwen3: non-finite hidden state" */
#define GPHQ_ERR_NON_FINITE_STATE (-25)
/* gptq_linalg.go:81-83 "qwen3: GPTQ Hessian is not positive definite" */
#define GPHQ_ERR_NOT_POSITIVE_DEFINITE (-26)
/* evaluator.go:539-541 "qwen3: destinations do not match sequences" */
#define GPHQ_ERR_SEQUENCE_COUNT (-27)
/* gpu_darwin.go:1494-1496 "qwen3: sequence exceeds the GPU context" (a
 * packed batch's sequence longer than one pass) */
#define GPHQ_ERR_PASS_ROWS (-28)
/* evaluator.go:325-327 "qwen3: logits of %d values into %d, want whole
 * states of %d and %d" */
#define GPHQ_ERR_LOGITS_SHAPE (-29)
/* No reference counterpart: a no-allocation entry point was asked for more
 * scratch than the library's static array holds (gphq_gemv_vec_noalloc). */
#define GPHQ_ERR_SCRATCH_LIMIT (-30)
/* evaluator.go:298-301 "qwen3: %d tail values for %d tokens of width %d" */
#define GPHQ_ERR_TAIL_SHAPE (-31)
/* evaluator.go:194-196 "qwen3: cannot reuse %d rows at anchor %d" */
#define GPHQ_ERR_REUSE (-32)
/* evaluator.go:208-210 "qwen3: %d embedding values for %d placeholders of width %d" */
#define GPHQ_ERR_EMBED_ROWS (-33)
/* File formats (safetensors, GPTQ file, weight cache); gphq_error_detail()
 * holds the reference's formatted message for each. */
#define GPHQ_ERR_IO (-34)              /* open / read / write / rename failed */
#define GPHQ_ERR_FORMAT (-35)          /* safetensors.go:85-127: bad header, index or offsets */
#define GPHQ_ERR_TENSOR_MISSING (-36)  /* safetensors.go:145 "checkpoint is missing %s" */
#define GPHQ_ERR_TENSOR_SHAPE (-37)    /* safetensors.go:151-156 "%s has shape %v, want %v" */
#define GPHQ_ERR_TENSOR_DTYPE (-38)    /* safetensors.go:157-160, 171-173 wrong dtype or size */
#define GPHQ_ERR_TENSOR_NON_FINITE (-39) /* safetensors.go:245-248 "%s has a non-finite value" */
#define GPHQ_ERR_READ_RANGE (-40)      /* safetensors.go:206-208 "read outside the tensor" */
/* GPTQ calibration (qwen3lm/gptq.go). */
#define GPHQ_ERR_GPTQ_WIDTH (-41)        /* gptq.go:211-213 "qwen3: GPTQ needs projection widths that are multiples of 4096" */
#define GPHQ_ERR_CALIBRATION_EMPTY (-42) /* gptq.go:324-326 "qwen3: empty calibration set" */
#define GPHQ_ERR_CALIBRATION_SHAPE (-43) /* a sequence outside 1..256 tokens (gptqMaxSeq) or more than 4096 rows
                                            (gptqMaxRows); the reference's own sequence builder never makes one */

/* The reference message for a status code ("" for GPHQ_OK). Static storage. */
const char *gphq_error_string(int status);
/* The calling thread's formatted message of its last file-format failure
 * (tensor names, shapes), "" after a success. Valid until the thread's next
 * file-format call. */
const char *gphq_error_detail(void);
/* The hipError_t of the most recent GPHQ_ERR_HIP on the calling thread. */
int gphq_last_hip_error(void);
/* Library version, "major.minor.patch". */
const char *gphq_version(void);

/* ---- weight formats of the qwen3lm GPU path ------------------------------
 * qwen3lm/gpu.metal:50-61 (enum Q4 = 4, Q8 = 8, Q8B = 9). All are row-major
 * over output rows [N][K]:
 *   GPHQ_FMT_Q8     int8 codes [N][K], one fp32 scale per row (scales f32[N]);
 *                   qwen3lm/gpu_darwin.go:582-594 quantizeRow, and the
 *                   q8gemv.MulInto contract (q8gemv/q8gemv.go:13-30).
 *   GPHQ_FMT_Q8B    int8 codes [N][K], one FP16 scale per 32 values
 *                   (scales f16[N][K/32]); gpu_darwin.go:599-614.
 *   GPHQ_FMT_Q8B_F32 int8 codes [N][K], one fp32 scale per 32 values
 *                   (scales f32[N][K/32]); the Q8B arithmetic with fp32 block
 *                   scales (the benchmark configuration's layout; it has no
 *                   counterpart format name in the reference).
 *   GPHQ_FMT_Q4     4-bit codes [N][K/2]: per 32 values, 16 bytes with value j
 *                   in the low nibble of byte j and value j+16 in the high
 *                   nibble, both stored plus 8; one FP16 scale per 32 values
 *                   (scales f16[N][K/32]); gpu_darwin.go:616-658 and the
 *                   cmd/qwen3-gptq 4-bit output (qwen3lm/gptq.go:703-766).
 */
#define GPHQ_FMT_Q4 4
#define GPHQ_FMT_Q8 8
#define GPHQ_FMT_Q8B 9
#define GPHQ_FMT_Q8B_F32 10

/* ---- q8gemv ---------------------------------------------------------------
 * Replaces q8gemv.MulInto (q8gemv/q8gemv.go:18-30):
 *   dst[j] = dot(x, float32(q[j*k:(j+1)*k])) * scales[j]
 * The *_len arguments are the Go slice lengths; the same checks as the
 * reference run first, in the same order, returning
 * GPHQ_ERR_INVALID_DIMENSIONS or GPHQ_ERR_INVALID_WEIGHT_LENGTH where it
 * panics. k == 0 is allowed (dst = 0 * scales). Inputs must not overlap dst.
 * fp32 sums are reassociated across the wavefront (the reference's own SIMD
 * kernel also reassociates, q8gemv/q8gemv.go:7-10). No allocation. */
int gphq_q8gemv_mul_into(const float *x_dev, int64_t x_len, const int8_t *q_dev, int64_t q_len,
                         const float *scales_dev, int64_t scales_len, float *dst_dev,
                         int64_t dst_len, int64_t k, int64_t n, void *stream);

/* ---- qwen3lm GEMV family --------------------------------------------------
 * Replaces the store-epilogue GEMV kernels of the Metal backend,
 * gemv<PRO_PLAIN, EPI_STORE, BITS, HEAD> (qwen3lm/gpu.metal:68-162, used as
 * gemv_head and by the projection stream,
 * gpu_projection_stream_darwin_test.go:22-111), dispatched from
 * gpuWorkspace.gemv (qwen3lm/gpu_darwin.go:1386-1404):
 *   y[j] = sum_k dequant(W)[j,k] * x[k]
 * fmt is a GPHQ_FMT_* value. Block formats need k % 32 == 0. Per 16 values
 * (8-bit) or 32 values (4-bit) the partial dot product is scaled once, as in
 * gpu.metal:88-123. Returns GPHQ_ERR_DIMENSIONS on a bad shape. */
int gphq_gemv(int fmt, const void *codes_dev, const void *scales_dev, const float *x_dev,
              float *y_dev, int64_t k, int64_t n, void *stream);

/* Multi-vector GEMV: `lanes` input vectors share one read of the weights,
 * y_dev[v*y_stride + j] = sum_k dequant(W)[j,k] * x_dev[v*x_stride + k].
 * Replaces gemvQ8BVector<V> (qwen3lm/gpu.metal:239-314) with its host side
 * gpuDecodeBatchWorkspace.gemv (gpu_darwin.go:1121-1159); any lanes in
 * 1..GPHQ_GEMV_VEC_MAX_LANES (the reference caps V at 8, decode_batch.go:31-33).
 * Formats Q8, Q8B, Q8B_F32, Q4; k % 32 == 0; x_dev 16-byte aligned and
 * x_stride a multiple of 4. Each 32-value block of each vector is split into
 * FP16 hi+lo parts after an exact power-of-two scaling and multiplied on MFMA
 * (products exact, fp32 sums), so results agree with gphq_gemv to the
 * reference's vector-vs-serial bound (1e-4 abs, 1e-5 rel,
 * gpu_vector_batch_darwin_test.go:218) but not bit for bit. work_dev: scratch
 * of at least gphq_gemv_vec_workspace_bytes(lanes, k) bytes, 16-byte aligned.
 * A NaN or Inf in a vector makes that vector's outputs NaN. */
#define GPHQ_GEMV_VEC_MAX_LANES 32
int64_t gphq_gemv_vec_workspace_bytes(int64_t lanes, int64_t k);
int gphq_gemv_vec(int fmt, const void *codes_dev, const void *scales_dev, const float *x_dev, int64_t x_stride,
                  float *y_dev, int64_t y_stride, int64_t lanes, int64_t k, int64_t n, void *work_dev,
                  int64_t work_bytes, void *stream);

/* gphq_gemv_vec without a workspace argument, allocating nothing. No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid
 * allocation). Same checks (the workspace ones aside), kernels and results as
 * gphq_gemv_vec, bit for bit; the scratch is a library-owned device array of
 * GPHQ_GEMV_VEC_NOALLOC_BYTES per GPU, held until the process ends, so
 * gphq_gemv_vec_workspace_bytes(lanes, k) must fit it (else
 * GPHQ_ERR_SCRATCH_LIMIT; 32 lanes fit up to k = 16384). The stream must
 * belong to the current device. Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (streams not ordered with each other)
 * race. */
#define GPHQ_GEMV_VEC_NOALLOC_BYTES (4 << 20)
int gphq_gemv_vec_noalloc(int fmt, const void *codes_dev, const void *scales_dev, const float *x_dev,
                          int64_t x_stride, float *y_dev, int64_t y_stride, int64_t lanes, int64_t k, int64_t n,
                          void *stream);

/* Up to GPHQ_GEMV_MAX_BATCH independent GEMVs of one format and one shape in
 * a single launch: y_dev[i] = dequant(codes_dev[i], scales_dev[i]) . x_dev[i].
 * The four arrays are host arrays of device pointers, count entries each.
 * Same arithmetic per GEMV as gphq_gemv. This is the device form of the
 * reference's projection stream, several gemv dispatches encoded into one
 * command buffer (qwen3lm/gpu_projection_stream_darwin_test.go:75-90); one
 * launch amortizes the fixed launch cost over all of them. Q8 here needs
 * k % 16 == 0. Outputs must not overlap each other or any input. */
#define GPHQ_GEMV_MAX_BATCH 32
int gphq_gemv_batch(int fmt, const void *const *codes_dev, const void *const *scales_dev,
                    const float *const *x_dev, float *const *y_dev, int count, int64_t k, int64_t n,
                    void *stream);

/* ---- q8gemm: int8 x int8 with exact int32 accumulation ---------------------
 * Replaces q8gemm.WeightsI8 / WorkspaceI8 / MulPanelsI8 / MulStripsI8
 * (q8gemm/int8.go:13-253). Results are bit-identical to the reference's
 * scalarMulPanelsI8 oracle (int8.go:199-211):
 *   dst[r*stride + c] = float32(sum_k qa[r,k]*qw[c,k]) * scales[c] * rowScale[r]
 * for any split of the columns into panels (64) or strips (16).
 * Weights and workspaces live in device memory in a tile layout of this
 * library's own ([16 rows][64 K] fragments); Pack takes the reference's
 * row-major input. A workspace holds up to max_rows activation rows (the
 * reference tile is fixed at 16 rows, ActivationRows, packed.go:19; a binding
 * maps its tiles onto one prepared workspace). Handles may be used from any
 * thread; calls on one workspace must not overlap (the reference's Prepare /
 * PackRange contract, int8.go:80-83). */
typedef struct gphq_weights_i8 gphq_weights_i8;
typedef struct gphq_workspace_i8 gphq_workspace_i8;

/* NewWeightsI8 (int8.go:20-32): zeroed device storage for an n x k matrix. */
int gphq_q8gemm_new_weights_i8(int64_t k, int64_t n, gphq_weights_i8 **out);
void gphq_q8gemm_weights_i8_free(gphq_weights_i8 *w);
/* (*WeightsI8).Pack (int8.go:35-41): q_host row-major int8 [n][k], scales_host
 * f32[n]; GPHQ_ERR_DIMENSIONS on a length mismatch, GPHQ_ERR_NON_FINITE on a
 * NaN/Inf scale. Synchronous (one-time model setup). */
int gphq_q8gemm_weights_i8_pack(gphq_weights_i8 *w, const int8_t *q_host, int64_t q_len,
                                const float *scales_host, int64_t scales_len);
/* (*WeightsI8).PackRows (int8.go:43-63): rows [row0, row0+rows) of freshly
 * allocated weights; q_len must be k*rows. */
int gphq_q8gemm_weights_i8_pack_rows(gphq_weights_i8 *w, const int8_t *q_host, int64_t q_len,
                                     const float *scales_host, int64_t rows, int64_t row0);
/* Dims / Panels / Strips / Bytes (int8.go:65-73, 216). Bytes counts this
 * library's device bytes (codes in the tile layout plus fp32 scales). */
int gphq_q8gemm_weights_i8_dims(const gphq_weights_i8 *w, int64_t *k, int64_t *n);
int64_t gphq_q8gemm_weights_i8_panels(const gphq_weights_i8 *w);
int64_t gphq_q8gemm_weights_i8_strips(const gphq_weights_i8 *w);
int64_t gphq_q8gemm_weights_i8_bytes(const gphq_weights_i8 *w);

/* NewWorkspaceI8 (int8.go:91-97) with a row capacity. */
int gphq_q8gemm_new_workspace_i8(int64_t k, int64_t max_rows, gphq_workspace_i8 **out);
void gphq_q8gemm_workspace_i8_free(gphq_workspace_i8 *ws);
/* (*WorkspaceI8).Prepare (int8.go:100-108): rows <= max_rows, k <= capacity;
 * clears the row scales. */
int gphq_q8gemm_workspace_i8_prepare(gphq_workspace_i8 *ws, int64_t rows, int64_t k);
/* (*WorkspaceI8).SetRowScale (int8.go:106-112): scale = max/127 and
 * inverse = 127/max for finite positive max_abs, else 0 and 0 (host value,
 * uploaded by the next pack_range). */
int gphq_q8gemm_workspace_i8_set_row_scale(gphq_workspace_i8 *ws, int64_t row, float max_abs);
/* (*WorkspaceI8).PackRange (int8.go:116-163): quantizes columns [k0, k1) of
 * the prepared rows of x_dev (rows stride floats apart) with the set row
 * scales: q = saturate_int8(round_half_even(x * inverse)). k0 and k1 must be
 * multiples of 4 unless k1 == k. Waits for its own upload of host-set scales. */
int gphq_q8gemm_workspace_i8_pack_range(gphq_workspace_i8 *ws, const float *x_dev, int64_t x_len,
                                        int64_t stride, int64_t k0, int64_t k1, void *stream);
/* Prepare(rows, k) + SetRowScale(r, MaxAbs(row r)) for every row +
 * PackRange(0, k), computed on the device in one launch (the packI8 sequence
 * of int8_test.go:32-43; MaxAbs as q8gemm/gemm.go:138-150). */
int gphq_q8gemm_workspace_i8_pack(gphq_workspace_i8 *ws, const float *x_dev, int64_t x_len, int64_t rows,
                                  int64_t k, int64_t stride, void *stream);
/* The prepared rows' scale (max/127) and inverse (127/max) arrays, copied to
 * device buffers of at least `rows` floats (either may be NULL). */
int gphq_q8gemm_workspace_i8_row_scales(const gphq_workspace_i8 *ws, float *scale_dev,
                                        float *inverse_dev, void *stream);
/* MulPanelsI8 (int8.go:174-197): columns [p0*64, min(p1*64, n)) of dst_dev;
 * other columns untouched. dst_len must be >= (rows-1)*stride + n. */
int gphq_q8gemm_mul_panels_i8(float *dst_dev, int64_t dst_len, int64_t stride, const gphq_workspace_i8 *ws,
                              const gphq_weights_i8 *w, int64_t p0, int64_t p1, void *stream);
/* MulStripsI8 (int8.go:224-241): columns [s0*16, min(s1*16, n)), bit-identical
 * to the panel form. */
int gphq_q8gemm_mul_strips_i8(float *dst_dev, int64_t dst_len, int64_t stride, const gphq_workspace_i8 *ws,
                              const gphq_weights_i8 *w, int64_t s0, int64_t s1, void *stream);

/* ---- q8gemm: FP16 activations x int8 or FP16 weights -----------------------
 * Replaces q8gemm.Weights / Workspace / MulPanels / MulInto
 * (q8gemm/packed.go:35-239, gemm.go:20-286):
 *   dst[r*stride + c] = (sum_k f16(x[r,k]*rowScale[r]) * w[c,k]) * scales[c] * rowInverse[r]
 * with rowScale = 2^e placing each row's max|x| in [2^14, 2^15)
 * (gemm.go:127-135). Products are exact in fp32; sums are fp32 on MFMA, in an
 * order of the hardware's (the reference's SME kernel also reorders; its
 * bound is 2e-5*sqrt(K) relative, q8gemm_test.go:58). Weights live in device
 * memory in this library's [16 rows][64 K] tile layout. */
typedef struct gphq_weights gphq_weights;
typedef struct gphq_workspace gphq_workspace;

/* NewWeights (packed.go:43-61): int8 storage. */
int gphq_q8gemm_new_weights(int64_t k, int64_t n, gphq_weights **out);
/* NewWeightsF16 (packed.go:63-76): FP16 storage, filled by pack_bf16. */
int gphq_q8gemm_new_weights_f16(int64_t k, int64_t n, gphq_weights **out);
/* WeightsF16Bytes (packed.go:78-93) for this library's device layout; a
 * negative status for invalid dimensions. */
int64_t gphq_q8gemm_weights_f16_bytes(int64_t k, int64_t n);
/* NewWeightsF16Buffer (packed.go:95-121): binds caller-owned zeroed device
 * storage (4-byte aligned, at least weights_f16_bytes). */
int gphq_q8gemm_new_weights_f16_buffer(int64_t k, int64_t n, void *data_dev, int64_t data_len, gphq_weights **out);
/* packed.go:78-93 WeightsF16Bytes as the reference computes it: the size of
 * the reference's own FP16 layout, panels [ceil(n/64)][ceil(k/2)][64][2] then
 * n fp32 row scales (K = 3, N = 65: 1284 bytes). */
int64_t gphq_q8gemm_reference_f16_bytes(int64_t k, int64_t n);
/* Loads FP16 weights from a buffer in the reference's layout -- the bytes a
 * reference NewWeightsF16Buffer + PackBF16[Rows] leave in caller storage,
 * such as a wcache mapping (qwen3lm/weights.go:362-370, packed.go:95-175) --
 * from host memory (ref_len >= gphq_q8gemm_reference_f16_bytes(k, n)) into F16
 * weights w of the same k and n: one upload, then a device repack into this
 * library's tile layout. A non-finite row scale gives GPHQ_ERR_NON_FINITE.
 * One-time setup; synchronizes. */
int gphq_q8gemm_weights_f16_load_reference(gphq_weights *w, const void *ref_host, int64_t ref_len);
void gphq_q8gemm_weights_free(gphq_weights *w);
/* (*Weights).Pack (packed.go:181-204): int8 row-major [n][k] + fp32 scales. */
int gphq_q8gemm_weights_pack(gphq_weights *w, const int8_t *q_host, int64_t q_len, const float *scales_host,
                             int64_t scales_len);
/* (*Weights).PackBF16 / PackBF16Rows (packed.go:123-175): raw BF16 bits,
 * row-major; *rounded receives the count of values FP16 could not hold
 * exactly; GPHQ_ERR_NON_FINITE stops at the first row holding NaN/Inf. */
int gphq_q8gemm_weights_pack_bf16(gphq_weights *w, const uint16_t *bf16_host, int64_t len, int64_t *rounded);
int gphq_q8gemm_weights_pack_bf16_rows(gphq_weights *w, const uint16_t *bf16_host, int64_t len, int64_t row0,
                                       int64_t *rounded);
/* Dims / Panels / Bytes / F16 (packed.go:206-231). */
int gphq_q8gemm_weights_dims(const gphq_weights *w, int64_t *k, int64_t *n);
int64_t gphq_q8gemm_weights_panels(const gphq_weights *w);
int64_t gphq_q8gemm_weights_bytes(const gphq_weights *w);
int gphq_q8gemm_weights_is_f16(const gphq_weights *w);

/* NewWorkspace (gemm.go:58-69) with a row capacity. */
int gphq_q8gemm_new_workspace(int64_t k, int64_t max_rows, gphq_workspace **out);
void gphq_q8gemm_workspace_free(gphq_workspace *ws);
/* Prepare (gemm.go:79-89): row scales reset to 1. */
int gphq_q8gemm_workspace_prepare(gphq_workspace *ws, int64_t rows, int64_t k);
/* PrepareRowF16 / PrepareRowsF16 (gemm.go:91-122) need the reference's SME
 * row kernel; without SME (amd64 included) the reference returns
 * ErrDimensions, and so do these. */
int gphq_q8gemm_workspace_prepare_row_f16(gphq_workspace *ws, int64_t k);
int gphq_q8gemm_workspace_prepare_rows_f16(gphq_workspace *ws, int64_t rows, int64_t k);
/* SetRowScale (gemm.go:124-136). */
int gphq_q8gemm_workspace_set_row_scale(gphq_workspace *ws, int64_t row, float max_abs);
/* PackRange (gemm.go:152-226): columns [k0, k1) (multiples of 2 unless
 * k1 == k) of the prepared rows, f16(x * rowScale). */
int gphq_q8gemm_workspace_pack_range(gphq_workspace *ws, const float *x_dev, int64_t x_len, int64_t stride,
                                     int64_t k0, int64_t k1, void *stream);
/* Pack (gemm.go:71-77): Prepare + SetRowScale(MaxAbs) + PackRange on the
 * device in one launch. */
int gphq_q8gemm_workspace_pack(gphq_workspace *ws, const float *x_dev, int64_t x_len, int64_t rows, int64_t k,
                               int64_t stride, void *stream);
/* The prepared rows' scales and inverses (device buffers, either NULL). */
int gphq_q8gemm_workspace_row_scales(const gphq_workspace *ws, float *scale_dev, float *inverse_dev, void *stream);
/* The packed FP16 activations as row-major [rows][k] bits (inspection;
 * synchronizes the stream). */
int gphq_q8gemm_workspace_activations(const gphq_workspace *ws, uint16_t *act_dev, void *stream);
/* MulPanels (gemm.go:228-272): columns [p0*64, min(p1*64, n)); the portable
 * path's scratch argument has no counterpart. */
int gphq_q8gemm_mul_panels(float *dst_dev, int64_t dst_len, int64_t stride, gphq_workspace *ws,
                           const gphq_weights *w, int64_t p0, int64_t p1, void *stream);
/* MulInto (gemm.go:274-286): pack `rows` rows of x and multiply all panels. */
int gphq_q8gemm_mul_into(float *dst_dev, int64_t dst_len, const float *x_dev, int64_t x_len, int64_t rows,
                         const gphq_weights *w, gphq_workspace *ws, void *stream);

/* ---- qwen3lm batched projection (mm) --------------------------------------
 * Replaces mm<PRO_PLAIN, EPI_STORE, BITS> (qwen3lm/gpu.metal:766-927, run by
 * gpuWorkspace.mmRun, gpu_darwin.go:1665-1699): y[M][N] = x[M][K] . W^T with
 * each K step's weights dequantized to FP16 (Q8: half(code); Q8B:
 * half(code)*half(d); Q4: (half(nib)-8)*d, each rounded to half), activations
 * half(x), fp32 accumulation, and Q8 rows scaled by their fp32 scale after
 * the sum. fmt: GPHQ_FMT_Q8, GPHQ_FMT_Q8B, GPHQ_FMT_Q8B_F32 (half(code) *
 * half(d): the Q8B tile once the scale is rounded to FP16), GPHQ_FMT_Q4, or
 * GPHQ_FMT_GPTQ4_G128: int32 codes [N][K/8] (nibble i of word j holds k = 8j+i,
 * unsigned 0..15), FP16 scales [N][K/128] and zero points zeros_dev
 * u8 [N][K/128] (low nibble), w = (q - z) * s -- the 4-bit group-128
 * zero-point layout of the benchmark configuration (cmd/qwen3-gptq itself
 * emits GPHQ_FMT_Q4). k must be a multiple of 32 (128 for GPTQ4_G128).
 * work_dev is scratch of at least gphq_mm_workspace_bytes(m, k) bytes
 * (16-byte aligned) for the FP16 activations. */
#define GPHQ_FMT_GPTQ4_G128 12
int64_t gphq_mm_workspace_bytes(int64_t m, int64_t k);
/* The workspace with room for split-K partial sums (gpu_darwin.go:1667-1699
 * mmRun: small grids split K and mm_finish adds the splits in order): with at
 * least this many bytes, a product whose grid of 128 x 128 tiles is under 512
 * blocks splits K (while the partial sums stay within 32 MiB); the sums are
 * then added split by split, deterministically. */
int64_t gphq_mm_split_workspace_bytes(int64_t m, int64_t k, int64_t n);
int gphq_mm(int fmt, const void *codes_dev, const void *scales_dev, const uint8_t *zeros_dev, const float *x_dev,
            float *y_dev, int64_t m, int64_t k, int64_t n, void *work_dev, int64_t work_bytes, void *stream);

/* ---- qwen3lm GPU decode provider (the lane API) ----------------------------
 * Replaces the Metal provider's single-token decode: gpuModel
 * (qwen3lm/gpu_darwin.go:62-102, loadGPU 161-338, loadHead 340-373),
 * gpuPrefix (800-893) and gpuDecodeBatchWorkspace (731-759, 1046-1281) behind
 * Evaluator.NewDecodeBatchWorkspace / DecodeBatchInto /
 * DecodeBatchGreedyInto (decode_batch.go:23-78). A step runs wholly on the
 * device: embedding + hidden rotation, per layer QKV (RMSNorm fused) ->
 * attention (head RMSNorm, RoPE, K/V append, softmax over 0..pos) -> O
 * (+ residual) -> gate/up (RMSNorm, SwiGLU) -> [down input Hadamard for Q8/Q4]
 * -> down (+ residual), then final norm, Q8B head and first-maximum argmax.
 * fp32 arithmetic; results agree with the reference's float64 semantics to
 * the reference GPU tests' bounds (gpu_decode_batch_darwin_test.go:121-131),
 * not bit for bit. */
#define GPHQ_DECODE_MAX_LANES 32

/* The model geometry (config.json fields the reference reads, weights.go:
 * 621-700) and the layer weight format (gpuModel.bits: GPHQ_FMT_Q8, Q8B or
 * Q4; GPHQ_FMT_Q8B_F32 is Q8B with fp32 block scales). */
typedef struct gphq_lm_config {
    int64_t hidden, layers, heads, kv_heads, head_dim, intermediate, vocab, max_positions;
    double eps, rope_theta;
    int32_t fmt;
    int32_t reserved;
} gphq_lm_config;

/* One layer (gpuLayer, gpu_darwin.go:45-56): a device buffer holding the
 * quantized projections as prepareGPU writes them (gpu_darwin.go:392-569):
 * fused QKV rows [q_dim + 2 kv_dim][hidden] = W.diag(input_norm).R^T (value
 * rows may carry the per-head Hadamard), O [hidden][q_dim], gate/up rows
 * interleaved [2 inter][hidden] (row 2i gate, 2i+1 up, post-attention norm
 * folded), down [hidden][inter]; each region's codes then scales at the byte
 * offsets given, the buffer 256-byte aligned. q_norm / k_norm: host float[128]
 * (copied at bind). */
typedef struct gphq_lm_layer {
    const void *buf_dev;
    int64_t buf_bytes;
    int64_t qkv, qkv_scale, o, o_scale, gu, gu_scale, d, d_scale;
    const float *q_norm_host, *k_norm_host;
} gphq_lm_layer;

typedef struct gphq_lm gphq_lm;
typedef struct gphq_prefix gphq_prefix;
typedef struct gphq_decode_batch gphq_decode_batch;

/* The reference's per-layer placement (gpu_darwin.go:243-283 place): fills the
 * offsets and buf_bytes of *out (buf_dev and norms untouched). */
int gphq_lm_layer_layout(const gphq_lm_config *cfg, gphq_lm_layer *out, int64_t *bytes);
/* loadHead's buffer (gpu_darwin.go:340-346): rows = vocab padded to 16, Q8B
 * codes [rows][hidden], FP16 scales at scale_offset. */
int gphq_lm_head_layout(const gphq_lm_config *cfg, int64_t *rows, int64_t *scale_offset, int64_t *bytes);
/* gpuGeometry check (gpu_darwin.go:116-129), RoPE table (232-241: float32 of
 * float64 cos/sin, min(max_positions, 65536) rows) and rotation signs
 * (hadamard.go:24-47). Weights are bound afterwards. */
int gphq_lm_new(const gphq_lm_config *cfg, gphq_lm **out);
void gphq_lm_free(gphq_lm *lm);
int gphq_lm_bind_layer(gphq_lm *lm, int64_t layer, const gphq_lm_layer *desc);
/* The embedding table as raw BF16 bits [vocab][hidden] in device memory
 * (Weights.embed, weights.go:614-619), unrotated. */
int gphq_lm_bind_embed(gphq_lm *lm, const uint16_t *embed_dev, int64_t len);
/* The Q8B head W.R^T (loadHead) and the final norm weight (host float[hidden]). */
int gphq_lm_bind_head(gphq_lm *lm, const void *head_dev, int64_t bytes, const float *final_norm_host);

/* gpuPrefix: a lane's private fp32 K/V cache [layers][capacity][kv_dim] each,
 * zeroed. The token count lives with the caller (PrefixKV.tokens), who passes
 * it as the lane's position. */
int gphq_prefix_new(const gphq_lm *lm, int64_t capacity, gphq_prefix **out);
void gphq_prefix_free(gphq_prefix *p);
int gphq_prefix_kv(const gphq_prefix *p, float **kc_dev, float **vc_dev, int64_t *capacity);
/* copyFrom (gpu_darwin.go:873-881): the first n rows of every layer. */
int gphq_prefix_copy(gphq_prefix *dst, const gphq_prefix *src, int64_t n, void *stream);

/* NewDecodeBatchWorkspace (decode_batch.go:27-39; gpu_darwin.go:1046-1108):
 * scratch for 1..GPHQ_DECODE_MAX_LANES lanes (the reference caps at 8). */
int gphq_decode_batch_new(const gphq_lm *lm, int64_t capacity, gphq_decode_batch **out);
void gphq_decode_batch_free(gphq_decode_batch *ws);
/* Lane count from which the step's GEMVs use the multi-vector MFMA kernel
 * (default 2; a larger value keeps the per-lane fp32 GEMV). */
int gphq_decode_batch_set_vec_min_lanes(gphq_decode_batch *ws, int64_t lanes);
/* DecodeBatchInto (decode_batch.go:41-59): lane l at position positions[l]
 * (its prefix's token count) takes host token tokens[l]; writes the lane's
 * post-final-norm hidden state to hidden_dev[l*hidden..] and its logits to
 * logits_dev[l*vocab..], and appends the K/V row. Validation follows
 * decode_batch.go:80-146 in order, before any device work. */
int gphq_decode_batch_into(gphq_decode_batch *ws, gphq_prefix *const *kvs, int64_t lanes, const int64_t *positions,
                           const int32_t *tokens, float *hidden_dev, int64_t hidden_len, float *logits_dev,
                           int64_t logits_len, void *stream);
/* DecodeBatchGreedyInto (decode_batch.go:61-78): as above, but next_dev[l]
 * receives the first-maximum token (greedy_argmax_rows, gpu.metal:192-237)
 * instead of the logits. */
int gphq_decode_batch_greedy_into(gphq_decode_batch *ws, gphq_prefix *const *kvs, int64_t lanes,
                                  const int64_t *positions, const int32_t *tokens, float *hidden_dev,
                                  int64_t hidden_len, int32_t *next_dev, void *stream);
/* `steps` chained greedy steps: step t of lane l consumes the token step t-1
 * chose (tokens[l] first) at position positions[l] + t; tokens_out_dev
 * [steps][lanes] receives every chosen token, hidden_dev (or NULL) the last
 * step's hidden states. The device keeps tokens and positions between
 * steps, so the host enqueues without waiting (the reference's Decoder run,
 * gpu_darwin.go:1913-2006, chains steps in one command buffer the same way). */
int gphq_decode_greedy_run(gphq_decode_batch *ws, gphq_prefix *const *kvs, int64_t lanes, const int64_t *positions,
                           const int32_t *tokens, int64_t steps, int32_t *tokens_out_dev, int64_t tokens_out_len,
                           float *hidden_dev, int64_t hidden_len, void *stream);
/* Whether gphq_decode_greedy_run replays one captured step as a HIP graph
 * (default 1) or launches each step's kernels (0). The graph is captured on
 * the workspace's own stream at the first run and kept while the lane
 * prefixes, hidden_dev and tokens_out_dev stay the same; it is launched on
 * the caller's stream. */
int gphq_decode_batch_set_graph(gphq_decode_batch *ws, int on);
/* Teacher-forced extension of each lane's prefix by tokens [steps][lanes]
 * (the one-token-at-a-time pass of encodeTokens, gpu_darwin.go:1768-1814):
 * appends K/V rows; no head. */
int gphq_decode_extend(gphq_decode_batch *ws, gphq_prefix *const *kvs, int64_t lanes, const int64_t *positions,
                       const int32_t *tokens, int64_t steps, void *stream);
/* Evaluator.LogitsRowsInto / LogitsInto on the GPU (evaluator.go:313-370;
 * gpuWorkspace.logitsRowsInto / logitsInto, gpu_darwin.go:1510-1572): the
 * head's logits of k = hidden_len / hidden post-final-norm states (device
 * [k][hidden], e.g. earlier hidden_dev results) into logits_dev [k][vocab].
 * Each state is rotated into the head's basis (hidden.apply) and multiplied by
 * the Q8B head; a chunk of L <= capacity rows takes the same GEMV a decode step
 * of L lanes takes, so the logits of a step's hidden states equal that step's
 * logits bit for bit. GPHQ_ERR_LOGITS_SHAPE unless 1 <= k <=
 * GPHQ_LOGITS_MAX_ROWS (the reference's maxTail) with whole rows on both
 * sides. Stream-ordered; the workspace's scratch is reused. */
#define GPHQ_LOGITS_MAX_ROWS 256
int gphq_decode_batch_logits(gphq_decode_batch *ws, const float *hidden_dev, int64_t hidden_len, float *logits_dev,
                             int64_t logits_len, void *stream);
/* Waits for the stream and reports GPHQ_ERR_NON_FINITE_HIDDEN if a step since
 * the last check produced a non-finite hidden value (the reference's error,
 * gpu_darwin.go:1245-1249, which it raises before returning). */
int gphq_decode_batch_check(gphq_decode_batch *ws, void *stream);

/* ---- weight preparation (prepareGPU's jobs) ---------------------------------
 * Replaces the body of one gpuJob of qwen3lm's prepareGPU
 * (qwen3lm/gpu_darwin.go:375-391, 511-567): BF16 rows [n][k] -> float32 ->
 * times the folded RMSNorm weight -> input rotation R.row -> output rotation
 * along the rows -> quantization into the layer buffer (Q8 quantizeRow, Q8B
 * quantizeRowQ8B, Q4 quantizeRowQ4; gpu_darwin.go:582-658), every step in the
 * reference's float32 operation order, so codes and scales are bit-identical
 * to the host path's. GPHQ_FMT_Q8B_F32 stores the Q8B codes of d = max/127
 * with fp32 scales (no counterpart in the reference).
 * A rotation is newRotation(width) (hadamard.go:24-47), or with tile > 0 the
 * signs of newRotation(tile) repeated every tile values (the per-head
 * rotation of value rows and o inputs, gpu_darwin.go:217-221); {0, 0} is
 * none. The input rotation spans k, the output rotation n (n a multiple of
 * its block). Source row r is written to destination row row0 + r*step
 * (gate/up interleave: step 2, row0 0 or 1), codes at byte offset base and
 * scales at sc of dst_dev (dst_bytes long). One-time setup: the call waits
 * for its stream. */
typedef struct gphq_rotation_spec {
    int64_t width, tile;
} gphq_rotation_spec;

typedef struct gphq_prepare_job {
    const uint16_t *src_bf16_dev; /* [n][k] BF16 bits */
    int64_t n, k;
    const float *norm_host;       /* k weights folded into every row, or NULL */
    gphq_rotation_spec in_rot, out_rot;
    int32_t fmt;
    int32_t reserved;
    void *dst_dev;
    int64_t dst_bytes;
    int64_t base, sc, step, row0;
    float scale_mul;
} gphq_prepare_job;

/* Scratch for gphq_prepare_projection: float32 rows plus tables (n*k*4 + ...). */
int64_t gphq_prepare_work_bytes(int64_t n, int64_t k);
int gphq_prepare_projection(const gphq_prepare_job *job, void *work_dev, int64_t work_bytes, void *stream);

/* prepareGPU's job list for a dense Qwen3 model (gpu_darwin.go:392-437), so a
 * loader (loadGPU, gpu_darwin.go:161-338) need not restate it. A layer's jobs,
 * in the reference's order: q, k, v (input norm folded, hidden input
 * rotation, v's rows also per-head rotated), o (per-head input, hidden output
 * rotation), gate, up (post-attention norm folded, interleaved rows: step 2,
 * row0 0 / 1), down (the intermediate input rotation except for Q8B, hidden
 * output rotation), at the offsets of gphq_lm_layer_layout in one layer
 * buffer, in cfg->fmt. gphq_prepare_layer_jobs fills jobs[7] (src_bf16_dev
 * left NULL; the norms are float32 host arrays of hidden values, the
 * checkpoint's BF16 widened); gphq_prepare_layer runs them from the seven
 * BF16 projections src_bf16_dev[7] (device, [n][k] each: q_proj, k_proj,
 * v_proj, o_proj, gate_proj, up_proj, down_proj). The head (lm_head, or the
 * tied embedding) is read in chunks of gphq_prepare_head_chunk_rows rows
 * (max(intermediate, 4096)) over hidden-rotated rows into the Q8B buffer of
 * gphq_lm_head_layout: gphq_prepare_head_job describes the chunk starting at
 * vocabulary row row0, gphq_prepare_head runs them all from src_bf16_dev
 * [vocab][hidden]. gphq_prepare_lm_work_bytes is the scratch every job of the
 * model fits in. Each run waits for its stream (one-time setup). */
#define GPHQ_LAYER_PROJECTIONS 7
int gphq_prepare_layer_jobs(const gphq_lm_config *cfg, const float *input_norm_host, const float *post_norm_host,
                            void *dst_dev, int64_t dst_bytes, gphq_prepare_job *jobs);
int64_t gphq_prepare_head_chunk_rows(const gphq_lm_config *cfg);
int gphq_prepare_head_job(const gphq_lm_config *cfg, int64_t row0, void *dst_dev, int64_t dst_bytes,
                          gphq_prepare_job *job);
int64_t gphq_prepare_lm_work_bytes(const gphq_lm_config *cfg);
int gphq_prepare_layer(const gphq_lm_config *cfg, const uint16_t *const *src_bf16_dev, const float *input_norm_host,
                       const float *post_norm_host, void *dst_dev, int64_t dst_bytes, void *work_dev,
                       int64_t work_bytes, void *stream);
int gphq_prepare_head(const gphq_lm_config *cfg, const uint16_t *src_bf16_dev, void *dst_dev, int64_t dst_bytes,
                      void *work_dev, int64_t work_bytes, void *stream);

/* ---- qwen3lm batched pass (prefill) ----------------------------------------
 * Replaces the GPU path of Evaluator.HiddenLastExtendInto (evaluator.go:
 * 146-262): gpuWorkspace.batchPacked with an unshared prefix, pass and
 * encodeBatch (gpu_darwin.go:1449-1480, 1574-1657, 1703-1764). Per pass of up
 * to `rows` tokens and per layer: QKV projection over RMS-normalized rows,
 * qkRope (head norm, RoPE, K/V append), causal attention (attendFlash),
 * O projection + residual, gate/up with norm and SwiGLU, the down input's
 * Hadamard (Q8/Q4) and down + residual; projections use FP16 weight and
 * activation tiles with fp32 sums (the reference mm's arithmetic), attention
 * FP16 MFMA tiles with fp32 sums and softmax. A one-token pass uses the fp32
 * GEMV (encodeTokens, gpu_darwin.go:1605-1614). Results agree with the
 * token-by-token path to the reference's bound (cosine >= 0.99999,
 * gpu_official_darwin_test.go:86), not bit for bit. */
#define GPHQ_PREFILL_MAX_ROWS 65536
typedef struct gphq_prefill gphq_prefill;

/* The batched part of NewWorkspace (newWorkspace, gpu_darwin.go:895-960): device
 * scratch for passes of up to `rows` tokens (the reference fixes 2048). */
int gphq_prefill_new(const gphq_lm *lm, int64_t rows, gphq_prefill **out);
void gphq_prefill_free(gphq_prefill *ws);
int gphq_prefill_rows(const gphq_prefill *ws);
/* HiddenLastExtendInto: evaluates tokens[0..n) (host array) as the
 * continuation of the first `keep` cache rows of kv, writing K/V rows
 * keep..keep+n-1, in passes of at most the workspace's rows; hidden_dev
 * (hidden_len == hidden floats) receives the last token's post-final-norm
 * state. The caller keeps the token count (keep + n afterwards). Validation
 * follows evaluator.go:178-194, 540-560 in order, before any device work.
 * Enqueued on `stream`; gphq_prefill_check waits and reports a non-finite
 * hidden state. */
int gphq_prefill_extend(gphq_prefill *ws, gphq_prefix *kv, int64_t keep, const int32_t *tokens, int64_t n,
                        float *hidden_dev, int64_t hidden_len, void *stream);
/* Embeds (evaluator.go:150-163): the i-th occurrence of `token` among a
 * call's tokens takes row i of rows_dev (device, rows_len = occurrences x
 * hidden fp32 values, unrotated like an embedding-table row) instead of the
 * embedding row. rows_len == 0 replaces nothing. */
typedef struct gphq_embeds {
    int32_t token;
    int32_t reserved;
    const float *rows_dev;
    int64_t rows_len;
} gphq_embeds;
/* evaluator.go:283-285 maxTail: states one tail call returns, at most. */
#define GPHQ_TAIL_MAX_ROWS 256
/* HiddenTailContinueEmbedInto (evaluator.go:293-310) and, with a one-row
 * tail, HiddenLastContinueEmbedInto / HiddenLastExtendEmbedInto
 * (evaluator.go:164-262); the provider seam is gpuWorkspace.batch with
 * Embeds (gpu_darwin.go:1412-1480, pass 1574-1657). tokens[0..n) (host)
 * continue the first `keep` of the `stored` tokens the caller records for
 * kv (PrefixKV.tokens stays on the caller's side); placeholder tokens of
 * `embeds` (may be NULL) take its rows. tail_dev receives the
 * post-final-norm states of the last tail_len / hidden positions, in order
 * (1 <= that count <= GPHQ_TAIL_MAX_ROWS and <= n); passes hold at most the
 * workspace's rows and the last pass holds the whole tail. `reuse` leading
 * rows may be declared unchanged (the reuse contract, checked as the
 * reference checks it); like the reference's GPU path every row is
 * recomputed, so the result does not depend on it. Afterwards the caller
 * records tokens[:keep] followed by the ids, each placeholder as -1.
 * Validation (evaluator.go:295-301, 182-213, 540-560) in order, before any
 * device work; returns once the host arrays are consumed (the stream is
 * synchronized). gphq_prefill_check reports a non-finite tail state. */
int gphq_prefill_extend_embed(gphq_prefill *ws, gphq_prefix *kv, int64_t stored, int64_t keep, int64_t reuse,
                              const int32_t *tokens, int64_t n, const gphq_embeds *embeds, float *tail_dev,
                              int64_t tail_len, void *stream);
/* HiddenLastBatchInto (evaluator.go:525-575) and, with a shared prefix,
 * HiddenLastSharedInto (evaluator.go:408-425): `count` independent sequences,
 * their tokens concatenated in `tokens` (host) with lengths lens[count], packed
 * into shared passes of at most the workspace's rows (batchPacked,
 * gpu_darwin.go:1445-1500). Each sequence attends to its own earlier tokens
 * and, when shared is not NULL, to the first `past` rows of shared, which is
 * only read; positions start at `past` (0 without a prefix). The new rows' K/V
 * live in the workspace's own cache (allocated on first use: layers x rows x
 * kv_dim x 8 bytes). hidden_dev receives count x hidden floats, row s the
 * post-final-norm state of sequence s's last token. Validation follows
 * HiddenLastSharedInto, then HiddenLastBatchInto's checks per sequence in
 * order, before any device work. */
int gphq_prefill_batch(gphq_prefill *ws, const gphq_prefix *shared, int64_t past, const int32_t *tokens,
                       const int64_t *lens, int64_t count, float *hidden_dev, int64_t hidden_len, void *stream);
/* Waits for the stream; GPHQ_ERR_NON_FINITE_STATE if an extension since the
 * last check produced a non-finite hidden value. */
int gphq_prefill_check(gphq_prefill *ws, void *stream);
/* Projection arithmetic of the workspace's passes. GPHQ_PASS_FP16 (the
 * default) is the GPU provider's mm (FP16 tiles, fp32 sums, the fp32 GEMV
 * for one-token passes). GPHQ_PASS_INT8 is the CPU provider's int8 route
 * (qwen3lm/ops.go:96-147, 198-215: each projection input row normalized where
 * the pass normalizes it, quantized with WorkspaceI8's per-row rule,
 * int8.go:106-168, and multiplied exactly in int32 with MulPanelsI8's scaling
 * (float32(sum) * weight row scale) * activation row scale, int8.go:170-211),
 * for every pass including one-token ones, over the Q8 layer format's per-row
 * int8 codes and scales on int8 MFMA. GPHQ_ERR_UNSUPPORTED for other layer
 * formats. The int8 route allocates rows x max(hidden, q_dim, intermediate)
 * bytes on first selection. */
#define GPHQ_PASS_FP16 0
#define GPHQ_PASS_INT8 1
int gphq_prefill_set_arith(gphq_prefill *ws, int arith);
int gphq_prefill_arith(const gphq_prefill *ws);
/* One projection of a pass (ops.go:198-215 projectPanel over every panel; the
 * GPU provider's mm dispatch of encodeBatch, gpu_darwin.go:1703-1764) on
 * `rows` (<= the workspace's rows) rows of x_dev with the workspace's
 * arithmetic: proj 0 = QKV of RMS-normalized rows stored into y_dev
 * [rows][q_dim + 2 kv_dim]; 1 = O, y_dev [rows][hidden] += x [rows][q_dim] W^T;
 * 2 = gate/up of normalized rows, SwiGLU stored into y_dev [rows][intermediate];
 * 3 = down, y_dev [rows][hidden] += x' [rows][intermediate] W^T, where x' is
 * x after the intermediate rotation for Q8/Q4 layers (rotate, gpu.metal:
 * 339-367, applied by the projection's input packing; a one-row FP16-route
 * call rotates x_dev in place). Enqueued on stream. */
int gphq_prefill_project(gphq_prefill *ws, int64_t layer, int proj, const float *x_dev, int64_t rows, float *y_dev,
                         void *stream);

/* ---- Block-32 int8 GEMM (benchmark configuration 2 as worded there) -----------
 * No counterpart in the reference, whose q8gemm int8 path scales per row
 * (gphq_q8gemm_* above). Activations and weights carry one fp32 scale per
 * 32-value block; each block is quantized with WorkspaceI8's per-row rule
 * (int8.go:106-168: scale max/127, inverse 127/max, both 0 unless
 * 0 < max < inf; codes RNE(x * inverse) saturated, NaN -> 0).
 * gphq_q8b_quantize: x [rows][x_stride] fp32 -> q [rows][k] int8 and
 * d [rows][k/32] fp32; k % 32 == 0, x_stride a multiple of 4 and >= k, x 16-byte
 * aligned. gphq_q8b_gemm: y [m][n] fp32 = for each output, over the blocks b
 * in order, acc = fmaf(float(dot_b), da[r][b] * dw[c][b], acc) from +0, dot_b
 * the exact int32 product of the block's codes; weights qw [n][k] int8
 * row-major (the Q8B_F32 code layout) with dw [n][k/32]. Bit-exact. */
int gphq_q8b_quantize(const float *x_dev, int64_t rows, int64_t k, int64_t x_stride, int8_t *q_dev, float *d_dev,
                      void *stream);
int gphq_q8b_gemm(const int8_t *qa_dev, const float *da_dev, const int8_t *qw_dev, const float *dw_dev, float *y_dev,
                  int64_t m, int64_t k, int64_t n, void *stream);

/* ---- GPTQ producer (cmd/qwen3-gptq) -------------------------------------------
 * Replaces the core of qwen3lm quantizeGroup (gptq.go:604-666) for one group of
 * projections that share their calibration inputs, on the device; the corpus,
 * its tokenization and the model pass that collects the inputs, and the
 * GPHQ0001 file writer, stay with the caller. fp32 products and storage as the
 * reference's; the small substitutions sum in float64 as the reference's do;
 * results agree with the reference to fp32 rounding, not bit for bit (its
 * products sum in whispergemm's order). */
/* Device scratch for gphq_gptq_factor: 4k^2 + 256k + 256 bytes. */
int64_t gphq_gptq_work_bytes(int64_t k);
/* H = X^T X of x_dev [rows][k] (fp32), dead channels (H[i][i] == 0 ->
 * dead_dev[i] = 1, H[i][i] = 1), H += 0.01*mean(diag(H))*I, and
 * u_dev [k][k] = U, upper triangular with H^-1 = U^T U (gptqInverseFactor,
 * gptq_linalg.go:185-223). Synchronizes the stream; returns
 * GPHQ_ERR_NOT_POSITIVE_DEFINITE where the reference returns its error. */
int gphq_gptq_factor(const float *x_dev, int64_t rows, int64_t k, float *u_dev, uint8_t *dead_dev, void *work_dev,
                     int64_t work_bytes, void *stream);
/* Device scratch for gphq_gptq_round: 512n + 4n bytes. */
int64_t gphq_gptq_round_work_bytes(int64_t n, int64_t k);
/* gptqRound (gptq.go:671-796) of w_dev [n][k] (fp32, in place: dead columns
 * zeroed, every value replaced by its rounded value) against U: bits 8 ->
 * codes int8 [n][k] and fp32 row scales max|row|/127; bits 4 -> the GPU Q4
 * bytes [n][k/2] (group of 32: value j low nibble of byte j, value j+16 high,
 * stored + 8) and FP16 group scales (q4GroupScale) [n][k/32]. */
int gphq_gptq_round(float *w_dev, int64_t n, int64_t k, const float *u_dev, const uint8_t *dead_dev, int bits,
                    void *codes_dev, void *scales_dev, void *work_dev, int64_t work_bytes, void *stream);

/* ---- GPTQ calibration pass (cmd/qwen3-gptq -> qwen3lm.QuantizeGPTQ) --------
 * Replaces QuantizeGPTQ's model pass (gptq.go:191-266) and its calibration
 * (newCalibration, calibration.weights / layer / attention, normalizedRows,
 * project; gptq.go:330-600) on the device: the model runs layer by layer in
 * FP32 over the calibration rows in the GPU backend's basis (residual rotated
 * by the hidden rotation, RMSNorm weights folded into the next projections,
 * value rows and o inputs per-head rotated, down inputs rotated by the
 * intermediate rotation), and each projection is rounded with GPTQ
 * (gphq_gptq_factor / gphq_gptq_round) against the inputs the rounded layers
 * before it produce; the next projections and the residual advance through the
 * rounded matrices. fp32 throughout; sums run in another order than the
 * reference's, so results agree to fp32 rounding, not bit for bit. The
 * tokenizer stays with the caller: calibration text arrives as token ids.
 *
 * gphq_gptq_calibration_new (newCalibration, gptq.go:344-383): nseq sequences
 * of seq_lens[s] tokens (1..256 each, gptqMaxSeq; at most 4096 in all,
 * gptqMaxRows), ids concatenated in ids; each row embedded from the BF16 table
 * [vocab][hidden] (device, embed_len values) and rotated; row positions count
 * from 0 in each sequence. cfg as gphq_lm_new (its fmt is ignored). Waits for
 * the stream. GPHQ_ERR_CALIBRATION_EMPTY without rows.
 * gphq_gptq_calibration_layer (calibration.layer, gptq.go:437-524): one layer
 * from its seven BF16 projections src_bf16_dev[7] (device [n][k]: q_proj,
 * k_proj, v_proj, o_proj, gate_proj, up_proj, down_proj), the float32 input /
 * post-attention norms [hidden] and q / k norms [128] (host); bits 8 or 4;
 * codes_dev[p] / scales_dev[p] receive projection p as gphq_gptq_round
 * writes it (gptqRowBytes per row), in the file's layout. The residual
 * advances through the rounded layer. Waits for the stream.
 * gphq_gptq_calibration_rows: the shape [rows][width] of one set of rows
 * and, with dst_dev, a stream-ordered copy of them (dst_len floats at least):
 * the residual (after the last layer run, or the embedded rows before any),
 * or the last layer's attention input (normalized rows, q/k/v's GPTQ input),
 * context (o's), MLP input (gate/up's) or down input (rotated SwiGLU rows).
 * gphq_gptq_calibration_sequences (calibrationSequences' add, gptq.go:275-287):
 * the sequence lengths ntexts tokenized texts give, each text cut into pieces
 * of at most 256 tokens until 4096 are taken; with seq_lens NULL only *nseq.
 * gphq_gptq_quantize (QuantizeGPTQ, gptq.go:197-266): format "gpu" (8 bits)
 * or "gpu-q4" (4 bits) -- else GPHQ_ERR_UNSUPPORTED --, widths that are
 * multiples of 4096 (GPHQ_ERR_GPTQ_WIDTH), the texts' token ids cut as above
 * (GPHQ_ERR_CALIBRATION_EMPTY without any), the checkpoint of dir
 * (model.embed_tokens.weight and the layers' BF16 projections and norms) and
 * its GPHQ0001 file written through gphq_gptq_create / commit, layer by layer;
 * progress(layer, layers, user) after each (may be NULL). The temporary file
 * is removed on any error. */
typedef struct gphq_gptq_calibration gphq_gptq_calibration;
typedef void (*gphq_gptq_progress)(int64_t layer, int64_t layers, void *user);
#define GPHQ_CAL_RESIDUAL 0
#define GPHQ_CAL_ATTN_INPUT 1
#define GPHQ_CAL_CONTEXT 2
#define GPHQ_CAL_MLP_INPUT 3
#define GPHQ_CAL_DOWN_INPUT 4
int gphq_gptq_calibration_new(const gphq_lm_config *cfg, const int32_t *ids, const int64_t *seq_lens, int64_t nseq,
                              const uint16_t *embed_bf16_dev, int64_t embed_len, gphq_gptq_calibration **out,
                              void *stream);
void gphq_gptq_calibration_free(gphq_gptq_calibration *cal);
int gphq_gptq_calibration_layer(gphq_gptq_calibration *cal, const uint16_t *const *src_bf16_dev,
                                const float *input_norm_host, const float *post_norm_host, const float *q_norm_host,
                                const float *k_norm_host, int bits, void *const *codes_dev, void *const *scales_dev,
                                void *stream);
int gphq_gptq_calibration_rows(const gphq_gptq_calibration *cal, int which, float *dst_dev, int64_t dst_len,
                               int64_t *rows, int64_t *width, void *stream);
int gphq_gptq_calibration_sequences(const int64_t *text_lens, int64_t ntexts, int64_t *seq_lens, int64_t max_seqs,
                                    int64_t *nseq);
int gphq_gptq_quantize(const char *dir, const char *format, const gphq_lm_config *cfg, const int32_t *ids,
                       const int64_t *text_lens, int64_t ntexts, gphq_gptq_progress progress, void *user,
                       void *stream);

/* ---- safetensors checkpoints (internal/safetensors/safetensors.go) --------
 * Open reads the tensor index of dir: model.safetensors, or the shards of
 * model.safetensors.index.json's weight_map (safetensors.go:39-82, header
 * rules 85-127). Tensors are read on demand: Lookup checks the shape and the
 * dtype's byte count (140-162); BF16 reads raw BF16 bits (165-176, host, or
 * device through a host copy); ReadBits reads count 16-bit values from
 * element offset (203-213); Float32 widens BF16 / F16 / F32 and rejects
 * non-finite values (217-251); MapBF16 maps the bits read-only (178-200,
 * released by gphq_mapping_free). dtype codes: */
#define GPHQ_DTYPE_BF16 1
#define GPHQ_DTYPE_F16 2
#define GPHQ_DTYPE_F32 3
typedef struct gphq_checkpoint gphq_checkpoint;
typedef struct gphq_mapping gphq_mapping;
int gphq_checkpoint_open(const char *dir, gphq_checkpoint **out);
void gphq_checkpoint_close(gphq_checkpoint *c);
int gphq_checkpoint_has(const gphq_checkpoint *c, const char *name);
/* Tensor.DType (0 for another type) and Tensor.Shape (up to max_ndim dims). */
int gphq_checkpoint_info(const gphq_checkpoint *c, const char *name, int32_t *dtype, int64_t *shape, int64_t max_ndim,
                         int64_t *ndim);
int gphq_checkpoint_lookup(const gphq_checkpoint *c, const char *name, const int64_t *shape, int64_t ndim,
                           int32_t *dtype);
int gphq_checkpoint_read_bits(const gphq_checkpoint *c, const char *name, uint16_t *dst, int64_t count,
                              int64_t offset);
int gphq_checkpoint_bf16(const gphq_checkpoint *c, const char *name, const int64_t *shape, int64_t ndim, uint16_t *dst,
                         int64_t dst_len);
int gphq_checkpoint_bf16_device(const gphq_checkpoint *c, const char *name, const int64_t *shape, int64_t ndim,
                                uint16_t *dst_dev, int64_t dst_len);
int gphq_checkpoint_float32(const gphq_checkpoint *c, const char *name, const int64_t *shape, int64_t ndim, float *dst,
                            int64_t dst_len);
int gphq_checkpoint_map_bf16(const gphq_checkpoint *c, const char *name, const int64_t *shape, int64_t ndim,
                             gphq_mapping **out, const uint16_t **bits);
void gphq_mapping_free(gphq_mapping *m);

/* ---- GPTQ weight file "GPHQ0001" (qwen3lm/gptq.go:36-196, 227-270) --------
 * The file cmd/qwen3-gptq writes next to the checkpoint as
 * gophonic-gptq-<format>.bin ("gpu": 8 bits, GPHQ_FMT_Q8 rows; "gpu-q4": 4
 * bits, GPHQ_FMT_Q4 rows): a 24-byte header (magic, bits, fingerprint, u64
 * LE), then per layer and projection (q, k, v, o, gate, up, down) all rows'
 * codes, then all rows' scales (gptqRowBytes: 8 bits k and 4 bytes a row, 4
 * bits k/2 and 2*(k/32)). The fingerprint is snapshotFingerprint: FNV-1a 64
 * over "name size mtime_ns\n" of the sorted *.safetensors and config.json
 * files of dir. gphq_gptq_open leaves *out NULL (status GPHQ_OK) when there is
 * no file, or it holds other bits, another fingerprint or another size.
 * gphq_gptq_projection gives a tensor's offsets from its name after the
 * decoder prefix ("layers.3.mlp.up_proj.weight"; 1 if held, else 0);
 * gphq_gptq_place copies one into a device layer buffer, source row r at row
 * row0 + r*step of the codes at byte base and of the scales at sc (*placed 0
 * when not held). The writer writes the header to <file>.tmp, appends
 * projections in file order (host bytes, or device bytes such as
 * gphq_gptq_round's), and renames on commit. */
typedef struct gphq_gptq_file gphq_gptq_file;
typedef struct gphq_gptq_writer gphq_gptq_writer;
int gphq_gptq_row_bytes(int bits, int64_t k, int64_t *codes, int64_t *scales);
int gphq_gptq_fingerprint(const char *dir, uint64_t *out);
int gphq_gptq_path(const char *dir, const char *format, char *out, int64_t out_len);
int gphq_gptq_open(const char *dir, const char *format, const gphq_lm_config *cfg, gphq_gptq_file **out);
void gphq_gptq_close(gphq_gptq_file *g);
int gphq_gptq_bits(const gphq_gptq_file *g);
int gphq_gptq_projection(const gphq_gptq_file *g, const char *name, int64_t *codes_off, int64_t *scales_off);
int gphq_gptq_place(const gphq_gptq_file *g, const char *name, int64_t n, int64_t k, void *buf_dev, int64_t buf_bytes,
                    int64_t base, int64_t sc, int64_t row0, int64_t step, int *placed);
int gphq_gptq_create(const char *dir, const char *format, gphq_gptq_writer **out);
int gphq_gptq_write(gphq_gptq_writer *w, const void *data, int64_t len);
int gphq_gptq_write_device(gphq_gptq_writer *w, const void *data_dev, int64_t len);
int gphq_gptq_commit(gphq_gptq_writer *w);
void gphq_gptq_abort(gphq_gptq_writer *w);

/* ---- prepared-weight cache "GPHWCACH" (internal/wcache/wcache.go) --------
 * Key (wcache.go:59-86): "<sanitized dir name>-<sha256(abs dir)[:4] hex>.
 * <sanitized kind>.<sha256(parts NUL-terminated, then name NUL size NUL
 * mtime_ns NUL of each regular file of dir in name order)[:12] hex>".
 * Open (109-140) maps the complete entry <cache_dir>/<key>.bin read-only
 * (fresh 0), or returns a zeroed writable fresh entry (a temporary file under
 * an advisory lock on <cache_dir>/<key up to its last '.'>.lock, so one
 * process prepares while others wait; anonymous memory when cache_dir is ""
 * or cannot be written; cache_dir NULL: $GOPHONIC_CACHE, else
 * $XDG_CACHE_HOME or ~/.cache, /gophonic). The file is a GPHQ_WCACHE_ALIGN
 * header (magic, total size, complete flag) and the payload rounded up to
 * GPHQ_WCACHE_ALIGN. Commit (207-258) syncs the payload, then the complete
 * flag, renames the entry into place, removes the entries it replaces (same
 * name and kind) and temporaries over an hour old, and maps it again
 * read-only (take payload pointers after Commit). Done (198-205) starts
 * writing a filled region back. Close discards a fresh entry. Layout's Take
 * rounds each region up with gphq_wcache_round_up. */
#define GPHQ_WCACHE_ALIGN (16 << 10)
typedef struct gphq_wcache_file gphq_wcache_file;
int64_t gphq_wcache_round_up(int64_t n);
int gphq_wcache_key(const char *dir, const char *kind, const char *const *parts, int64_t nparts, char *out,
                    int64_t out_len);
int gphq_wcache_sha256(const void *data, int64_t len, uint8_t *out32);
int gphq_wcache_open(const char *cache_dir, const char *key, int64_t size, gphq_wcache_file **out);
int gphq_wcache_fresh(const gphq_wcache_file *f);
void *gphq_wcache_payload(gphq_wcache_file *f, int64_t *len);
void gphq_wcache_done(gphq_wcache_file *f, const void *region, int64_t len);
void gphq_wcache_commit(gphq_wcache_file *f);
int gphq_wcache_close(gphq_wcache_file *f);

#ifdef __cplusplus
}
#endif
#endif /* GPHQ_H */
