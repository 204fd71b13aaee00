// Shared declarations of the FP16-operand GEMM (gemm_f16.hip) and its host
// callers (q8gemm_f16.hip, lm_prefill.hip).
#pragma once
#include "common.h"

namespace gphq {

enum WFmt {
    W_I8_TILE = 0,    // q8gemm int8 weights, tile layout (1 KiB groups)
    W_F16_TILE = 1,   // q8gemm FP16 weights, tile layout (2 KiB groups)
    W_Q8_ROW = 2,     // qwen3lm Q8 codes [N][K] (fp32 row scales in the epilogue)
    W_Q8B_ROW = 3,    // qwen3lm Q8B codes [N][K], f16 scales [N][K/32]
    W_Q4_ROW = 4,     // qwen3lm Q4 codes [N][K/2], f16 scales [N][K/32]
    W_GPTQ_ROW = 5,   // int32 [N][K/8] (nibble i of word j = k 8j+i), f16 scales and u8 zeros [N][K/128]
    W_Q8BF_ROW = 6,   // qwen3lm Q8B codes [N][K] with fp32 scales [N][K/32]
};

// EPI_ADD: dst += v (the residual stream). EPI_SWIGLU: columns 2i (gate) and
// 2i+1 (up) give dst[row][i] = g / (1 + exp(-g)) * u. Both multiply by
// colScale[col] first when it is set (Q8 row scales).
enum Epi { EPI_PANELS = 0, EPI_PLAIN = 1, EPI_ROWSCALE = 2, EPI_ADD = 3, EPI_SWIGLU = 4 };

struct F16GemmArgs {
    const _Float16 *A;   // activations, FP16 tile layout, MT x KT groups
    const void *B;       // weights (layout per WFmt)
    const void *bScale;  // Q8B/Q4: f16 [N][K/32]; GPTQ: f16 [N][K/128]
    const uint8_t *bZero;  // GPTQ: u8 [N][K/128]
    const float *colScale;  // EPI_PANELS, EPI_ROWSCALE: fp32 [N]
    const float *rowInv;    // EPI_PANELS: fp32 [M]
    float *dst;
    long stride;
    int M, N, K, KT, NT;
    int c0, c1, tileN0;
    int gridM, gridN;
    float *part;   // split-K partial sums [splits][M][c1 - c0], or null
    int splits;    // K splits (1: none)
};

// Dispatch over weight format and epilogue; arguments were validated.
int f16gemm_launch(int wf, int epi, F16GemmArgs a, hipStream_t stream);
// K splits of a 128 x 128-tile GEMM whose grid has `tiles` blocks (1: none).
int mm_split_count(long tiles, int KT, long outs);

}  // namespace gphq
