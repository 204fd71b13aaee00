// The qwen3lm model and prefix objects shared by the decode provider
// (lm_decode.hip) and the batched pass (lm_prefill.hip).
#pragma once
#include <atomic>
#include <vector>

#include "common.h"

struct gphq_lm {
    gphq_lm_config cfg;
    int64_t qd, kvd, group, hblock, iblock, positions;
    std::vector<gphq_lm_layer> layers;
    std::vector<char> bound;
    float *norms = nullptr;   // [layers][2][128]: q_norm, k_norm
    float *rope = nullptr;    // [2][positions][64]: cos, then sin
    float *hsigns = nullptr;  // hidden rotation sign*scale [hidden]
    float *isigns = nullptr;  // intermediate rotation sign*scale [inter]
    float *final_norm = nullptr;
    const uint16_t *embed = nullptr;
    const uint8_t *head = nullptr;
    int64_t head_scale = 0, head_rows = 0;
    // New value on every bind (layer, embedding, head): a captured step graph
    // holds the bound addresses, so it is valid only for the generation it
    // was captured under.
    uint64_t gen = 0;
};

struct gphq_prefix {
    const gphq_lm *lm;
    float *kc = nullptr, *vc = nullptr;  // [layers][capacity][kvd]
    int64_t capacity = 0;
    // Unique per prefix object for the life of the process (host addresses
    // of freed prefixes are reused; generations are not).
    uint64_t gen = 0;
};

namespace gphq {

constexpr int kLmHeadDim = 128;

// Process-wide source of model-binding and prefix generations (never 0).
inline uint64_t next_generation() {
    static std::atomic<uint64_t> counter{0};
    return counter.fetch_add(1, std::memory_order_relaxed) + 1;
}

// Whether the embedding, head, final norm and every layer are bound.
bool lm_model_ready(const gphq_lm *lm);
// h[r] = R . float32(bf16 embedding row of tok[r]) for r < rows (tok on the
// device, clamped into the vocabulary); with a splice table, a token -1-j
// takes R . splice[j] (an fp32 Embeds row) instead.
int lm_embed_launch(const gphq_lm *lm, const int32_t *tok, int rows, float *h, hipStream_t st,
                    const float *splice = nullptr);
// The down input's online Hadamard over `rows` rows of the intermediate
// width, rows `stride` floats apart.
int lm_rotate_launch(const gphq_lm *lm, float *act, int rows, long stride, hipStream_t st);
// Final norm of `rows` residual rows: hidden[r] (post-final-norm state),
// hn[r] = R hidden[r] (the head's input; skipped for a null hn); sets
// nonfinite[r] (nonfinite[0] with one_flag) on a non-finite hidden value.
int lm_final_launch(const gphq_lm *lm, const float *h, int rows, float *hidden, float *hn, int32_t *nonfinite,
                    hipStream_t st, bool one_flag = false);

}  // namespace gphq
