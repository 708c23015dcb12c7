// Launchers for the token loop's non-product kernels.
#pragma once

#include "q8_internal.h"

constexpr uint32_t ATTN_MAX_KEYS = 4096;      // visible keys one query attends to
constexpr uint32_t ATTN_MAX_HEAD_DIM = 256;

struct AttnArgs {
    const int32_t* q;        // [tokens][heads*head_dim]
    uint32_t q_stride;
    const int32_t* k_cache;  // [position][kv_heads*head_dim]
    const int32_t* v_cache;
    uint32_t kv_stride;
    int32_t* ctx;            // [tokens][heads*head_dim]
    uint32_t ctx_stride;
    const int32_t* d_pos;    // absolute position of token 0
    uint32_t heads, kv_heads, head_dim;
    int scaled;              // 1: mistral scaled_score; 0: gemma requantized dot
    uint32_t scale_q32;
    uint32_t window;         // 0 = every earlier position is visible
};

struct SelectArgs {
    const int32_t* logits;
    uint32_t vocab;
    int32_t* tokens_out;     // [steps]
    int32_t* logits_keep;    // [steps][vocab] or null
    int32_t* d_step;
    int32_t* d_pos;
    uint32_t rows_in_pass;
    const uint8_t* embed_raw;  // Q8_0 rows, reference layout
    uint32_t row_bytes;
    uint32_t hidden;
    int32_t embed_scale;     // 0 = unscaled
    int32_t* x_next;         // [hidden]
};

// Attention for `tokens` query rows; max_keys bounds the visible keys of the
// last row (checked against the kernel's capacity).
int iris_attention_launch(const AttnArgs& a, uint32_t tokens, uint32_t max_keys, hipStream_t stream);
int iris_select_embed_launch(const SelectArgs& a, hipStream_t stream);
int iris_embed_rows_launch(const int32_t* d_ids, uint32_t count, const uint8_t* embed_raw, uint32_t row_bytes,
                           uint32_t hidden, int32_t scale, int32_t* out, hipStream_t stream);
