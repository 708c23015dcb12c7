// Launchers for the token loop's non-product kernels.
#pragma once

#include "q8_internal.h"

constexpr uint32_t ATTN_MAX_KEYS = 4096;      // visible keys one query attends to
constexpr uint32_t ATTN_MAX_HEAD_DIM = 256;

struct AttnArgs {
    const int32_t* q;        // [tokens][heads*head_dim]
    uint32_t q_stride;
    const int32_t* k_cache;  // transposed: [kv_heads*head_dim][k_pos_stride positions]
    uint32_t k_pos_stride;
    const int32_t* v_cache;  // [position][kv_heads*head_dim]
    uint32_t kv_stride;
    int32_t* ctx;            // [tokens][heads*head_dim]
    uint32_t ctx_stride;
    const int32_t* d_pos;    // absolute position of token 0
    uint32_t heads, kv_heads, head_dim;
    int scaled;              // 1: mistral scaled_score; 0: gemma requantized dot
    uint32_t scale_q32;
    uint32_t window;         // 0 = every earlier position is visible
    // Scratch for the split decode path (one query row), sized for
    // heads x ATTN_MAX_KEYS scores, heads x ATTN_MAX_CHUNKS chunk records.
    int32_t* scores;         // [heads][ATTN_MAX_KEYS]
    uint64_t* chunk_max;     // [heads][ATTN_MAX_CHUNKS]: (index << 32) | (uint32)score
    int64_t* chunk_acc;      // [heads][ATTN_MAX_CHUNKS][head_dim]
    int32_t* chunk_wsum;     // [heads][ATTN_MAX_CHUNKS]
    int32_t* max_weight;     // [heads]: the first maximum's weight before the residual
};

constexpr uint32_t ATTN_CHUNK = 128;  // keys per workgroup in the split decode path
constexpr uint32_t ATTN_MAX_CHUNKS = ATTN_MAX_KEYS / ATTN_CHUNK;

// Attention for `tokens` query rows; max_keys bounds the visible keys of the
// last row (checked against the kernel's capacity).
int iris_attention_launch(const AttnArgs& a, uint32_t tokens, uint32_t max_keys, hipStream_t stream);
int iris_embed_rows_launch(const int32_t* d_ids, uint32_t count, const uint8_t* embed_raw, uint32_t row_bytes,
                           uint32_t hidden, int32_t scale, int32_t* out, hipStream_t stream);
