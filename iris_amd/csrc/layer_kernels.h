// Launchers for the token loop's non-product kernels.
#pragma once

#include "q8_internal.h"

// Visible keys one query attends to: the matrix-core prefill's value sums
// stay in int32 below 2^16 keys (each 64-key step adds at most 2 * 64 * 2^14).
constexpr uint32_t ATTN_MAX_KEYS = 65535;
// Keys whose weights one workgroup holds in LDS at a time; longer views take
// the tiled paths (scores re-read or re-formed per pass).
constexpr uint32_t ATTN_TILE_KEYS = 4096;
// Scores workgroups per query head of a one-row launch, at most (longer
// views loop over 64-position chunks).
constexpr uint32_t ATTN_DECODE_CHUNKS = 32;
// Head sizes up to 512 (gemma-dense full-attention layers, global_head_dim
// 512 in the reference's gemma-4 manifests).
constexpr uint32_t ATTN_MAX_HEAD_DIM = 512;

// Work space of the multi-row attention: the signed byte digits (four
// planes) of the queries, keys and values in MFMA operand tiles, and the
// digits each tile needs (5 = a value beyond four digits: scalar path).
struct AttnPlanes {
    int8_t* q;               // [4][heads][qt_cap][head_dim/64][1 KB]
    int8_t* k;               // [4][kv_heads][ks_cap*4][head_dim/64][1 KB]
    int8_t* v;               // [4][kv_heads][ks_cap][head_dim/16][1 KB]
    uint8_t* q_limbs;        // [heads][qt_cap]
    uint8_t* kv_limbs;       // [kv_heads][ks_cap][2]: keys', values' digits per 64-key step
    uint32_t* e_store;       // [heads][qt_cap][ks_cap*4][64][4]: exp terms between the softmax passes
    uint32_t qt_cap;         // 16-row query tiles
    uint32_t ks_cap;         // 64-key steps
};

// Bytes of each plane buffer for heads x head_dim queries over qt_cap tiles
// and kv_heads x head_dim keys over ks_cap steps.
inline uint64_t attn_q_planes_bytes(uint32_t heads, uint32_t head_dim, uint32_t qt_cap) {
    return 4ull * heads * qt_cap * 16 * head_dim;
}
inline uint64_t attn_kv_planes_bytes(uint32_t kv_heads, uint32_t head_dim, uint32_t ks_cap) {
    return 4ull * kv_heads * ks_cap * 64 * head_dim;
}
inline uint64_t attn_e_store_bytes(uint32_t heads, uint32_t qt_cap, uint32_t ks_cap) {
    return 4096ull * heads * qt_cap * ks_cap;
}

// int32 elements of AttnArgs::scores for `heads` query heads.
inline uint64_t attn_scores_ints(uint32_t heads, uint32_t k_pos_stride) {
    return (uint64_t)heads * k_pos_stride + 2ull * heads * ATTN_DECODE_CHUNKS;
}

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
    // One-row launches: the head's scores between the two decode kernels,
    // [heads][k_pos_stride], then each scores workgroup's first maximum,
    // [heads][ATTN_DECODE_CHUNKS] 64-bit keys; attn_scores_ints elements
    // (null: the one-workgroup-per-head kernel).
    int32_t* scores;
    // Digit planes for the multi-row MFMA path (planes.q null: the scalar
    // kernel), sized by attn_q_planes_bytes / attn_kv_planes_bytes /
    // attn_e_store_bytes.
    AttnPlanes planes;
    // One-row launches (iris_attention_decode_applies): the context row's
    // digit planes too, in the act_planes layout over heads*head_dim values
    // (null: not written).
    uint32_t* ctx_planes;
    uint8_t* ctx_counts;
};


// Attention for `tokens` query rows; max_keys bounds the visible keys of the
// last row (checked against the kernel's capacity).
int iris_attention_launch(const AttnArgs& a, uint32_t tokens, uint32_t max_keys, hipStream_t stream);
// One row through the two decode launches (chunked scores, then values per
// 32-dimension slice): the only path that writes ctx_planes.
bool iris_attention_decode_applies(const AttnArgs& a, uint32_t tokens, uint32_t max_keys);
// The multi-row MFMA attention (attn_prefill.hip): applies to head sizes 64,
// 128, 256 and 512 (the last two from 128 workgroups on) with a multiple of
// four query heads, given plane space for `tokens` rows and `max_keys` keys.
bool iris_attention_prefill_applies(const AttnArgs& a, uint32_t tokens, uint32_t max_keys);
int iris_attention_prefill_launch(const AttnArgs& a, uint32_t tokens, uint32_t max_keys, hipStream_t stream);
// *d_pos = pos and *d_step = step, in stream order.
int iris_set_counters_launch(int32_t* d_pos, int32_t pos, int32_t* d_step, int32_t step, hipStream_t stream);
int iris_embed_rows_launch(const int32_t* d_ids, uint32_t count, const uint8_t* embed_raw, uint32_t row_bytes,
                           uint32_t hidden, int32_t scale, int32_t* out, hipStream_t stream);

// ---- gemma-dense (gemma_kernels.hip) ----

constexpr uint32_t GEMMA_MAX_HEAD_DIM = ATTN_MAX_HEAD_DIM;
constexpr uint32_t GEMMA_MAX_PLE = 4096;

struct GemmaQkvArgs {
    const int32_t* qkv;      // [rows][(heads + 2*kv_heads) * head_dim], the raw q|k|v products
    uint32_t qkv_stride;
    uint32_t heads, kv_heads, head_dim, rotary_dim;
    const int32_t* q_norm;   // [head_dim]
    const int32_t* k_norm;   // [head_dim]
    int64_t eps;             // Q32.32
    const int64_t* inv_freq; // [rotary_dim / 2] Q32.32
    const int32_t* d_pos;    // absolute position of row 0
    int32_t* q_out;          // [rows][heads*head_dim]
    uint32_t q_stride;
    int32_t* k_cache;        // transposed: [kv_heads*head_dim][k_pos_stride]
    uint32_t k_pos_stride;
    int32_t* v_cache;        // [position][kv_heads*head_dim]
};

struct I32GemvArgs {
    const int32_t* w;        // Q16.16 [rows][cols], cols % 4 == 0
    uint32_t rows, cols;
    const int32_t* x;        // [tokens][x_stride]
    uint32_t x_stride;
    int32_t* out;            // [tokens][out_stride]
    uint32_t out_stride;
    const int32_t* aux;      // nullable: out = mul_sat(gelu(dot), aux[t][r])
    uint32_t aux_stride;
    // One row (tokens == 1) only:
    // - res_in set: the product's input is y = add_sat(rms_norm(x, res_norm_w, eps), res_in),
    //   the norm's sum of squares from ssq_in[0 .. ssq_n); workgroup 0 writes y to res_out
    //   (nullable; not x or res_in); cols <= I32_GEMV_MAX_STAGED;
    // - ssq_out set: one saturating sum of squares of the outputs per workgroup,
    //   ssq_out[0 .. i32_gemv_slots(rows)).
    const int32_t* res_in;
    const int32_t* res_norm_w;
    int64_t eps;
    const int64_t* ssq_in;
    uint32_t ssq_n;
    int32_t* res_out;
    int64_t* ssq_out;
};

constexpr uint32_t I32_GEMV_MAX_STAGED = 8192;  // elements of a staged input row (32 KiB of LDS)
constexpr uint32_t I32_GEMV_MAX_SLOTS = 256;
// Workgroups (and sum-of-squares slots) of a one-row launch with ssq_out:
// four waves, each taking rows_per_wave rows, so that at most
// I32_GEMV_MAX_SLOTS workgroups cover the rows.
uint32_t i32_gemv_slots(uint32_t rows);

struct PleArgs {
    const int32_t* proj;     // [rows][row_stride]: dot_bits of the projection, all segments
    uint32_t row_stride;     // layers * ple_width
    const int32_t* ids;      // [rows] token ids
    const uint8_t* emb;      // embed_tokens_per_layer, Q8_0 rows of row_stride values
    uint32_t emb_row_bytes;
    uint32_t ple_width;
    const int32_t* norm_w;   // per_layer_projection_norm [ple_width]
    int64_t eps;
    int32_t projection_scalar, embedding_scale, input_scale;
    int32_t* out;            // [rows][row_stride]
};

int iris_gemma_qkv_finish_launch(const GemmaQkvArgs& a, uint32_t rows, hipStream_t stream);
int iris_norm_residual_launch(const int32_t* a, uint32_t a_stride, const int32_t* w, int64_t eps, const int32_t* res,
                              uint32_t res_stride, int32_t scalar, int32_t* out, uint32_t out_stride, uint32_t n,
                              uint32_t rows, hipStream_t stream);
int iris_i32_gemv_launch(const I32GemvArgs& a, uint32_t tokens, hipStream_t stream);
// The device's silu table (dn::SILU_TAB_N values of dn::silu), made on the
// first call on a device and kept until the process ends.
int iris_silu_table(const int32_t** out);
int iris_ple_prepare_launch(const PleArgs& a, uint32_t segments, uint32_t rows, hipStream_t stream);
// (sin, cos) in Q30 (mistral.rs:84-109) of position * inv_freq[j] for the
// `rows` positions from *d_pos and j < half: out[row][j][2].
int iris_rope_table_launch(const int64_t* inv_freq, uint32_t half, const int32_t* d_pos, uint32_t rows, int64_t* out,
                           hipStream_t stream);
int iris_rope_ladder_launch(int64_t base, uint32_t freq_base_dim, uint32_t half, int64_t* out, hipStream_t stream);
