/*
 * CPU oracle, layer level: the reference's product dispatch, the two layer
 * families, the per-layer-embedding prepare step and the head, restated in C
 * over det-num (detnum.h). TEST INFRASTRUCTURE ONLY: tests, the smoke check
 * and the benchmark's CPU-baseline leg call it; the shipped library never does.
 *
 * Layouts: activations are row-major int32 [tokens][width]; Q8_0 matrices
 * are the reference's raw bytes, rows of cols/32 blocks of 34 bytes; a key
 * cache is int32 [positions][kv_heads*head_dim], one row per position.
 * All functions return 0 on success and a negative code on a malformed input.
 *
 * Parity unpinned: the reference holds no expected outputs for a whole layer,
 * the head or a generation, and its Rust source cannot be built here. The
 * layer forwards, orc_gemma_ple_prepare and orc_head_logits are pinned only
 * by structural invariants (batched prefill == chunked decode, the per-value
 * products equal dot_row) and by the det-num pieces they compose.
 */
#ifndef IRIS_ORACLE_LAYERS_H
#define IRIS_ORACLE_LAYERS_H

#include <stddef.h>
#include <stdint.h>

/* crates/inference/kernels/src/tensor.rs:437-520 linear_slab_from_source over a
 * Q8Matrix: out[t][r] = q8::dot_row(in[t], W[r]). Rows are shared out over
 * `threads` OpenMP threads (1 = serial). */
int orc_linear_q8(const int32_t* in, size_t tokens, size_t cols, const uint8_t* w, size_t rows,
                  int32_t* out, int threads);

/* tensor.rs:201-323 Matrix (Q16.16 values) product: out[t][r] = dot_bits(in[t], W[r]). */
int orc_linear_i32(const int32_t* in, size_t tokens, size_t cols, const int32_t* w, size_t rows,
                   int32_t* out, int threads);

/* crates/inference/kernels/src/mistral/layer.rs:24-40 LayerParams + LayerMatrices */
typedef struct {
    uint32_t hidden, ffn, heads, kv_heads, head_dim;
    int64_t norm_eps;
    uint32_t attention_scale_q32;
    const int64_t* inv_freq; /* head_dim/2 Q32.32 angles per position */
    uint32_t max_positions;
    const int32_t* norm_attention;
    const int32_t* norm_feed_forward;
    const uint8_t *w_q, *w_k, *w_v, *w_o, *w_gate, *w_up, *w_down;
} orc_mistral_layer;

/* mistral/layer.rs:107-270 layer_rows_and_keys. `k_cache`/`v_cache` hold the
 * keys of positions 0..start (read) and receive this range's own keys at
 * start..start+count (written). out is [count][hidden]. */
int orc_mistral_layer_forward(const orc_mistral_layer* L, const int32_t* x, size_t count, uint32_t start,
                              int32_t* k_cache, int32_t* v_cache, int32_t* out, int threads);

/* orc_mistral_layer_forward for the rows listed in sel (indices into the
 * range, each < count): every row's keys and values go to the caches, as the
 * full forward writes them, but q, attention, W_o and the feed-forward block
 * run only for the listed rows; out is [n_sel][hidden], each row equal to the
 * full forward's row of that index. */
int orc_mistral_layer_rows(const orc_mistral_layer* L, const int32_t* x, size_t count, uint32_t start,
                           int32_t* k_cache, int32_t* v_cache, const uint32_t* sel, size_t n_sel, int32_t* out,
                           int threads);

/* raster-stages/prefill-range/src/input.rs:91-190 LayerParams + TransformerLayer */
typedef struct {
    uint32_t hidden, ffn, heads, kv_heads, head_dim, ple_width;
    uint32_t sliding_window; /* 0 = full attention */
    int32_t layer_scalar;    /* 0 = absent */
    int64_t norm_eps;
    int64_t rope_base;
    uint32_t rotary_dim, rope_freq_base_dim;
    const int32_t *norm_input, *norm_post_attn, *norm_pre_ffw, *norm_post_ffw;
    const int32_t *q_norm, *k_norm, *ple_post_norm;
    const uint8_t *w_q, *w_k, *w_v, *w_o, *w_gate, *w_up, *w_down;
    const int32_t* ple_input_gate;       /* [ple_width][hidden] Q16.16 */
    const int32_t* ple_layer_projection; /* [hidden][ple_width] Q16.16 */
} orc_gemma_layer;

/* crates/inference/kernels/src/prefill_range.rs:307-958 layer_rows_and_keys.
 * Own keys go to own_k/own_v at start..start+count. Attention reads
 * attend_k/attend_v (the layer's own cache, or its KV donor's), positions
 * 0..start+count. ple_rows is [count][ple_width]. */
int orc_gemma_layer_forward(const orc_gemma_layer* L, const int32_t* x, size_t count, uint32_t start,
                            int32_t* own_k, int32_t* own_v, const int32_t* attend_k,
                            const int32_t* attend_v, const int32_t* ple_rows, int32_t* out,
                            int threads);

/* crates/inference/direct/src/view_kernels.rs:59-99 run_ple_prepare_view for
 * one token and one layer. `projection` is the layer's [ple_width][hidden]
 * rows of per_layer_model_projection; `emb_row` is the token's Q8_0 row of
 * embed_tokens_per_layer and `emb_start` the layer's first column. */
int orc_gemma_ple_prepare(const int32_t* embedded_row, size_t hidden, const int32_t* projection,
                          size_t ple_width, int32_t projection_scalar, const int32_t* norm_weights,
                          int64_t norm_eps, const uint8_t* emb_row, size_t emb_start,
                          int32_t embedding_scale, int32_t input_scale, int32_t* out);

/* view_kernels.rs:203-235 score_prefill_logits_view: rms_norm of the last row
 * (copied), then softcap(dot_row(x, head[id]), cap) for every id. */
int orc_head_logits(const int32_t* last_row, size_t hidden, const int32_t* norm, int64_t eps,
                    int32_t softcap, const uint8_t* head, size_t vocab, int32_t* logits, int threads);

/* crates/inference/direct/src/model.rs:316-330 scaled_embedding_row: the
 * dequantized row, then mul_sat by embedding_scale when `scaled` (gemma-dense
 * only; a zero scale gives a zero row). */
int orc_embedding_row(const uint8_t* emb_row, size_t hidden, int scaled, int32_t embedding_scale, int32_t* out);

/* mistral.rs:72-77 silu of n values (out[i] = silu(x[i])). */
int orc_silu_many(const int32_t* x, size_t n, int32_t* out, int threads);

#endif
