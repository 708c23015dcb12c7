/*
 * CPU oracle, layer level. TEST INFRASTRUCTURE ONLY (see layers.h).
 */
#include "layers.h"

#include <stdlib.h>
#include <string.h>

#include "detnum.h"

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_EBAD (-1)
#define ORC_ENOMEM (-2)
#define ORC_ESCALE (-3)

static size_t q8_row_bytes(size_t cols) { return cols / DN_Q8_BLOCK * DN_Q8_BLOCK_BYTES; }

int orc_linear_q8(const int32_t* in, size_t tokens, size_t cols, const uint8_t* w, size_t rows,
                  int32_t* out, int threads) {
    if (cols == 0 || cols % DN_Q8_BLOCK) return ORC_EBAD;
    size_t rb = q8_row_bytes(cols);
    int bad = 0;
    long long total = (long long)tokens * (long long)rows;
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1) reduction(| : bad)
    for (long long i = 0; i < total; i++) {
        size_t r = (size_t)(i % (long long)rows);
        size_t t = (size_t)(i / (long long)rows);
        int32_t v;
        if (dn_q8_dot_row(in + t * cols, w + r * rb, cols, &v)) { bad = 1; v = 0; }
        out[t * rows + r] = v;
    }
    return bad ? ORC_ESCALE : 0;
}

int orc_linear_i32(const int32_t* in, size_t tokens, size_t cols, const int32_t* w, size_t rows,
                   int32_t* out, int threads) {
    long long total = (long long)tokens * (long long)rows;
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
    for (long long i = 0; i < total; i++) {
        size_t r = (size_t)(i % (long long)rows);
        size_t t = (size_t)(i / (long long)rows);
        out[t * rows + r] = dn_dot_bits(in + t * cols, w + r * cols, cols);
    }
    return 0;
}

/* mistral/layer.rs:274-318 attention_context for one query row. */
static void mistral_attention_context(const orc_mistral_layer* L, const int32_t* q, size_t position,
                                      const int32_t* k_cache, const int32_t* v_cache, int32_t* ctx,
                                      int32_t* logits, int64_t* scratch, int32_t* weights) {
    size_t heads = L->heads, hd = L->head_dim, kvw = (size_t)L->kv_heads * hd;
    size_t group = heads / L->kv_heads;
    size_t visible = position + 1;
    for (size_t h = 0; h < heads; h++) {
        size_t kv = h / group;
        const int32_t* qh = q + h * hd;
        for (size_t j = 0; j < visible; j++)
            logits[j] = dn_scaled_score(qh, k_cache + j * kvw + kv * hd, hd, L->attention_scale_q32);
        dn_attention_softmax(logits, visible, scratch, weights);
        for (size_t d = 0; d < hd; d++) {
            uint64_t acc = 0; /* wrapping mac_bits */
            for (size_t j = 0; j < visible; j++)
                acc += (uint64_t)((int64_t)weights[j] * (int64_t)v_cache[j * kvw + kv * hd + d]);
            ctx[h * hd + d] = dn_requantize((int64_t)acc);
        }
    }
}

/* mistral/layer.rs:144-162: rms_norm(norm_attention) of every row, then the
 * range's own keys and values into the caches at start.., k rotated at its
 * absolute position (:163-185). */
static int mistral_keys(const orc_mistral_layer* L, const int32_t* x, size_t count, uint32_t start,
                        int32_t* normed, int32_t* k_cache, int32_t* v_cache, int threads) {
    size_t H = L->hidden, hd = L->head_dim, kvw = (size_t)L->kv_heads * hd;
    int rc;
    memcpy(normed, x, count * H * 4);
    for (size_t i = 0; i < count; i++) dn_rms_norm(normed + i * H, L->norm_attention, H, L->norm_eps);
    if ((rc = orc_linear_q8(normed, count, H, L->w_k, kvw, k_cache + (size_t)start * kvw, threads))) return rc;
    if ((rc = orc_linear_q8(normed, count, H, L->w_v, kvw, v_cache + (size_t)start * kvw, threads))) return rc;
    for (size_t i = 0; i < count; i++) {
        int32_t* kr = k_cache + ((size_t)start + i) * kvw;
        for (size_t h = 0; h < L->kv_heads; h++)
            dn_rotate_consecutive_pairs(kr + h * hd, hd, L->inv_freq, hd / 2, start + (uint32_t)i);
    }
    return 0;
}

/* The rest of mistral/layer.rs:149-267 for n rows whose inputs are x (and
 * their normed copies), at absolute positions pos[i], over caches that hold
 * every key up to each row's position: q (rotated), attention (:229-236), W_o
 * + x (:237-242), rms_norm(norm_feed_forward), mul(silu(gate), up), W_down +
 * attended (:243-267). */
static int mistral_rows(const orc_mistral_layer* L, const int32_t* x, const int32_t* normed, const uint32_t* pos,
                        size_t n, const int32_t* k_cache, const int32_t* v_cache, int32_t* out, int threads) {
    size_t H = L->hidden, F = L->ffn, hd = L->head_dim;
    size_t qw = (size_t)L->heads * hd;
    int rc = 0;
    int32_t* q = malloc(n * qw * 4);
    int32_t* ctx = malloc(n * qw * 4);
    int32_t* attended = malloc(n * H * 4);
    int32_t* ffin = malloc(n * H * 4);
    int32_t* gate = malloc(n * F * 4);
    int32_t* up = malloc(n * F * 4);
    if (!q || !ctx || !attended || !ffin || !gate || !up) { rc = ORC_ENOMEM; goto done; }
    if ((rc = orc_linear_q8(normed, n, H, L->w_q, qw, q, threads))) goto done;
    for (size_t i = 0; i < n; i++)
        for (size_t h = 0; h < L->heads; h++)
            dn_rotate_consecutive_pairs(q + i * qw + h * hd, hd, L->inv_freq, hd / 2, pos[i]);
    {
        size_t end = 0;
        for (size_t i = 0; i < n; i++) end = pos[i] + 1 > end ? pos[i] + 1 : end;
        int rc2 = 0;
#pragma omp parallel num_threads(threads > 0 ? threads : 1) reduction(| : rc2)
        {
            int32_t* logits = malloc(end * 4);
            int64_t* scratch = malloc(end * 8);
            int32_t* weights = malloc(end * 4);
            if (!logits || !scratch || !weights) rc2 = 1;
            else {
#pragma omp for schedule(dynamic)
                for (long long i = 0; i < (long long)n; i++)
                    mistral_attention_context(L, q + i * qw, pos[i], k_cache, v_cache, ctx + i * qw, logits, scratch,
                                              weights);
            }
            free(logits); free(scratch); free(weights);
        }
        if (rc2) { rc = ORC_ENOMEM; goto done; }
    }
    if ((rc = orc_linear_q8(ctx, n, qw, L->w_o, H, attended, threads))) goto done;
    for (size_t i = 0; i < n * H; i++) attended[i] = dn_add_sat(attended[i], x[i]);
    memcpy(ffin, attended, n * H * 4);
    for (size_t i = 0; i < n; i++) dn_rms_norm(ffin + i * H, L->norm_feed_forward, H, L->norm_eps);
    if ((rc = orc_linear_q8(ffin, n, H, L->w_gate, F, gate, threads))) goto done;
    if ((rc = orc_linear_q8(ffin, n, H, L->w_up, F, up, threads))) goto done;
    for (size_t i = 0; i < n * F; i++) gate[i] = dn_mul_sat(dn_silu(gate[i]), up[i]);
    if ((rc = orc_linear_q8(gate, n, F, L->w_down, H, out, threads))) goto done;
    for (size_t i = 0; i < n * H; i++) out[i] = dn_add_sat(out[i], attended[i]);
done:
    free(q); free(ctx); free(attended); free(ffin); free(gate); free(up);
    return rc;
}

static int mistral_check(const orc_mistral_layer* L) {
    if (!L->hidden || !L->ffn || !L->heads || !L->kv_heads || !L->head_dim || L->heads % L->kv_heads ||
        L->head_dim % 2)
        return ORC_EBAD;
    return 0;
}

int orc_mistral_layer_forward(const orc_mistral_layer* L, const int32_t* x, size_t count, uint32_t start,
                              int32_t* k_cache, int32_t* v_cache, int32_t* out, int threads) {
    if (mistral_check(L)) return ORC_EBAD;
    if (count == 0) return 0;
    if ((uint64_t)start + count > L->max_positions) return ORC_EBAD; /* layer.rs:116-123 */
    int32_t* normed = malloc(count * L->hidden * 4);
    uint32_t* pos = malloc(count * 4);
    int rc = normed && pos ? 0 : ORC_ENOMEM;
    for (size_t i = 0; rc == 0 && i < count; i++) pos[i] = start + (uint32_t)i;
    if (rc == 0) rc = mistral_keys(L, x, count, start, normed, k_cache, v_cache, threads);
    if (rc == 0) rc = mistral_rows(L, x, normed, pos, count, k_cache, v_cache, out, threads);
    free(normed);
    free(pos);
    return rc;
}

int orc_mistral_layer_rows(const orc_mistral_layer* L, const int32_t* x, size_t count, uint32_t start,
                           int32_t* k_cache, int32_t* v_cache, const uint32_t* sel, size_t n_sel, int32_t* out,
                           int threads) {
    if (mistral_check(L)) return ORC_EBAD;
    if (count == 0 || n_sel == 0) return 0;
    if ((uint64_t)start + count > L->max_positions) return ORC_EBAD;
    size_t H = L->hidden;
    for (size_t i = 0; i < n_sel; i++)
        if (sel[i] >= count) return ORC_EBAD;
    int32_t* normed = malloc(count * H * 4);
    int32_t* xs = malloc(n_sel * H * 4);
    int32_t* ns = malloc(n_sel * H * 4);
    uint32_t* pos = malloc(n_sel * 4);
    int rc = normed && xs && ns && pos ? 0 : ORC_ENOMEM;
    if (rc == 0) rc = mistral_keys(L, x, count, start, normed, k_cache, v_cache, threads);
    for (size_t i = 0; rc == 0 && i < n_sel; i++) {
        memcpy(xs + i * H, x + (size_t)sel[i] * H, H * 4);
        memcpy(ns + i * H, normed + (size_t)sel[i] * H, H * 4);
        pos[i] = start + sel[i];
    }
    if (rc == 0) rc = mistral_rows(L, xs, ns, pos, n_sel, k_cache, v_cache, out, threads);
    free(normed); free(xs); free(ns); free(pos);
    return rc;
}

/* prefill_range.rs:864-877 */
static uint32_t window_start(uint32_t query_position, uint32_t sliding_window) {
    if (sliding_window == 0) return 0;
    uint64_t p1 = (uint64_t)query_position + 1;
    return p1 > sliding_window ? (uint32_t)(p1 - sliding_window) : 0;
}

/* prefill_range.rs:755-845 attention_context (Gemma): unscaled dot_bits
 * scores over the window, softmax per head, weighted values. */
static void gemma_attention_context(const orc_gemma_layer* L, const int32_t* q, uint32_t position,
                                    const int32_t* k_cache, const int32_t* v_cache, int32_t* ctx,
                                    int32_t* logits, int64_t* scratch, int32_t* weights) {
    size_t heads = L->heads, hd = L->head_dim, kvw = (size_t)L->kv_heads * hd;
    size_t group = heads / L->kv_heads;
    uint32_t ws = window_start(position, L->sliding_window);
    size_t n = (size_t)(position - ws) + 1;
    for (size_t h = 0; h < heads; h++) {
        size_t kv = h / group;
        for (size_t j = 0; j < n; j++)
            logits[j] = dn_dot_bits(q + h * hd, k_cache + ((size_t)ws + j) * kvw + kv * hd, hd);
        dn_attention_softmax(logits, n, scratch, weights);
        for (size_t d = 0; d < hd; d++) {
            uint64_t acc = 0;
            for (size_t j = 0; j < n; j++)
                acc += (uint64_t)((int64_t)weights[j] * (int64_t)v_cache[((size_t)ws + j) * kvw + kv * hd + d]);
            ctx[h * hd + d] = dn_requantize((int64_t)acc);
        }
    }
}

int orc_gemma_layer_forward(const orc_gemma_layer* L, const int32_t* x, size_t count, uint32_t start,
                            int32_t* own_k, int32_t* own_v, const int32_t* attend_k,
                            const int32_t* attend_v, const int32_t* ple_rows, int32_t* out,
                            int threads) {
    size_t H = L->hidden, F = L->ffn, hd = L->head_dim, P = L->ple_width;
    size_t qw = (size_t)L->heads * hd, kvw = (size_t)L->kv_heads * hd;
    /* prefill_range.rs:394-466 validate_layer_params (the checks that bear on values) */
    if (!H || !F || !L->heads || !L->kv_heads || !hd || L->heads % L->kv_heads) return ORC_EBAD;
    if (L->rotary_dim % 2 || L->rotary_dim > hd) return ORC_EBAD;
    if (L->rotary_dim > 0 && (L->rope_freq_base_dim < 2 || L->rope_freq_base_dim % 2 || L->rope_base <= 0))
        return ORC_EBAD;
    if (count == 0) return 0;
    int rc = 0;
    int32_t* normed = malloc(count * H * 4);
    int32_t* q = malloc(count * qw * 4);
    int32_t* ctx = malloc(count * qw * 4);
    int32_t* resid = malloc(count * H * 4);
    int32_t* ffin = malloc(count * H * 4);
    int32_t* gate = malloc(count * F * 4);
    int32_t* up = malloc(count * F * 4);
    int32_t* xs = malloc(count * H * 4);
    int32_t* pg = malloc(count * (P ? P : 1) * 4);
    if (!normed || !q || !ctx || !resid || !ffin || !gate || !up || !xs || !pg) { rc = ORC_ENOMEM; goto done; }
    /* project_tokens :497-579 */
    memcpy(normed, x, count * H * 4);
    for (size_t i = 0; i < count; i++) dn_rms_norm(normed + i * H, L->norm_input, H, L->norm_eps);
    int32_t* kown = own_k + (size_t)start * kvw;
    int32_t* vown = own_v + (size_t)start * kvw;
    if ((rc = orc_linear_q8(normed, count, H, L->w_q, qw, q, threads))) goto done;
    if ((rc = orc_linear_q8(normed, count, H, L->w_k, kvw, kown, threads))) goto done;
    if ((rc = orc_linear_q8(normed, count, H, L->w_v, kvw, vown, threads))) goto done;
    /* finish_qkv_row :607-629, apply_rope :631-647 */
    for (size_t i = 0; i < count; i++) {
        size_t pos = (size_t)start + i;
        for (size_t h = 0; h < L->heads; h++) {
            int32_t* head = q + i * qw + h * hd;
            dn_rms_norm(head, L->q_norm, hd, L->norm_eps);
            dn_rope_rotate_pairs(head, hd, L->rotary_dim, L->rope_freq_base_dim, L->rope_base, pos);
        }
        for (size_t h = 0; h < L->kv_heads; h++) {
            int32_t* head = kown + i * kvw + h * hd;
            dn_rms_norm(head, L->k_norm, hd, L->norm_eps);
            dn_rope_rotate_pairs(head, hd, L->rotary_dim, L->rope_freq_base_dim, L->rope_base, pos);
        }
        for (size_t h = 0; h < L->kv_heads; h++) dn_value_rms_norm(vown + i * kvw + h * hd, hd, L->norm_eps);
    }
    /* attend_chunk :692-740 */
    {
        size_t end = (size_t)start + count;
        int rc2 = 0;
#pragma omp parallel num_threads(threads > 0 ? threads : 1) reduction(| : rc2)
        {
            int32_t* logits = malloc(end * 4);
            int64_t* scratch = malloc(end * 8);
            int32_t* weights = malloc(end * 4);
            if (!logits || !scratch || !weights) rc2 = 1;
            else {
#pragma omp for schedule(dynamic)
                for (long long i = 0; i < (long long)count; i++)
                    gemma_attention_context(L, q + i * qw, start + (uint32_t)i, attend_k, attend_v,
                                            ctx + i * qw, logits, scratch, weights);
            }
            free(logits); free(scratch); free(weights);
        }
        if (rc2) { rc = ORC_ENOMEM; goto done; }
    }
    /* attn_residual :879-892: rms_norm(post_attn) then + residual */
    if ((rc = orc_linear_q8(ctx, count, qw, L->w_o, H, resid, threads))) goto done;
    for (size_t i = 0; i < count; i++) {
        dn_rms_norm(resid + i * H, L->norm_post_attn, H, L->norm_eps);
        for (size_t c = 0; c < H; c++) resid[i * H + c] = dn_add_sat(resid[i * H + c], x[i * H + c]);
    }
    /* pre_ff_norm :894-903 */
    memcpy(ffin, resid, count * H * 4);
    for (size_t i = 0; i < count; i++) dn_rms_norm(ffin + i * H, L->norm_pre_ffw, H, L->norm_eps);
    if ((rc = orc_linear_q8(ffin, count, H, L->w_gate, F, gate, threads))) goto done;
    if ((rc = orc_linear_q8(ffin, count, H, L->w_up, F, up, threads))) goto done;
    /* gelu_mul :905-913 */
    for (size_t i = 0; i < count * F; i++) gate[i] = dn_mul_sat(dn_gelu(gate[i]), up[i]);
    if ((rc = orc_linear_q8(gate, count, F, L->w_down, H, xs, threads))) goto done;
    /* finish_mlp :915-929 */
    for (size_t i = 0; i < count; i++) {
        dn_rms_norm(xs + i * H, L->norm_post_ffw, H, L->norm_eps);
        for (size_t c = 0; c < H; c++) xs[i * H + c] = dn_add_sat(xs[i * H + c], resid[i * H + c]);
    }
    /* PLE block :723-737, ple_gate_mul :931-944, finish_layer :946-958 */
    if ((rc = orc_linear_i32(xs, count, H, L->ple_input_gate, P, pg, threads))) goto done;
    for (size_t i = 0; i < count * P; i++) pg[i] = dn_mul_sat(dn_gelu(pg[i]), ple_rows[i]);
    if ((rc = orc_linear_i32(pg, count, P, L->ple_layer_projection, H, out, threads))) goto done;
    for (size_t i = 0; i < count; i++) {
        int32_t* o = out + i * H;
        dn_rms_norm(o, L->ple_post_norm, H, L->norm_eps);
        for (size_t c = 0; c < H; c++) o[c] = dn_add_sat(o[c], xs[i * H + c]);
        if (L->layer_scalar != 0)
            for (size_t c = 0; c < H; c++) o[c] = dn_mul_sat(o[c], L->layer_scalar);
    }
done:
    free(normed); free(q); free(ctx); free(resid); free(ffin); free(gate); free(up); free(xs); free(pg);
    return rc;
}

int orc_gemma_ple_prepare(const int32_t* embedded_row, size_t hidden, const int32_t* projection,
                          size_t ple_width, int32_t projection_scalar, const int32_t* norm_weights,
                          int64_t norm_eps, const uint8_t* emb_row, size_t emb_start,
                          int32_t embedding_scale, int32_t input_scale, int32_t* out) {
    if (ple_width == 0 || ple_width % DN_Q8_BLOCK || emb_start % DN_Q8_BLOCK) return ORC_EBAD;
    int32_t* proj = malloc(ple_width * 4);
    if (!proj) return ORC_ENOMEM;
    /* view_kernels.rs:74-77: matvec, scale_row, rms_norm */
    for (size_t r = 0; r < ple_width; r++) proj[r] = dn_dot_bits(projection + r * hidden, embedded_row, hidden);
    for (size_t r = 0; r < ple_width; r++) proj[r] = dn_mul_sat(proj[r], projection_scalar);
    dn_rms_norm(proj, norm_weights, ple_width, norm_eps);
    /* :79-88: dequantized columns, scale, add, scale */
    const uint8_t* cols = emb_row + emb_start / DN_Q8_BLOCK * DN_Q8_BLOCK_BYTES;
    if (dn_q8_dequantize_row(cols, ple_width, out)) { free(proj); return ORC_ESCALE; }
    for (size_t c = 0; c < ple_width; c++) {
        int32_t e = dn_mul_sat(out[c], embedding_scale);
        e = dn_add_sat(e, proj[c]);
        out[c] = dn_mul_sat(e, input_scale);
    }
    free(proj);
    return 0;
}

int orc_head_logits(const int32_t* last_row, size_t hidden, const int32_t* norm, int64_t eps,
                    int32_t softcap, const uint8_t* head, size_t vocab, int32_t* logits, int threads) {
    int32_t* x = malloc(hidden * 4);
    if (!x) return ORC_ENOMEM;
    memcpy(x, last_row, hidden * 4);
    dn_rms_norm(x, norm, hidden, eps);
    int rc = orc_linear_q8(x, 1, hidden, head, vocab, logits, threads);
    /* raster-stages/sequence-check/src/input.rs:429-434 softcap: cap <= 0 passes through */
    if (!rc && softcap > 0)
        for (size_t i = 0; i < vocab; i++) logits[i] = dn_softcap_act(logits[i], softcap);
    free(x);
    return rc;
}

int orc_embedding_row(const uint8_t* emb_row, size_t hidden, int scaled, int32_t embedding_scale, int32_t* out) {
    if (dn_q8_dequantize_row(emb_row, hidden, out)) return ORC_ESCALE;
    if (scaled)
        for (size_t c = 0; c < hidden; c++) out[c] = dn_mul_sat(out[c], embedding_scale);
    return 0;
}

int orc_silu_many(const int32_t* x, size_t n, int32_t* out, int threads) {
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
    for (long long i = 0; i < (long long)n; i++) out[i] = dn_silu(x[i]);
    return 0;
}
