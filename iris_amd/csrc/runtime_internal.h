// Model and session state of the device-resident token loop.
#pragma once

#include <map>
#include <string>
#include <vector>

#include "layer_kernels.h"
#include "q8_internal.h"

struct HostTensor {
    uint64_t rows = 0, cols = 0;
    std::vector<uint8_t> bytes;
};

struct LayerWeights {
    Q8GpuMatrix* wqkv = nullptr;   // q|k|v rows stacked
    Q8GpuMatrix* wo = nullptr;
    Q8GpuMatrix* wgu = nullptr;    // gate/up rows interleaved
    Q8GpuMatrix* wdown = nullptr;
    int32_t* norm_attn = nullptr;  // input_layernorm
    int32_t* norm_ff = nullptr;    // pre_feedforward_layernorm
    uint32_t q_rows = 0, kv_rows = 0, ffn = 0;
    // gemma-dense only
    int32_t* norm_post_attn = nullptr;
    int32_t* norm_post_ffw = nullptr;
    int32_t* norm_post_ple = nullptr;  // post_per_layer_input_norm
    int32_t* q_norm = nullptr;
    int32_t* k_norm = nullptr;
    int32_t* ple_gate = nullptr;       // per_layer_input_gate, Q16.16 [ple][hidden]
    int32_t* ple_proj = nullptr;       // per_layer_projection, Q16.16 [hidden][ple]
    int32_t layer_scalar = 0;          // 0 = absent
    // derived at finalize (model.rs:817-877)
    uint32_t head_dim = 0, rotary_dim = 0, window = 0;
    int32_t kv_source = -1;            // the layer whose cache attention reads
    const int64_t* inv_freq = nullptr; // [rotary_dim / 2]
};

struct IrisModel {
    IrisModelDesc d{};
    std::vector<uint8_t> layer_is_sliding;
    std::vector<LayerWeights> layers;
    // Q8_0 matrices of a layer waiting for the rest of their set.
    std::vector<std::map<std::string, HostTensor>> pending;
    uint8_t* embed_raw = nullptr;   // reference layout, for row lookups
    uint32_t embed_row_bytes = 0;
    // Per token id, 1 = the embedding row (embed_bad) or the PLE row
    // (ple_bad) has a non-finite block scale, refused when the token is
    // embedded; empty when every row's scales are finite.
    std::vector<uint8_t> embed_bad, ple_bad;
    Q8GpuMatrix* head = nullptr;
    int32_t* final_norm = nullptr;
    int64_t* inv_freq = nullptr;
    int32_t head_softcap = 0;   // 0 = uncapped (mistral-dense)
    int32_t embed_scale = 1 << 16;  // mul_sat of each embedded value; 1.0 (exact) for mistral-dense
    // gemma-dense only
    uint8_t* embed_ple = nullptr;        // embed_tokens_per_layer, reference Q8_0 rows
    uint32_t embed_ple_row_bytes = 0;
    int32_t* ple_model_proj = nullptr;   // per_layer_model_projection, Q16.16 [layers*ple][hidden]
    int32_t* ple_proj_norm = nullptr;    // per_layer_projection_norm [ple]
    int64_t* rope_sliding = nullptr;     // frequency ladders of the two layer kinds
    int64_t* rope_full = nullptr;
    uint32_t max_head_dim = 0, max_ffn = 0, max_qkv = 0;
    hipStream_t stream = nullptr;
    bool finalized = false;
};

struct IrisSession {
    IrisModel* model = nullptr;
    uint32_t max_positions = 0, max_rows = 0;
    uint32_t k_pos_stride = 0;  // positions per row of the transposed K cache: max_positions rounded up to 64
    hipStream_t stream = nullptr;
    std::vector<int32_t*> k_cache, v_cache;  // per layer [position][kv_heads*head_dim]
    // Per layer, the positions [kv_lo, kv_hi) its cache holds, as passes and
    // carried keys (iris_session_write_kv) left them; a range over positions
    // start.. needs its attention source's cache to hold what the range's
    // first row sees before `start`.
    std::vector<uint32_t> kv_lo, kv_hi;
    int32_t *x = nullptr, *attended = nullptr, *q = nullptr, *ctx = nullptr, *gated = nullptr;
    int32_t* scores = nullptr;  // one-row attention: attn_scores_ints(heads, k_pos_stride)
    // One-row passes: per-tile sums of squares of x and attended, written by
    // the residual products and read by the norms that follow them.
    int64_t *ssq_x = nullptr, *ssq_att = nullptr;
    bool ssq_x_valid = false;  // the last pass left ssq_x for the head's norm
    // mistral-dense one-row passes: the context and gated rows as digit
    // planes from their producers (act_planes layout), read by the O and
    // down products, and those products' k-split scratch (partial sums,
    // arrival counters zeroed at allocation).
    uint32_t *ctx_planes = nullptr, *gated_planes = nullptr;
    uint8_t *ctx_counts = nullptr, *gated_counts = nullptr;
    int64_t* kpart = nullptr;
    uint32_t* kcount = nullptr;
    // gemma-dense one-row passes carry each post-norm into the next product:
    // the product's row stays in tmp with its sums of squares in ssq_x, to be
    // rms_norm'ed with norm_w, added to res and scaled by scalar (0 = none).
    // After the pass, `pending` says the last layer's post-norm is still
    // carried (for the head).
    struct GemmaCarry {
        bool pending = false;
        const int32_t* norm_w = nullptr;
        int32_t scalar = 0;
        int32_t* res = nullptr;    // the residual row
        int32_t* spare = nullptr;  // the other of x and attended, free
        uint32_t slots = 0;
    } carry;
    bool rope_ready = false;   // the last selection left rope_sc for the next one-row pass
    // gemma-dense only: raw q|k|v rows, a product's rows before their norm,
    // the PLE projections and inputs of every layer, the PLE gate output
    int32_t *qkv = nullptr, *tmp = nullptr, *ple_proj = nullptr, *ple_rows = nullptr, *ple_gated = nullptr;
    // digit planes of a multi-row pass's activations for the MFMA products
    int8_t* planes = nullptr;        // gemm_planes_bytes(widest product input, max_rows)
    // multi-row passes: the gated rows' planes and counts, written by the
    // gate/up product for the down product
    int8_t* gated_gemm_planes = nullptr;   // gemm_planes_bytes(max_ffn, max_rows)
    int32_t* gated_gemm_limbs = nullptr;   // gemm_limb_ints(max_ffn, max_rows)
    const int32_t* silu_tab = nullptr;  // mistral-dense: the device's silu table (not owned)
    int32_t* token_limbs = nullptr;  // [2][max_rows]: digit counts, norm scales
    int32_t *logits = nullptr, *ids = nullptr, *tokens = nullptr;
    int32_t *d_pos = nullptr, *d_step = nullptr;
    int32_t* logits_keep = nullptr;
    size_t logits_keep_cap = 0;
    bool keep_logits = false;
    uint64_t* sel_partial = nullptr;
    int64_t* rope_sc = nullptr;      // mistral-dense: [max_rows][head_dim/2][sin, cos] of the pass's positions
    // multi-row attention digit planes (null for single-row sessions)
    AttnPlanes attn_planes{};
    // per-layer checkpoint staging, made on the first checkpointing pass
    int32_t* ckpt_dev = nullptr;              // [layers][max_rows][hidden]
    uint8_t* ckpt_host = nullptr;             // pinned, same shape
    hipStream_t copy_stream = nullptr;
    std::vector<hipEvent_t> ckpt_events;      // [2][layers]: rows copied on the device, on the host
    hipGraphExec_t graph_exec = nullptr;
    bool graph_keep_logits = false;
};

// SHA-256 (FIPS 180-4) of `len` bytes into out[32].
void iris_sha256(const uint8_t* data, size_t len, uint8_t out[32]);
