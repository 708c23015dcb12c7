// The device-resident token loop: model upload, sessions with a KV cache,
// greedy generation and the teacher-forced per-layer pass.
//
// A mistral-dense layer (crates/inference/kernels/src/mistral/layer.rs:107-270)
// runs as five launches:
//   1. q|k|v product, rms_norm(norm_attention) fused in front, RoPE and the
//      K/V cache store fused behind;
//   2. attention over the cache;
//   3. W_o product + residual;
//   4. gate/up product (rows interleaved at upload), rms_norm(norm_feed_forward)
//      in front, mul(silu(gate), up) behind;
//   5. W_down product + residual.
// The head is the final-norm product (softcap behind for gemma), and one
// kernel selects the first maximum and embeds the next row. Positions and
// the step counter live in device memory, so a decode pass is the same
// launch sequence every time and is captured once as a HIP graph.
#include <link.h>

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <thread>
#include <vector>

#include "layer_kernels.h"
#include "q8_internal.h"
#include "runtime_internal.h"

namespace {

constexpr const char* PREFIX = "model.language_model.";

bool starts_with(const std::string& s, const std::string& p) { return s.compare(0, p.size(), p) == 0; }

int layer_of(const std::string& name, std::string* suffix) {
    const std::string lp = std::string(PREFIX) + "layers.";
    if (!starts_with(name, lp)) return -1;
    size_t dot = name.find('.', lp.size());
    if (dot == std::string::npos) return -1;
    int layer = std::atoi(name.substr(lp.size(), dot - lp.size()).c_str());
    *suffix = name.substr(dot + 1);
    return layer;
}

#define RT_CHECK(expr)                  \
    do {                                \
        int rc_ = (int)(expr);          \
        if (rc_ != 0) return rc_;       \
    } while (0)

// The rows of a Q8_0 table (rows of row_bytes) holding a block with a
// non-finite f16 scale (exponent 0x1f), which dequantize_row refuses
// (q8.rs:45-47, 76-92): one flag per row, or none at all when every scale
// is finite.
std::vector<uint8_t> q8_rows_refused(const uint8_t* raw, size_t rows, size_t row_bytes) {
    std::vector<uint8_t> bad;
    for (size_t r = 0; r < rows; r++)
        for (size_t b = 0; b < row_bytes / 34; b++)
            if ((raw[r * row_bytes + b * 34 + 1] & 0x7c) == 0x7c) {
                if (bad.empty()) bad.assign(rows, 0);
                bad[r] = 1;
                break;
            }
    return bad;
}

template <class T>
hipError_t dev_alloc_copy(T** dst, const void* src, size_t bytes) {
    hipError_t st = hipMalloc((void**)dst, bytes ? bytes : 4);
    if (st == hipSuccess && bytes) st = hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice);
    return st;
}

}  // namespace

// Multi-row passes hand the products the session's digit-plane work space,
// which routes row-scale matrices through the MFMA GEMM.
static inline void with_gemm_space(GemvArgs& g, const IrisSession* s, uint32_t rows) {
    if (rows > 1) {
        g.planes = s->planes;
        g.token_limbs = s->token_limbs;
    }
}

// ---------------------------------------------------------------- model

int iris_model_build_layer_if_complete(IrisModel* m, uint32_t l) {
    LayerWeights& L = m->layers[l];
    auto& p = m->pending[l];
    const uint32_t H = m->d.hidden;
    auto have = [&](const char* k) { return p.count(k) != 0; };
    if (!L.wqkv && have("self_attn.q_proj.weight") && have("self_attn.k_proj.weight") &&
        have("self_attn.v_proj.weight")) {
        const HostTensor& q = p["self_attn.q_proj.weight"];
        const HostTensor& k = p["self_attn.k_proj.weight"];
        const HostTensor& v = p["self_attn.v_proj.weight"];
        if (q.cols != H || k.cols != H || v.cols != H || k.rows != v.rows) return IRIS_E_INVALID;
        const uint8_t* parts[3] = {q.bytes.data(), k.bytes.data(), v.bytes.data()};
        uint32_t rows[3] = {(uint32_t)q.rows, (uint32_t)k.rows, (uint32_t)v.rows};
        RT_CHECK(iris_q8_upload_parts(parts, rows, 3, H, 0, &L.wqkv, m->stream));
        L.q_rows = rows[0];
        L.kv_rows = rows[1];
        p.erase("self_attn.q_proj.weight");
        p.erase("self_attn.k_proj.weight");
        p.erase("self_attn.v_proj.weight");
    }
    if (!L.wgu && have("mlp.gate_proj.weight") && have("mlp.up_proj.weight")) {
        const HostTensor& g = p["mlp.gate_proj.weight"];
        const HostTensor& u = p["mlp.up_proj.weight"];
        if (g.cols != H || u.cols != H || g.rows != u.rows) return IRIS_E_INVALID;
        const uint8_t* parts[2] = {g.bytes.data(), u.bytes.data()};
        uint32_t rows[2] = {(uint32_t)g.rows, (uint32_t)u.rows};
        RT_CHECK(iris_q8_upload_parts(parts, rows, 2, H, 1, &L.wgu, m->stream));
        L.ffn = rows[0];
        p.erase("mlp.gate_proj.weight");
        p.erase("mlp.up_proj.weight");
    }
    for (auto name : {"self_attn.o_proj.weight", "mlp.down_proj.weight"}) {
        if (!have(name)) continue;
        const HostTensor& t = p[name];
        Q8GpuMatrix** dst = std::strcmp(name, "self_attn.o_proj.weight") == 0 ? &L.wo : &L.wdown;
        const uint8_t* part = t.bytes.data();
        uint32_t rows = (uint32_t)t.rows;
        RT_CHECK(iris_q8_upload_parts(&part, &rows, 1, (uint32_t)t.cols, 0, dst, m->stream));
        p.erase(name);
    }
    return (int)hipStreamSynchronize(m->stream);
}

extern "C" {

int iris_model_create(const IrisModelDesc* desc, IrisModel** out) {
    if (!desc || !out) return IRIS_E_INVALID;
    *out = nullptr;
    const IrisModelDesc& d = *desc;
    const bool gemma = d.family == IRIS_FAMILY_GEMMA_DENSE;
    if (d.family != IRIS_FAMILY_MISTRAL_DENSE && !gemma) return IRIS_E_INVALID;
    if (!d.hidden || !d.vocab || d.hidden % 32 || d.norm_eps < 0) return IRIS_E_INVALID;
    // A model of no layers is embedding, final norm, head and selection
    // (executor.rs:293-360 over an empty layer list; build_ple_params,
    // model.rs:679-686, makes no PLE inputs): the attention, FFN and PLE
    // shape fields are not read.
    if (d.layers) {
        if (!d.heads || !d.kv_heads || !d.head_dim || !d.ffn) return IRIS_E_INVALID;
        if (d.heads % d.kv_heads || d.head_dim % 4 || d.head_dim > ATTN_MAX_HEAD_DIM) return IRIS_E_INVALID;
    }
    if (gemma && d.layers) {
        const uint32_t ghd = d.global_head_dim ? d.global_head_dim : d.head_dim;
        // The PLE segments are whole Q8_0 blocks of embed_tokens_per_layer.
        if (ghd % 4 || ghd > ATTN_MAX_HEAD_DIM || !d.ple_width || d.ple_width % 32 || d.ple_width > GEMMA_MAX_PLE)
            return IRIS_E_INVALID;
        if (d.num_kv_shared_layers > d.layers || d.partial_rotary_q16 < 0 || d.partial_rotary_q16 > 65536)
            return IRIS_E_INVALID;
    }
    IrisModel* m = new (std::nothrow) IrisModel();
    if (!m) return IRIS_E_NOMEM;
    m->d = d;
    if (gemma) {
        if (!m->d.global_head_dim) m->d.global_head_dim = d.head_dim;
        m->head_softcap = d.final_logit_softcap;
        m->embed_scale = d.embedding_scale;
    }
    m->layer_is_sliding.assign(d.layers, 0);
    if (d.layer_is_sliding) m->layer_is_sliding.assign(d.layer_is_sliding, d.layer_is_sliding + d.layers);
    m->d.layer_is_sliding = nullptr;
    m->layers.resize(d.layers);
    m->pending.resize(d.layers);
    hipError_t st = hipStreamCreate(&m->stream);
    if (st != hipSuccess) {
        delete m;
        return (int)st;
    }
    *out = m;
    return 0;
}

int iris_model_set_tensor(IrisModel* m, const char* cname, int32_t width, const void* data, uint64_t rows,
                          uint64_t cols) {
    if (!m || !cname || !data || m->finalized) return m && m->finalized ? IRIS_E_STATE : IRIS_E_INVALID;
    const std::string name(cname);
    size_t bytes;
    if (width == 8) {
        if (cols == 0 || cols % 32) return IRIS_E_INVALID;
        bytes = rows * (cols / 32) * 34;
    } else if (width == 32) {
        bytes = rows * cols * 4;
    } else if (width == 64) {
        bytes = rows * cols * 8;
    } else {
        return IRIS_E_INVALID;
    }
    std::string suffix;
    const int layer = layer_of(name, &suffix);
    const IrisModelDesc& d = m->d;
    if (layer >= 0) {
        if ((uint32_t)layer >= d.layers) return IRIS_E_INVALID;
        LayerWeights& L = m->layers[layer];
        if (width == 32) {
            const bool gemma = d.family == IRIS_FAMILY_GEMMA_DENSE;
            const uint32_t hd = m->layer_is_sliding[layer] ? d.head_dim : d.global_head_dim;
            struct {
                const char* name;
                int32_t** dst;
                uint64_t count;
                bool gemma_only;
            } vecs[] = {
                {"input_layernorm.weight", &L.norm_attn, d.hidden, false},
                {"pre_feedforward_layernorm.weight", &L.norm_ff, d.hidden, false},
                {"post_attention_layernorm.weight", &L.norm_post_attn, d.hidden, true},
                {"post_feedforward_layernorm.weight", &L.norm_post_ffw, d.hidden, true},
                {"post_per_layer_input_norm.weight", &L.norm_post_ple, d.hidden, true},
                {"self_attn.q_norm.weight", &L.q_norm, hd, true},
                {"self_attn.k_norm.weight", &L.k_norm, hd, true},
                {"per_layer_input_gate.weight", &L.ple_gate, (uint64_t)d.ple_width * d.hidden, true},
                {"per_layer_projection.weight", &L.ple_proj, (uint64_t)d.hidden * d.ple_width, true},
            };
            for (auto& v : vecs) {
                if (suffix != v.name || (v.gemma_only && !gemma)) continue;
                if (rows * cols != v.count) return IRIS_E_INVALID;
                if (*v.dst) return IRIS_E_STATE;
                RT_CHECK(dev_alloc_copy(v.dst, data, bytes));
                return 0;
            }
            if (gemma && suffix == "layer_scalar") {
                if (rows * cols != 1) return IRIS_E_INVALID;
                L.layer_scalar = *(const int32_t*)data;
            }
            return 0;
        }
        if (width != 8) return 0;  // tensors the family does not read are ignored
        HostTensor t;
        t.rows = rows;
        t.cols = cols;
        try {
            t.bytes.assign((const uint8_t*)data, (const uint8_t*)data + bytes);
        } catch (...) {
            return IRIS_E_NOMEM;
        }
        m->pending[layer][suffix] = std::move(t);
        return iris_model_build_layer_if_complete(m, (uint32_t)layer);
    }
    if (name == std::string(PREFIX) + "embed_tokens.weight") {
        if (width != 8 || rows != d.vocab || cols != d.hidden) return IRIS_E_INVALID;
        // A row with a non-finite scale is refused when its token is
        // embedded (model.rs:316-330), as the reference's lazy dequantize
        // does; a tied head reads every row for every logit, so there the
        // upload refuses it.
        m->embed_bad = q8_rows_refused((const uint8_t*)data, rows, cols / 32 * 34);
        RT_CHECK(dev_alloc_copy(&m->embed_raw, data, bytes));
        m->embed_row_bytes = (uint32_t)(cols / 32 * 34);
        if (d.tied_head) {
            const uint8_t* part = (const uint8_t*)data;
            uint32_t r = (uint32_t)rows;
            RT_CHECK(iris_q8_upload_parts(&part, &r, 1, (uint32_t)cols, 0, &m->head, m->stream));
        }
        return (int)hipStreamSynchronize(m->stream);
    }
    if (name == std::string(PREFIX) + "lm_head.weight") {
        if (d.tied_head) return 0;
        if (width != 8 || rows != d.vocab || cols != d.hidden) return IRIS_E_INVALID;
        const uint8_t* part = (const uint8_t*)data;
        uint32_t r = (uint32_t)rows;
        RT_CHECK(iris_q8_upload_parts(&part, &r, 1, (uint32_t)cols, 0, &m->head, m->stream));
        return (int)hipStreamSynchronize(m->stream);
    }
    if (name == std::string(PREFIX) + "norm.weight") {
        if (width != 32 || rows * cols != d.hidden) return IRIS_E_INVALID;
        RT_CHECK(dev_alloc_copy(&m->final_norm, data, bytes));
        return 0;
    }
    if (d.family == IRIS_FAMILY_GEMMA_DENSE) {
        const uint64_t lp = (uint64_t)d.layers * d.ple_width;
        if (name == std::string(PREFIX) + "embed_tokens_per_layer.weight") {
            if (width != 8 || rows != d.vocab || cols != lp) return IRIS_E_INVALID;
            m->ple_bad = q8_rows_refused((const uint8_t*)data, rows, cols / 32 * 34);
            RT_CHECK(dev_alloc_copy(&m->embed_ple, data, bytes));
            m->embed_ple_row_bytes = (uint32_t)(cols / 32 * 34);
            return 0;
        }
        if (name == std::string(PREFIX) + "per_layer_model_projection.weight") {
            if (width != 32 || rows * cols != lp * d.hidden) return IRIS_E_INVALID;
            RT_CHECK(dev_alloc_copy(&m->ple_model_proj, data, bytes));
            return 0;
        }
        if (name == std::string(PREFIX) + "per_layer_projection_norm.weight") {
            if (width != 32 || rows * cols != d.ple_width) return IRIS_E_INVALID;
            RT_CHECK(dev_alloc_copy(&m->ple_proj_norm, data, bytes));
            return 0;
        }
    }
    if (name == "rope_inverse_frequencies") {
        if (width != 64 || rows * cols != d.head_dim / 2) return IRIS_E_INVALID;
        const int64_t* f = (const int64_t*)data;
        for (uint64_t i = 0; i < rows * cols; i++)
            if (f[i] < 0 || f[i] > ((int64_t)1 << 32)) return IRIS_E_INVALID;  // layer.rs:75-83
        RT_CHECK(dev_alloc_copy(&m->inv_freq, data, bytes));
        return 0;
    }
    return 0;
}

// The per-layer derivations of a gemma-dense model
// (crates/inference/direct/src/model.rs:817-877): head size, RoPE and
// window by layer kind, the KV donor of the shared layers, and the two RoPE
// frequency ladders (validated as prefill_range.rs:394-466 does).
static int gemma_finalize(IrisModel* m) {
    const IrisModelDesc& d = m->d;
    if (d.layers == 0) return 0;
    if (!m->embed_ple || !m->ple_model_proj || !m->ple_proj_norm) return IRIS_E_STATE;
    const uint32_t rot_full = (uint32_t)(((uint64_t)d.global_head_dim * (uint32_t)d.partial_rotary_q16) >> 16);
    struct Kind {
        int64_t base;
        uint32_t hd, rotary;
        int64_t** table;
    } kinds[2] = {{d.rope_base_full, d.global_head_dim, rot_full, &m->rope_full},
                  {d.rope_base_sliding, d.head_dim, d.head_dim, &m->rope_sliding}};
    for (int kind = 0; kind < 2; kind++) {
        Kind& k = kinds[kind];
        bool used = false;
        for (uint32_t l = 0; l < d.layers; l++) used |= (m->layer_is_sliding[l] != 0) == (kind == 1);
        if (!used) continue;
        if (k.rotary % 2 || k.rotary > k.hd) return IRIS_E_INVALID;
        if (k.rotary == 0) continue;
        if (k.hd < 2 || k.hd % 2 || k.base <= 0) return IRIS_E_INVALID;
        if (*k.table) continue;
        RT_CHECK(hipMalloc((void**)k.table, (k.rotary / 2) * sizeof(int64_t)));
        RT_CHECK(iris_rope_ladder_launch(k.base, k.hd, k.rotary / 2, *k.table, m->stream));
    }
    const uint32_t shared = d.num_kv_shared_layers;
    const uint32_t first_shared = d.layers > shared ? d.layers - shared : 0;
    for (uint32_t l = 0; l < d.layers; l++) {
        LayerWeights& L = m->layers[l];
        if (!L.norm_post_attn || !L.norm_post_ffw || !L.norm_post_ple || !L.q_norm || !L.k_norm || !L.ple_gate ||
            !L.ple_proj)
            return IRIS_E_STATE;
        const bool sliding = m->layer_is_sliding[l] != 0;
        const Kind& k = kinds[sliding ? 1 : 0];
        L.head_dim = k.hd;
        L.rotary_dim = k.rotary;
        L.inv_freq = *k.table;
        L.window = sliding ? d.sliding_window : 0;
        L.kv_source = (int32_t)l;
        if (shared != 0 && l >= first_shared) {
            for (int32_t c = (int32_t)first_shared - 1; c >= 0; c--)
                if (m->layer_is_sliding[c] == m->layer_is_sliding[l]) {
                    L.kv_source = c;
                    break;
                }
        }
    }
    return (int)hipStreamSynchronize(m->stream);
}

int iris_model_finalize(IrisModel* m) {
    if (!m) return IRIS_E_INVALID;
    const IrisModelDesc& d = m->d;
    const bool gemma = d.family == IRIS_FAMILY_GEMMA_DENSE;
    if (!m->embed_raw || !m->head || !m->final_norm || (!gemma && d.layers && !m->inv_freq)) return IRIS_E_STATE;
    if (gemma) RT_CHECK(gemma_finalize(m));
    for (uint32_t l = 0; l < d.layers; l++) {
        LayerWeights& L = m->layers[l];
        if (!L.wqkv || !L.wo || !L.wgu || !L.wdown || !L.norm_attn || !L.norm_ff) return IRIS_E_STATE;
        if (!gemma) {
            L.head_dim = d.head_dim;
            L.kv_source = (int32_t)l;
        }
        if (L.q_rows != d.heads * L.head_dim || L.kv_rows != d.kv_heads * L.head_dim || (!gemma && L.ffn != d.ffn))
            return IRIS_E_INVALID;
        if (L.wo->rows != d.hidden || L.wo->cols != L.q_rows || L.wdown->rows != d.hidden || L.wdown->cols != L.ffn)
            return IRIS_E_INVALID;
        m->max_head_dim = std::max(m->max_head_dim, L.head_dim);
        m->max_ffn = std::max(m->max_ffn, L.ffn);
        m->max_qkv = std::max(m->max_qkv, L.q_rows + 2 * L.kv_rows);
        m->pending[l].clear();
    }
    m->finalized = true;
    return 0;
}

uint64_t iris_model_device_bytes(const IrisModel* m) {
    if (!m) return 0;
    uint64_t b = 0;
    for (const auto& L : m->layers)
        for (const Q8GpuMatrix* w : {L.wqkv, L.wo, L.wgu, L.wdown})
            if (w) b += w->device_bytes;
    if (m->head) b += m->head->device_bytes;
    if (m->d.family == IRIS_FAMILY_GEMMA_DENSE) {
        const uint64_t hp = (uint64_t)m->d.hidden * m->d.ple_width * 4;
        b += (uint64_t)m->layers.size() * 2 * hp + (uint64_t)m->d.layers * hp;  // PLE matrices
    }
    return b;
}

void iris_model_free(IrisModel* m) {
    if (!m) return;
    for (auto& L : m->layers) {
        q8gpu_free(L.wqkv);
        q8gpu_free(L.wo);
        q8gpu_free(L.wgu);
        q8gpu_free(L.wdown);
        for (int32_t* p : {L.norm_attn, L.norm_ff, L.norm_post_attn, L.norm_post_ffw, L.norm_post_ple, L.q_norm,
                           L.k_norm, L.ple_gate, L.ple_proj})
            hipFree(p);
    }
    q8gpu_free(m->head);
    hipFree(m->embed_raw);
    hipFree(m->final_norm);
    hipFree(m->inv_freq);
    hipFree(m->embed_ple);
    hipFree(m->ple_model_proj);
    hipFree(m->ple_proj_norm);
    hipFree(m->rope_sliding);
    hipFree(m->rope_full);
    if (m->stream) hipStreamDestroy(m->stream);
    delete m;
}

}  // extern "C"

// ---------------------------------------------------------------- session

// Where a checkpointing pass leaves each layer's rows: a device copy per
// layer, and an event recorded on the pass's stream once it is made.
struct CkptSink {
    int32_t* dev;        // [layers][rows][hidden]
    hipEvent_t* events;  // [layers]
};

static int checkpoint_layer(IrisSession* s, const CkptSink* sink, uint32_t l, uint32_t rows) {
    if (!sink) return 0;
    const size_t n = (size_t)rows * s->model->d.hidden;
    RT_CHECK(hipMemcpyAsync(sink->dev + l * n, s->x, n * 4, hipMemcpyDeviceToDevice, s->stream));
    return (int)hipEventRecord(sink->events[l], s->stream);
}

// A one-row product's input as digit planes left by its producer, with the
// session's k-split scratch (the launch stages the row from x instead where
// the broadcast product does not apply).
static void bcast_input(GemvArgs& g, IrisSession* s, const uint32_t* planes, const uint8_t* counts) {
    g.x_planes = planes;
    g.x_counts = counts;
    g.kpart = s->kpart;
    g.kcount = s->kcount;
}

// One mistral-dense layer over the session's rows in s->x (positions from
// *d_pos; the rows' RoPE table already in rope_sc), its output back in s->x.
// With `slots` (one row), the residual products leave per-tile sums of
// squares for the norms after them; ssq_x_in says whether s->ssq_x already
// holds those of the layer's input.
static int mistral_layer(IrisSession* s, uint32_t l, uint32_t rows, bool slots, bool ssq_x_in) {
    IrisModel* m = s->model;
    const IrisModelDesc& d = m->d;
    const uint32_t H = d.hidden;
    const uint32_t qw = d.heads * d.head_dim, kvw = d.kv_heads * d.head_dim;
    const uint32_t h_tiles = (H + Q8_TILE_ROWS - 1) / Q8_TILE_ROWS;
    hipStream_t st = s->stream;
    {
        const LayerWeights& L = m->layers[l];
        GemvArgs g{};
        // 1. q|k|v = W_qkv rms_norm(x); RoPE; K/V into the cache.
        g.w = q8_view(L.wqkv);
        g.x = s->x;
        g.x_stride = H;
        g.tokens = rows;
        g.prologue = PRO_RMSNORM;
        g.norm_w = L.norm_attn;
        g.norm_eps = d.norm_eps;
        g.epilogue = EPI_ROPE_KV;
        g.out = s->q;
        g.out_stride = qw;
        g.d_pos = s->d_pos;
        g.inv_freq = m->inv_freq;
        g.rope_sc = s->rope_sc;
        g.head_dim = d.head_dim;
        g.q_rows = qw;
        g.kv_rows = kvw;
        g.k_cache = s->k_cache[l];
        g.k_pos_stride = s->k_pos_stride;
        g.v_cache = s->v_cache[l];
        if (slots && ssq_x_in) {
            g.ssq_in = s->ssq_x;
            g.ssq_n = h_tiles;
        }
        with_gemm_space(g, s, rows);
        RT_CHECK(iris_gemv_launch(g, st));
        // 2. attention.
        AttnArgs a{};
        a.q = s->q;
        a.q_stride = qw;
        a.k_cache = s->k_cache[l];
        a.k_pos_stride = s->k_pos_stride;
        a.v_cache = s->v_cache[l];
        a.kv_stride = kvw;
        a.ctx = s->ctx;
        a.ctx_stride = qw;
        a.d_pos = s->d_pos;
        a.heads = d.heads;
        a.kv_heads = d.kv_heads;
        a.head_dim = d.head_dim;
        a.scaled = 1;
        a.scale_q32 = d.attention_scale_q32;
        a.window = 0;
        a.planes = s->attn_planes;
        a.scores = s->scores;
        // One row: the values launch leaves the context row's digit planes
        // for the O product.
        const bool ctx_planes = iris_attention_decode_applies(a, rows, s->max_positions);
        if (ctx_planes) {
            a.ctx_planes = s->ctx_planes;
            a.ctx_counts = s->ctx_counts;
        }
        RT_CHECK(iris_attention_launch(a, rows, s->max_positions, st));
        // 3. attended = W_o ctx + x.
        g = GemvArgs{};
        g.w = q8_view(L.wo);
        g.x = s->ctx;
        g.x_stride = qw;
        g.tokens = rows;
        g.epilogue = EPI_RESIDUAL;
        g.out = s->attended;
        g.out_stride = H;
        g.residual = s->x;
        g.residual_stride = H;
        if (slots) g.ssq_out = s->ssq_att;
        if (ctx_planes) bcast_input(g, s, s->ctx_planes, s->ctx_counts);
        with_gemm_space(g, s, rows);
        RT_CHECK(iris_gemv_launch(g, st));
        // 4. gated = mul(silu(W_gate m), W_up m), m = rms_norm(attended).
        g = GemvArgs{};
        g.w = q8_view(L.wgu);
        g.x = s->attended;
        g.x_stride = H;
        g.tokens = rows;
        g.prologue = PRO_RMSNORM;
        g.norm_w = L.norm_ff;
        g.norm_eps = d.norm_eps;
        g.epilogue = EPI_SWIGLU;
        g.silu_tab = s->silu_tab;
        g.out = s->gated;
        g.out_stride = d.ffn;
        if (slots) {
            g.ssq_in = s->ssq_att;
            g.ssq_n = h_tiles;
        }
        // One row: the gated row's digit planes too, for the down product.
        const bool gated_planes = rows == 1;
        if (gated_planes) {
            g.out_planes = s->gated_planes;
            g.out_counts = s->gated_counts;
        }
        with_gemm_space(g, s, rows);
        // 5. x = W_down gated + attended.
        GemvArgs dn{};
        dn.w = q8_view(L.wdown);
        dn.x = s->gated;
        dn.x_stride = d.ffn;
        dn.tokens = rows;
        dn.epilogue = EPI_RESIDUAL;
        dn.out = s->x;
        dn.out_stride = H;
        dn.residual = s->attended;
        dn.residual_stride = H;
        if (slots) dn.ssq_out = s->ssq_x;
        if (gated_planes) bcast_input(dn, s, s->gated_planes, s->gated_counts);
        with_gemm_space(dn, s, rows);
        // Several rows, both products on the matrix cores: the gate/up
        // product writes the gated rows' digit planes for the down product.
        if (rows > 1 && s->gated_gemm_planes && iris_gemm_applies(g) && iris_gemm_applies(dn)) {
            g.out = nullptr;  // nothing reads the gated rows themselves
            g.out_gemm_planes = s->gated_gemm_planes;
            g.out_gemm_limbs = s->gated_gemm_limbs;
            dn.planes = s->gated_gemm_planes;
            dn.token_limbs = s->gated_gemm_limbs;
            dn.planes_ready = 1;
        }
        RT_CHECK(iris_gemv_launch(g, st));
        RT_CHECK(iris_gemv_launch(dn, st));
    }
    return 0;
}

static int mistral_pass(IrisSession* s, uint32_t rows, const CkptSink* sink) {
    IrisModel* m = s->model;
    const IrisModelDesc& d = m->d;
    // The rows' RoPE (sin, cos) pairs, shared by every layer (for a one-row
    // pass after a selection, the selection kernel has formed them).
    if (!(rows == 1 && s->rope_ready) && d.layers)
        RT_CHECK(iris_rope_table_launch(m->inv_freq, d.head_dim / 2, s->d_pos, rows, s->rope_sc, s->stream));
    s->rope_ready = false;
    // One row: sums of squares pass from each residual product to the norm
    // after it (hidden rows in 16-row tiles, within the slot count).
    const uint32_t h_tiles = (d.hidden + Q8_TILE_ROWS - 1) / Q8_TILE_ROWS;
    const bool slots = rows == 1 && h_tiles <= GEMV_SSQ_SLOTS;
    s->ssq_x_valid = false;
    for (uint32_t l = 0; l < d.layers; l++) {
        RT_CHECK(mistral_layer(s, l, rows, slots, l > 0));
        RT_CHECK(checkpoint_layer(s, sink, l, rows));
    }
    s->ssq_x_valid = slots && d.layers > 0;
    return 0;
}

// One gemma-dense pass (crates/inference/kernels/src/prefill_range.rs:307-958
// per layer, the PLE prepare of view_kernels.rs:59-99 first): eleven launches
// per layer, eight for one row.
//
// The PLE inputs of every layer (view_kernels.rs:59-99) from the embedded
// rows in s->x and their ids, into s->ple_rows [rows][layers * ple_width].
static int gemma_ple(IrisSession* s, uint32_t rows) {
    IrisModel* m = s->model;
    const IrisModelDesc& d = m->d;
    const uint32_t H = d.hidden, P = d.ple_width, LP = d.layers * d.ple_width;
    hipStream_t st = s->stream;
    I32GemvArgs ig{};
    ig.w = m->ple_model_proj;
    ig.rows = LP;
    ig.cols = H;
    ig.x = s->x;
    ig.x_stride = H;
    ig.out = s->ple_proj;
    ig.out_stride = LP;
    RT_CHECK(iris_i32_gemv_launch(ig, rows, st));
    PleArgs pa{};
    pa.proj = s->ple_proj;
    pa.row_stride = LP;
    pa.ids = s->ids;
    pa.emb = m->embed_ple;
    pa.emb_row_bytes = m->embed_ple_row_bytes;
    pa.ple_width = P;
    pa.norm_w = m->ple_proj_norm;
    pa.eps = d.norm_eps;
    pa.projection_scalar = d.ple_projection_scalar;
    pa.embedding_scale = d.ple_embedding_scale;
    pa.input_scale = d.ple_input_scale;
    pa.out = s->ple_rows;
    return iris_ple_prepare_launch(pa, d.layers, rows, st);
}

// One gemma-dense layer over the rows in s->x (positions from *d_pos), with
// the layer's PLE inputs in s->ple_rows; the output back in s->x.
//
// With `carry` (one row): no separate norm launches. The previous layer's
// PLE post-norm, still carried, is formed in the q|k|v product's prologue;
// the o and down products leave their row in tmp with per-tile sums of
// squares, and the post-norm and residual are formed in the prologue of
// the product after each (gate|up, the PLE gate); this layer's PLE
// post-norm is left carried. The residual alternates between x and
// attended (a prologue writes its row apart from the one it reads).
static int gemma_layer(IrisSession* s, uint32_t l, uint32_t rows, bool carry) {
    IrisModel* m = s->model;
    const IrisModelDesc& d = m->d;
    const uint32_t H = d.hidden, P = d.ple_width, LP = d.layers * d.ple_width;
    const uint32_t h_tiles = (H + Q8_TILE_ROWS - 1) / Q8_TILE_ROWS;
    hipStream_t st = s->stream;
    IrisSession::GemmaCarry& c = s->carry;
    I32GemvArgs ig{};
    {
        const LayerWeights& L = m->layers[l];
        const uint32_t hd = L.head_dim, qw = L.q_rows, kvw = L.kv_rows, qkvw = qw + 2 * kvw;
        // The layer's input row (its residual) and the free one.
        int32_t* xin = s->x;
        int32_t* other = s->attended;
        // 1. q|k|v = W_qkv rms_norm(x, input_layernorm)  (project_tokens :497-579)
        GemvArgs g{};
        g.w = q8_view(L.wqkv);
        g.x = s->x;
        g.x_stride = H;
        g.tokens = rows;
        g.prologue = PRO_RMSNORM;
        g.norm_w = L.norm_attn;
        g.norm_eps = d.norm_eps;
        if (carry && c.pending) {
            // x = (rms_norm(tmp, post_ple) + res) * layer scalar of the layer below
            g.x = s->tmp;
            g.prologue = PRO_NORM_RES_NORM;
            g.ssq_in = s->ssq_x;
            g.ssq_n = c.slots;
            g.res_norm_w = c.norm_w;
            g.res_in = c.res;
            g.res_scalar = c.scalar;
            g.res_out = c.spare;
            xin = c.spare;
            other = c.res;
        }
        g.epilogue = EPI_STORE;
        g.out = s->qkv;
        g.out_stride = qkvw;
        with_gemm_space(g, s, rows);
        RT_CHECK(iris_gemv_launch(g, st));
        // 2. per-head norms and RoPE, K/V into the layer's own cache (:607-647)
        GemmaQkvArgs qa{};
        qa.qkv = s->qkv;
        qa.qkv_stride = qkvw;
        qa.heads = d.heads;
        qa.kv_heads = d.kv_heads;
        qa.head_dim = hd;
        qa.rotary_dim = L.rotary_dim;
        qa.q_norm = L.q_norm;
        qa.k_norm = L.k_norm;
        qa.eps = d.norm_eps;
        qa.inv_freq = L.inv_freq;
        qa.d_pos = s->d_pos;
        qa.q_out = s->q;
        qa.q_stride = qw;
        qa.k_cache = s->k_cache[l];
        qa.k_pos_stride = s->k_pos_stride;
        qa.v_cache = s->v_cache[l];
        RT_CHECK(iris_gemma_qkv_finish_launch(qa, rows, st));
        // 3. attention over the window of the source layer's cache (:692-845)
        AttnArgs a{};
        a.q = s->q;
        a.q_stride = qw;
        a.k_cache = s->k_cache[L.kv_source];
        a.k_pos_stride = s->k_pos_stride;
        a.v_cache = s->v_cache[L.kv_source];
        a.kv_stride = kvw;
        a.ctx = s->ctx;
        a.ctx_stride = qw;
        a.d_pos = s->d_pos;
        a.heads = d.heads;
        a.kv_heads = d.kv_heads;
        a.head_dim = hd;
        a.scaled = 0;
        a.window = L.window;
        a.planes = s->attn_planes;
        a.scores = s->scores;
        // One row: the context row's digit planes too, for the O product.
        const bool ctx_planes = iris_attention_decode_applies(a, rows, s->max_positions);
        if (ctx_planes) {
            a.ctx_planes = s->ctx_planes;
            a.ctx_counts = s->ctx_counts;
        }
        RT_CHECK(iris_attention_launch(a, rows, s->max_positions, st));
        // 4. attended = rms_norm(W_o ctx, post_attention) + x  (:879-892)
        g = GemvArgs{};
        g.w = q8_view(L.wo);
        g.x = s->ctx;
        g.x_stride = qw;
        g.tokens = rows;
        g.epilogue = EPI_STORE;
        g.out = s->tmp;
        g.out_stride = H;
        if (carry) g.ssq_out = s->ssq_x;
        if (ctx_planes) bcast_input(g, s, s->ctx_planes, s->ctx_counts);
        with_gemm_space(g, s, rows);
        RT_CHECK(iris_gemv_launch(g, st));
        if (!carry)
            RT_CHECK(iris_norm_residual_launch(s->tmp, H, L.norm_post_attn, d.norm_eps, s->x, H, 0, s->attended, H, H,
                                               rows, st));
        // 5. gated = mul(gelu(W_gate f), W_up f), f = rms_norm(attended, pre_ffw)  (:894-913)
        g = GemvArgs{};
        g.w = q8_view(L.wgu);
        g.x = s->attended;
        g.x_stride = H;
        g.tokens = rows;
        g.prologue = PRO_RMSNORM;
        g.norm_w = L.norm_ff;
        g.norm_eps = d.norm_eps;
        if (carry) {
            g.x = s->tmp;
            g.prologue = PRO_NORM_RES_NORM;
            g.ssq_in = s->ssq_x;
            g.ssq_n = h_tiles;
            g.res_norm_w = L.norm_post_attn;
            g.res_in = xin;
            g.res_out = other;  // attended
        }
        g.epilogue = EPI_GEGLU;
        g.out = s->gated;
        g.out_stride = L.ffn;
        // One row: the gated row's digit planes too, for the down product.
        const bool gated_planes = rows == 1;
        if (gated_planes) {
            g.out_planes = s->gated_planes;
            g.out_counts = s->gated_counts;
        }
        with_gemm_space(g, s, rows);
        // 6. attended = rms_norm(W_down gated, post_ffw) + attended  (finish_mlp :915-929)
        GemvArgs dn{};
        dn.w = q8_view(L.wdown);
        dn.x = s->gated;
        dn.x_stride = L.ffn;
        dn.tokens = rows;
        dn.epilogue = EPI_STORE;
        dn.out = s->tmp;
        dn.out_stride = H;
        if (carry) dn.ssq_out = s->ssq_x;
        if (gated_planes) bcast_input(dn, s, s->gated_planes, s->gated_counts);
        with_gemm_space(dn, s, rows);
        // Several rows, both products on the matrix cores: the gate/up
        // product writes the gated rows' digit planes for the down product.
        if (rows > 1 && s->gated_gemm_planes && iris_gemm_applies(g) && iris_gemm_applies(dn)) {
            g.out = nullptr;  // nothing reads the gated rows themselves
            g.out_gemm_planes = s->gated_gemm_planes;
            g.out_gemm_limbs = s->gated_gemm_limbs;
            dn.planes = s->gated_gemm_planes;
            dn.token_limbs = s->gated_gemm_limbs;
            dn.planes_ready = 1;
        }
        RT_CHECK(iris_gemv_launch(g, st));
        RT_CHECK(iris_gemv_launch(dn, st));
        if (!carry)
            RT_CHECK(iris_norm_residual_launch(s->tmp, H, L.norm_post_ffw, d.norm_eps, s->attended, H, 0, s->attended,
                                               H, H, rows, st));
        // 7. PLE block: g = mul(gelu(gate attended), ple); x = rms_norm(proj g) + attended,
        //    times the layer scalar (:931-958)
        ig = I32GemvArgs{};
        ig.w = L.ple_gate;
        ig.rows = P;
        ig.cols = H;
        ig.x = s->attended;
        ig.x_stride = H;
        ig.out = s->ple_gated;
        ig.out_stride = P;
        ig.aux = s->ple_rows + (size_t)l * P;
        ig.aux_stride = LP;
        if (carry) {
            // attended = rms_norm(tmp, post_ffw) + attended, over the layer's input row
            ig.x = s->tmp;
            ig.res_in = other;
            ig.res_norm_w = L.norm_post_ffw;
            ig.eps = d.norm_eps;
            ig.ssq_in = s->ssq_x;
            ig.ssq_n = h_tiles;
            ig.res_out = xin;
        }
        RT_CHECK(iris_i32_gemv_launch(ig, rows, st));
        ig = I32GemvArgs{};
        ig.w = L.ple_proj;
        ig.rows = H;
        ig.cols = P;
        ig.x = s->ple_gated;
        ig.x_stride = P;
        ig.out = s->tmp;
        ig.out_stride = H;
        if (carry) ig.ssq_out = s->ssq_x;
        RT_CHECK(iris_i32_gemv_launch(ig, rows, st));
        if (carry) {
            c.pending = true;
            c.norm_w = L.norm_post_ple;
            c.scalar = L.layer_scalar;
            c.res = xin;
            c.spare = other;
            c.slots = i32_gemv_slots(H);
        } else {
            RT_CHECK(iris_norm_residual_launch(s->tmp, H, L.norm_post_ple, d.norm_eps, s->attended, H, L.layer_scalar,
                                               s->x, H, H, rows, st));
        }
    }
    return 0;
}

// One row with no per-layer checkpoints: the post-norms are carried (the
// row fits the slot counts and the staged-row limits).
static bool gemma_carries(const IrisSession* s, uint32_t rows, const CkptSink* sink) {
    const uint32_t H = s->model->d.hidden;
    return rows == 1 && !sink && H % 4 == 0 && (H + Q8_TILE_ROWS - 1) / Q8_TILE_ROWS <= GEMV_SSQ_SLOTS &&
           H <= 4096 && H <= I32_GEMV_MAX_STAGED;
}

static int gemma_pass(IrisSession* s, uint32_t rows, const CkptSink* sink) {
    const bool carry = gemma_carries(s, rows, sink);
    s->carry = IrisSession::GemmaCarry{};
    if (s->model->d.layers) RT_CHECK(gemma_ple(s, rows));
    for (uint32_t l = 0; l < s->model->d.layers; l++) {
        RT_CHECK(gemma_layer(s, l, rows, carry));
        RT_CHECK(checkpoint_layer(s, sink, l, rows));
    }
    return 0;
}

static int session_pass(IrisSession* s, uint32_t rows, const CkptSink* sink) {
    s->ssq_x_valid = false;
    s->carry.pending = false;
    if (s->model->d.family == IRIS_FAMILY_GEMMA_DENSE) return gemma_pass(s, rows, sink);
    return mistral_pass(s, rows, sink);
}

static int session_head_select(IrisSession* s, uint32_t rows) {
    IrisModel* m = s->model;
    const IrisModelDesc& d = m->d;
    GemvArgs g{};
    g.w = q8_view(m->head);
    g.x = s->x + (size_t)(rows - 1) * d.hidden;
    g.x_stride = d.hidden;
    g.tokens = 1;
    g.prologue = PRO_RMSNORM;
    g.norm_w = m->final_norm;
    g.norm_eps = d.norm_eps;
    if (rows == 1 && s->ssq_x_valid) {
        g.ssq_in = s->ssq_x;
        g.ssq_n = (d.hidden + Q8_TILE_ROWS - 1) / Q8_TILE_ROWS;
    }
    if (rows == 1 && s->carry.pending) {
        // the last layer's PLE post-norm, carried into the final norm
        g.x = s->tmp;
        g.prologue = PRO_NORM_RES_NORM;
        g.ssq_in = s->ssq_x;
        g.ssq_n = s->carry.slots;
        g.res_norm_w = s->carry.norm_w;
        g.res_in = s->carry.res;
        g.res_scalar = s->carry.scalar;
        g.res_out = nullptr;
    }
    g.epilogue = EPI_HEAD_SELECT;
    g.softcap = m->head_softcap;
    g.out = s->logits;
    g.out_stride = d.vocab;
    g.logits_keep = s->keep_logits ? s->logits_keep : nullptr;
    g.d_step = s->d_step;
    g.d_pos_rw = s->d_pos;
    g.rows_in_pass = rows;
    g.tokens_out = s->tokens;
    g.embed_raw = m->embed_raw;
    g.embed_row_bytes = m->embed_row_bytes;
    g.hidden = d.hidden;
    g.embed_scale = m->embed_scale;
    g.x_next = s->x;
    g.ids_next = m->d.family == IRIS_FAMILY_GEMMA_DENSE ? s->ids : nullptr;
    g.sel_partial = s->sel_partial;
    const bool rope = m->d.family != IRIS_FAMILY_GEMMA_DENSE && d.layers;
    if (rope) {
        g.rope_next = s->rope_sc;
        g.rope_half = d.head_dim / 2;
        g.inv_freq = m->inv_freq;
    }
    RT_CHECK(iris_gemv_launch(g, s->stream));
    RT_CHECK(iris_select_launch(g, s->stream));
    s->rope_ready = rope;
    return 0;
}

// True when embedding token `id` is refused: its embedding row, or for a
// gemma-dense model with layers its PLE row, has a non-finite block scale
// (dequantize_row, q8.rs:76-92, when model.rs:316-330 or the PLE prepare
// reads the row).
static bool embedding_refused(const IrisModel* m, int32_t id) {
    return (!m->embed_bad.empty() && m->embed_bad[id]) || (!m->ple_bad.empty() && m->ple_bad[id]);
}

// The pass's rows: the embedding of `ids` at positions start.., the step
// counter reset.
static int session_reset_and_embed(IrisSession* s, const int32_t* ids, uint32_t count, uint32_t start = 0) {
    IrisModel* m = s->model;
    s->rope_ready = false;
    for (uint32_t i = 0; i < count; i++) {
        if (ids[i] < 0 || (uint32_t)ids[i] >= m->d.vocab) return IRIS_E_INVALID;
        if (embedding_refused(m, ids[i])) return IRIS_E_SCALE;
    }
    RT_CHECK(iris_set_counters_launch(s->d_pos, (int32_t)start, s->d_step, 0, s->stream));
    RT_CHECK(hipMemcpyAsync(s->ids, ids, (size_t)count * 4, hipMemcpyHostToDevice, s->stream));
    return iris_embed_rows_launch(s->ids, count, m->embed_raw, m->embed_row_bytes, m->d.hidden, m->embed_scale, s->x,
                                  s->stream);
}

// ---- KV coverage (raster-stages/layer-mistral/src/lib.rs:889-940,
// raster-stages/prefill-range/src/lib.rs:1237-1290): a range at `start`
// needs, in its attention source's cache, every position before it that its
// first row sees: all of 0..start, or for a sliding layer the window's part.

// First position the rows of a range at `start` read from before it.
static uint32_t range_needs_from(const LayerWeights& L, uint32_t start) {
    if (L.window == 0 || start == 0) return 0;
    return start + 1 > L.window ? start + 1 - L.window : 0;
}

static bool range_covered(const IrisSession* s, uint32_t start) {
    const IrisModel* m = s->model;
    for (uint32_t l = 0; l < m->d.layers; l++) {
        const LayerWeights& L = m->layers[l];
        const uint32_t src = (uint32_t)L.kv_source;
        const uint32_t from = range_needs_from(L, start);
        if (from < start && (s->kv_lo[src] > from || s->kv_hi[src] < start)) return false;
    }
    return true;
}

// Positions [pos0, pos0 + count) of a layer's cache now hold keys; a block
// that does not touch what the cache held starts it afresh.
static void cover(IrisSession* s, uint32_t l, uint32_t pos0, uint32_t count) {
    uint32_t& lo = s->kv_lo[l];
    uint32_t& hi = s->kv_hi[l];
    const uint32_t end = pos0 + count;
    if (lo == hi || pos0 > hi || end < lo) {
        lo = pos0;
        hi = end;
    } else {
        lo = std::min(lo, pos0);
        hi = std::max(hi, end);
    }
}

static void cover_all(IrisSession* s, uint32_t pos0, uint32_t count, bool fresh) {
    for (uint32_t l = 0; l < s->model->d.layers; l++) {
        if (fresh) s->kv_lo[l] = s->kv_hi[l] = 0;
        cover(s, l, pos0, count);
    }
}

// A pass is about to write positions [pos0, pos0 + count) of a layer's
// cache: until it has succeeded they hold no keys, so the coverage keeps
// only what lies before them (or after, when nothing lies before). A pass
// that fails partway then leaves no claim on positions it may have
// overwritten; a pass that succeeds covers them again.
static void uncover(IrisSession* s, uint32_t l, uint32_t pos0, uint32_t count) {
    uint32_t& lo = s->kv_lo[l];
    uint32_t& hi = s->kv_hi[l];
    const uint32_t end = pos0 + count;
    if (lo == hi || end <= lo || pos0 >= hi) return;
    if (lo < pos0) hi = pos0;
    else if (end < hi) lo = end;
    else lo = hi = 0;
}

static void uncover_all(IrisSession* s, uint32_t pos0, uint32_t count, bool fresh) {
    for (uint32_t l = 0; l < s->model->d.layers; l++) {
        if (fresh) s->kv_lo[l] = s->kv_hi[l] = 0;
        uncover(s, l, pos0, count);
    }
}

// True when a kernel tracer is loaded in this process: the ROCm profiler
// SDK (rocprofv3 preloads its tool, which loads the SDK) or the older
// rocprofiler. Graph replays of the decode pass ended twice in a segfault
// inside the HIP runtime under rocprofv3 --kernel-trace with no cause shown
// on the library's side, so they are refused while a tracer is present;
// the same pass launched kernel by kernel traces normally.
static bool kernel_tracer_loaded() {
    int found = 0;
    dl_iterate_phdr(
        [](struct dl_phdr_info* info, size_t, void* data) -> int {
            const char* n = info->dlpi_name;
            if (n && (std::strstr(n, "librocprofiler-sdk.so") || std::strstr(n, "librocprofiler-sdk-tool") ||
                      std::strstr(n, "librocprofiler64"))) {
                *(int*)data = 1;
                return 1;
            }
            return 0;
        },
        &found);
    return found != 0;
}

// Captures the decode pass (one row, head, select) as a graph. Each
// generation captures its own (a few hundred nodes, outside any timed
// region), so no graph outlives the call that made it.
static int ensure_graph(IrisSession* s, bool fresh) {
    if (kernel_tracer_loaded()) return IRIS_E_TRACED;
    if (!fresh && s->graph_exec && s->graph_keep_logits == s->keep_logits) return 0;
    if (s->graph_exec) {
        hipGraphExecDestroy(s->graph_exec);
        s->graph_exec = nullptr;
    }
    hipGraph_t graph = nullptr;
    RT_CHECK(hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal));
    int rc = session_pass(s, 1, nullptr);
    if (rc == 0) rc = session_head_select(s, 1);
    hipError_t st = hipStreamEndCapture(s->stream, &graph);
    if (rc == 0) rc = (int)st;
    if (rc == 0) rc = (int)hipGraphInstantiate(&s->graph_exec, graph, nullptr, nullptr, 0);
    if (graph) hipGraphDestroy(graph);
    if (rc == 0) s->graph_keep_logits = s->keep_logits;
    return rc;
}

static int session_decode_pass(IrisSession* s, int use_graph) {
    if (!use_graph) {
        RT_CHECK(session_pass(s, 1, nullptr));
        return session_head_select(s, 1);
    }
    RT_CHECK(ensure_graph(s, false));
    return (int)hipGraphLaunch(s->graph_exec, s->stream);
}

extern "C" {

int iris_session_create(IrisModel* m, uint32_t max_positions, uint32_t max_rows, IrisSession** out) {
    if (!m || !out || !m->finalized || max_positions == 0 || max_rows == 0) return IRIS_E_INVALID;
    *out = nullptr;
    const IrisModelDesc& d = m->d;
    if (max_rows > max_positions || max_positions > ATTN_MAX_KEYS) return IRIS_E_RANGE;
    iris_gemv_prepare();
    IrisSession* s = new (std::nothrow) IrisSession();
    if (!s) return IRIS_E_NOMEM;
    s->model = m;
    s->max_positions = max_positions;
    s->k_pos_stride = (max_positions + 63) & ~63u;
    s->max_rows = max_rows;
    const size_t qw = (size_t)d.heads * m->max_head_dim;
    hipError_t st = hipStreamCreate(&s->stream);
    s->k_cache.assign(d.layers, nullptr);
    s->v_cache.assign(d.layers, nullptr);
    s->kv_lo.assign(d.layers, 0);
    s->kv_hi.assign(d.layers, 0);
    for (uint32_t l = 0; l < d.layers && st == hipSuccess; l++) {
        const size_t kvw = m->layers[l].kv_rows;
        st = hipMalloc((void**)&s->k_cache[l], (size_t)s->k_pos_stride * kvw * 4);
        if (st == hipSuccess) st = hipMalloc((void**)&s->v_cache[l], (size_t)max_positions * kvw * 4);
    }
    auto alloc = [&](int32_t** p, size_t n) {
        if (st == hipSuccess) st = hipMalloc((void**)p, (n ? n : 1) * 4);
    };
    if (d.family != IRIS_FAMILY_GEMMA_DENSE && st == hipSuccess)
        st = hipMalloc((void**)&s->rope_sc, (size_t)max_rows * d.head_dim * sizeof(int64_t));
    alloc(&s->x, (size_t)max_rows * d.hidden);
    alloc(&s->attended, (size_t)max_rows * d.hidden);
    if (st == hipSuccess) st = hipMalloc((void**)&s->ssq_x, GEMV_SSQ_SLOTS * sizeof(int64_t));
    if (st == hipSuccess) st = hipMalloc((void**)&s->ssq_att, GEMV_SSQ_SLOTS * sizeof(int64_t));
    alloc(&s->q, (size_t)max_rows * qw);
    alloc(&s->scores, attn_scores_ints(d.heads, s->k_pos_stride));
    alloc(&s->ctx, (size_t)max_rows * qw);
    alloc(&s->gated, (size_t)max_rows * m->max_ffn);
    {
        auto allocb = [&](void** p, uint64_t bytes) {
            if (st == hipSuccess) st = hipMalloc(p, (bytes + 15) / 16 * 16);
        };
        const uint32_t h_rows = (d.hidden + Q8_TILE_ROWS - 1) / Q8_TILE_ROWS * Q8_TILE_ROWS;
        allocb((void**)&s->ctx_planes, act_planes_dwords(qw) * 4);
        allocb((void**)&s->ctx_counts, act_counts_bytes(qw));
        allocb((void**)&s->gated_planes, act_planes_dwords(m->max_ffn) * 4);
        allocb((void**)&s->gated_counts, act_counts_bytes(m->max_ffn));
        allocb((void**)&s->kpart, (uint64_t)BCAST_MAX_PARTS * h_rows * sizeof(int64_t));
        allocb((void**)&s->kcount, (uint64_t)bcast_groups(d.hidden) * sizeof(uint32_t));
        if (st == hipSuccess) st = hipMemset(s->kcount, 0, (uint64_t)bcast_groups(d.hidden) * sizeof(uint32_t));
    }
    if (max_rows > 1) {
        // Per-block scale matrices go through the matrix cores folded.
        for (uint32_t l = 0; l < d.layers && st == hipSuccess; l++)
            for (Q8GpuMatrix* w : {m->layers[l].wqkv, m->layers[l].wo, m->layers[l].wgu, m->layers[l].wdown})
                if (st == hipSuccess) st = (hipError_t)iris_q8_prepare_fold(w, s->stream);
        // The matrix-core SwiGLU epilogues look silu up.
        if (d.family != IRIS_FAMILY_GEMMA_DENSE && st == hipSuccess) st = (hipError_t)iris_silu_table(&s->silu_tab);
        size_t widest = std::max<size_t>(d.hidden, std::max<size_t>(qw, m->max_ffn));
        if (st == hipSuccess) st = hipMalloc((void**)&s->planes, gemm_planes_bytes((uint32_t)widest, max_rows));
        alloc(&s->token_limbs, (size_t)gemm_limb_ints((uint32_t)widest, max_rows));
        if (st == hipSuccess) st = hipMalloc((void**)&s->gated_gemm_planes, gemm_planes_bytes(m->max_ffn, max_rows));
        alloc(&s->gated_gemm_limbs, (size_t)gemm_limb_ints(m->max_ffn, max_rows));
        AttnPlanes& ap = s->attn_planes;
        ap.qt_cap = (max_rows + 15) / 16;
        ap.ks_cap = (max_positions + 63) / 64;
        auto alloc8 = [&](void** p, uint64_t bytes) {
            if (st == hipSuccess) st = hipMalloc(p, bytes);
        };
        alloc8((void**)&ap.q, attn_q_planes_bytes(d.heads, m->max_head_dim, ap.qt_cap));
        alloc8((void**)&ap.k, attn_kv_planes_bytes(d.kv_heads, m->max_head_dim, ap.ks_cap));
        alloc8((void**)&ap.v, attn_kv_planes_bytes(d.kv_heads, m->max_head_dim, ap.ks_cap));
        alloc8((void**)&ap.q_limbs, (uint64_t)d.heads * ap.qt_cap);
        alloc8((void**)&ap.kv_limbs, 2ull * d.kv_heads * ap.ks_cap);
        alloc8((void**)&ap.e_store, attn_e_store_bytes(d.heads, ap.qt_cap, ap.ks_cap));
    }
    if (d.family == IRIS_FAMILY_GEMMA_DENSE) {
        const size_t lp = (size_t)d.layers * d.ple_width;
        alloc(&s->qkv, (size_t)max_rows * m->max_qkv);
        alloc(&s->tmp, (size_t)max_rows * d.hidden);
        alloc(&s->ple_proj, (size_t)max_rows * lp);
        alloc(&s->ple_rows, (size_t)max_rows * lp);
        alloc(&s->ple_gated, (size_t)max_rows * d.ple_width);
    }
    alloc(&s->logits, d.vocab);
    alloc(&s->ids, max_rows);
    alloc(&s->tokens, max_positions + 1);
    alloc(&s->d_pos, 1);
    alloc(&s->d_step, 1);
    if (st == hipSuccess) st = hipMalloc((void**)&s->sel_partial, (size_t)m->head->tiles * sizeof(uint64_t));
    if (st != hipSuccess) {
        iris_session_free(s);
        return (int)st;
    }
    *out = s;
    return 0;
}

void iris_session_free(IrisSession* s) {
    if (!s) return;
    if (s->graph_exec) hipGraphExecDestroy(s->graph_exec);
    for (auto p : s->k_cache) hipFree(p);
    for (auto p : s->v_cache) hipFree(p);
    for (int32_t* p : {s->x, s->attended, s->q, s->scores, s->ctx, s->gated, s->logits, s->ids, s->tokens, s->d_pos, s->d_step,
                       s->logits_keep, s->qkv, s->tmp, s->ple_proj, s->ple_rows, s->ple_gated})
        hipFree(p);
    hipFree(s->sel_partial);
    hipFree(s->planes);
    hipFree(s->token_limbs);
    hipFree(s->gated_gemm_planes);
    hipFree(s->gated_gemm_limbs);
    hipFree(s->ssq_x);
    hipFree(s->ssq_att);
    hipFree(s->ctx_planes);
    hipFree(s->ctx_counts);
    hipFree(s->gated_planes);
    hipFree(s->gated_counts);
    hipFree(s->kpart);
    hipFree(s->kcount);
    hipFree(s->attn_planes.q);
    hipFree(s->attn_planes.k);
    hipFree(s->attn_planes.v);
    hipFree(s->attn_planes.q_limbs);
    hipFree(s->attn_planes.kv_limbs);
    hipFree(s->attn_planes.e_store);
    hipFree(s->rope_sc);
    hipFree(s->ckpt_dev);
    if (s->ckpt_host) hipHostFree(s->ckpt_host);
    for (auto e : s->ckpt_events)
        if (e) hipEventDestroy(e);
    if (s->copy_stream) hipStreamDestroy(s->copy_stream);
    if (s->stream) hipStreamDestroy(s->stream);
    delete s;
}

static int session_generate(IrisSession* s, const int32_t* prompt, uint32_t prompt_len, uint32_t tokens,
                            const int32_t* eos_ids, uint32_t n_eos, int32_t* out_tokens, uint32_t* out_count,
                            int32_t* out_logits, int32_t use_graph) {
    if (!s || !prompt || !out_tokens || !out_count) return IRIS_E_INVALID;
    *out_count = 0;
    if (prompt_len == 0 || tokens == 0) return tokens == 0 ? 0 : IRIS_E_INVALID;
    IrisModel* m = s->model;
    const IrisModelDesc& d = m->d;
    if (prompt_len > s->max_rows) return IRIS_E_RANGE;
    if (use_graph && tokens > 1 && kernel_tracer_loaded()) return IRIS_E_TRACED;
    // The last pass runs at position prompt_len + tokens - 2.
    const uint64_t end = (uint64_t)prompt_len + tokens - 1;
    if (end > s->max_positions || end > d.max_positions) return IRIS_E_RANGE;
    s->keep_logits = out_logits != nullptr;
    if (s->keep_logits) {
        const size_t need = (size_t)tokens * d.vocab;
        if (need > s->logits_keep_cap) {
            hipFree(s->logits_keep);
            s->logits_keep = nullptr;
            s->logits_keep_cap = 0;
            RT_CHECK(hipMalloc((void**)&s->logits_keep, need * 4));
            s->logits_keep_cap = need;
        }
    }
    // The passes fill positions 0..prompt_len + tokens - 1 of every cache
    // (covered once they have run).
    uncover_all(s, 0, (uint32_t)end, true);
    RT_CHECK(session_reset_and_embed(s, prompt, prompt_len));
    RT_CHECK(session_pass(s, prompt_len, nullptr));
    RT_CHECK(session_head_select(s, prompt_len));
    if (use_graph && tokens > 1) RT_CHECK(ensure_graph(s, true));
    for (uint32_t t = 1; t < tokens; t++) RT_CHECK(session_decode_pass(s, use_graph));
    RT_CHECK(hipMemcpyAsync(out_tokens, s->tokens, (size_t)tokens * 4, hipMemcpyDeviceToHost, s->stream));
    if (out_logits)
        RT_CHECK(hipMemcpyAsync(out_logits, s->logits_keep, (size_t)tokens * d.vocab * 4, hipMemcpyDeviceToHost,
                                s->stream));
    RT_CHECK(hipStreamSynchronize(s->stream));
    // Stop at the first EOS (it is kept), as executor.rs:163-168 does; the
    // passes after it do not change the tokens before it.
    uint32_t count = tokens;
    for (uint32_t t = 0; t < tokens; t++) {
        bool eos = false;
        for (uint32_t e = 0; e < n_eos; e++) eos |= out_tokens[t] == eos_ids[e];
        if (eos) {
            count = t + 1;
            break;
        }
    }
    // Each selection but the last is embedded for the next pass
    // (executor.rs:157-183): a refused row fails the run there.
    for (uint32_t t = 0; t + 1 < count; t++)
        if (embedding_refused(m, out_tokens[t])) return IRIS_E_SCALE;
    *out_count = count;
    cover_all(s, 0, (uint32_t)end, true);
    return 0;
}

extern "C" int iris_session_generate(IrisSession* s, const int32_t* prompt, uint32_t prompt_len, uint32_t tokens,
                                     const int32_t* eos_ids, uint32_t n_eos, int32_t* out_tokens,
                                     uint32_t* out_count, int32_t* out_logits, int32_t use_graph) {
    return session_generate(s, prompt, prompt_len, tokens, eos_ids, n_eos, out_tokens, out_count, out_logits,
                            use_graph);
}

// Staging for the per-layer checkpoints of passes of up to max_rows rows:
// device copies, pinned host copies, a copy stream and per-layer events.
static int ensure_checkpoint_space(IrisSession* s) {
    if (s->ckpt_dev) return 0;
    const IrisModelDesc& d = s->model->d;
    const size_t bytes = (size_t)d.layers * s->max_rows * d.hidden * 4;
    RT_CHECK(hipMalloc((void**)&s->ckpt_dev, bytes));
    RT_CHECK(hipHostMalloc((void**)&s->ckpt_host, bytes, hipHostMallocDefault));
    RT_CHECK(hipStreamCreate(&s->copy_stream));
    s->ckpt_events.assign(2 * (size_t)d.layers, nullptr);
    for (auto& e : s->ckpt_events) RT_CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    return 0;
}

static int layer_range_run(IrisSession* s, const int32_t* ids, uint32_t count, uint32_t start_position,
                           int32_t* out_rows, uint8_t* out_hashes);

// The pass runs on the session's stream, copying each layer's rows aside on
// the device as it finishes; a second stream brings them to pinned host
// memory behind it, and host threads hash (and copy out) each layer as it
// arrives, so the transfers and the hashing overlap the later layers.
int iris_session_layer_range(IrisSession* s, const int32_t* ids, uint32_t count, uint32_t start_position,
                             int32_t* out_rows, uint8_t* out_hashes) {
    if (!s || !ids || count == 0) return IRIS_E_INVALID;
    IrisModel* m = s->model;
    const IrisModelDesc& d = m->d;
    const uint64_t end = (uint64_t)start_position + count;
    if (count > s->max_rows || end > d.max_positions || end > s->max_positions) return IRIS_E_RANGE;
    if (!range_covered(s, start_position)) return IRIS_E_STATE;
    // A range at position 0 starts the caches afresh.
    uncover_all(s, start_position, count, start_position == 0);
    const int rc = layer_range_run(s, ids, count, start_position, out_rows, out_hashes);
    if (rc == 0) cover_all(s, start_position, count, false);
    return rc;
}

static int layer_range_run(IrisSession* s, const int32_t* ids, uint32_t count, uint32_t start_position,
                           int32_t* out_rows, uint8_t* out_hashes) {
    IrisModel* m = s->model;
    const IrisModelDesc& d = m->d;
    if (!out_rows && !out_hashes) {
        RT_CHECK(session_reset_and_embed(s, ids, count, start_position));
        RT_CHECK(session_pass(s, count, nullptr));
        return (int)hipStreamSynchronize(s->stream);
    }
    RT_CHECK(ensure_checkpoint_space(s));
    const uint32_t layers = d.layers;
    const size_t n = (size_t)count * d.hidden;
    hipEvent_t* on_device = s->ckpt_events.data();
    hipEvent_t* on_host = on_device + layers;
    const CkptSink sink{s->ckpt_dev, on_device};
    RT_CHECK(session_reset_and_embed(s, ids, count, start_position));
    RT_CHECK(session_pass(s, count, &sink));
    for (uint32_t l = 0; l < layers; l++) {
        RT_CHECK(hipStreamWaitEvent(s->copy_stream, on_device[l], 0));
        RT_CHECK(hipMemcpyAsync(s->ckpt_host + l * n * 4, s->ckpt_dev + l * n, n * 4, hipMemcpyDeviceToHost,
                                s->copy_stream));
        RT_CHECK(hipEventRecord(on_host[l], s->copy_stream));
    }
    const unsigned hw = std::thread::hardware_concurrency();
    const uint32_t workers = std::max(1u, std::min({layers, 16u, hw ? hw : 1u}));
    std::atomic<int> status{0};
    std::vector<std::thread> pool;
    for (uint32_t t = 0; t < workers; t++)
        pool.emplace_back([&, t] {
            for (uint32_t l = t; l < layers; l += workers) {
                const hipError_t st = hipEventSynchronize(on_host[l]);
                if (st != hipSuccess) {
                    status = (int)st;
                    continue;
                }
                const uint8_t* rows = s->ckpt_host + l * n * 4;
                if (out_rows) std::memcpy(out_rows + l * n, rows, n * 4);
                if (out_hashes) iris_sha256(rows, n * 4, out_hashes + 32 * l);
            }
        });
    for (auto& th : pool) th.join();
    RT_CHECK(hipStreamSynchronize(s->stream));
    return status;
}

int iris_session_layer_pass(IrisSession* s, const int32_t* ids, uint32_t count, int32_t* out_rows,
                            uint8_t* out_hashes) {
    return iris_session_layer_range(s, ids, count, 0, out_rows, out_hashes);
}

static int layer_stage_run(IrisSession* s, uint32_t layer, const int32_t* in_rows, uint32_t count,
                           uint32_t start_position, const int32_t* ple_rows, int32_t* out_rows);

// One layer over one range (run_layer_stage, mistral/stage.rs:172-226;
// run_prefill_range_direct, prefill_range.rs:82-172): the layer's input rows
// come from the host, its output rows go back, and its own keys and values
// of positions start.. land in the layer's cache beside the carried ones.
int iris_session_layer_stage(IrisSession* s, uint32_t layer, const int32_t* in_rows, uint32_t count,
                             uint32_t start_position, const int32_t* ple_rows, int32_t* out_rows) {
    if (!s || !in_rows || !out_rows || count == 0) return IRIS_E_INVALID;
    IrisModel* m = s->model;
    const IrisModelDesc& d = m->d;
    const bool gemma = d.family == IRIS_FAMILY_GEMMA_DENSE;
    if (layer >= d.layers || (gemma && !ple_rows)) return IRIS_E_INVALID;
    const uint64_t end = (uint64_t)start_position + count;
    if (count > s->max_rows || end > d.max_positions || end > s->max_positions) return IRIS_E_RANGE;
    const LayerWeights& L = m->layers[layer];
    const uint32_t src = (uint32_t)L.kv_source, from = range_needs_from(L, start_position);
    if (from < start_position && (s->kv_lo[src] > from || s->kv_hi[src] < start_position)) return IRIS_E_STATE;
    // A KV-shared gemma layer attends over its donor's cache, which must also
    // hold the range's own positions: the donor's stage for this range runs
    // first (model.rs:824-877 donors are earlier layers).
    if (src != layer && (s->kv_lo[src] == s->kv_hi[src] || s->kv_lo[src] > from || s->kv_hi[src] < end))
        return IRIS_E_STATE;
    uncover(s, layer, start_position, count);
    const int rc = layer_stage_run(s, layer, in_rows, count, start_position, ple_rows, out_rows);
    if (rc == 0) cover(s, layer, start_position, count);
    return rc;
}

static int layer_stage_run(IrisSession* s, uint32_t layer, const int32_t* in_rows, uint32_t count,
                           uint32_t start_position, const int32_t* ple_rows, int32_t* out_rows) {
    IrisModel* m = s->model;
    const IrisModelDesc& d = m->d;
    const bool gemma = d.family == IRIS_FAMILY_GEMMA_DENSE;
    s->rope_ready = false;
    s->ssq_x_valid = false;
    hipStream_t st = s->stream;
    const size_t H = d.hidden;
    RT_CHECK(iris_set_counters_launch(s->d_pos, (int32_t)start_position, s->d_step, 0, st));
    RT_CHECK(hipMemcpyAsync(s->x, in_rows, (size_t)count * H * 4, hipMemcpyHostToDevice, st));
    if (gemma) {
        // The layer's PLE inputs in their column of the pass's PLE rows.
        const size_t P = d.ple_width, LP = (size_t)d.layers * d.ple_width;
        RT_CHECK(hipMemcpy2DAsync(s->ple_rows + (size_t)layer * P, LP * 4, ple_rows, P * 4, P * 4, count,
                                  hipMemcpyHostToDevice, st));
        RT_CHECK(gemma_layer(s, layer, count, false));
    } else {
        RT_CHECK(iris_rope_table_launch(m->inv_freq, d.head_dim / 2, s->d_pos, count, s->rope_sc, st));
        RT_CHECK(mistral_layer(s, layer, count, false, false));
    }
    RT_CHECK(hipMemcpyAsync(out_rows, s->x, (size_t)count * H * 4, hipMemcpyDeviceToHost, st));
    return (int)hipStreamSynchronize(st);
}

// Carried keys into a layer's cache: one kv row of k and of v per position,
// the K side transposed into the cache's [kv_rows][k_pos_stride] layout.
int iris_session_write_kv(IrisSession* s, uint32_t layer, uint32_t pos0, uint32_t count, const int32_t* k,
                          const int32_t* v) {
    if (!s || (count && (!k || !v))) return IRIS_E_INVALID;
    const IrisModelDesc& d = s->model->d;
    if (layer >= d.layers) return IRIS_E_INVALID;
    if ((uint64_t)pos0 + count > s->max_positions) return IRIS_E_RANGE;
    if (count == 0) return 0;
    const size_t kvw = s->model->layers[layer].kv_rows;
    std::vector<int32_t> kt;
    try {
        kt.resize(kvw * count);
    } catch (...) {
        return IRIS_E_NOMEM;
    }
    for (size_t p = 0; p < count; p++)
        for (size_t c = 0; c < kvw; c++) kt[c * count + p] = k[p * kvw + c];
    RT_CHECK(hipStreamSynchronize(s->stream));
    RT_CHECK(hipMemcpy2D(s->k_cache[layer] + pos0, (size_t)s->k_pos_stride * 4, kt.data(), (size_t)count * 4,
                         (size_t)count * 4, kvw, hipMemcpyHostToDevice));
    RT_CHECK(hipMemcpy(s->v_cache[layer] + (size_t)pos0 * kvw, v, (size_t)count * kvw * 4, hipMemcpyHostToDevice));
    cover(s, layer, pos0, count);
    return 0;
}

// The K cache is transposed ([kv_rows][k_pos_stride]): the block of the
// asked positions comes over as kv_rows strided runs and is transposed into
// position rows on the host; V rows are already position rows.
int iris_session_read_kv(IrisSession* s, uint32_t layer, uint32_t pos0, uint32_t count, int32_t* k_out,
                         int32_t* v_out) {
    if (!s || (count && (!k_out || !v_out))) return IRIS_E_INVALID;
    const IrisModelDesc& d = s->model->d;
    if (layer >= d.layers) return IRIS_E_INVALID;
    if ((uint64_t)pos0 + count > s->max_positions) return IRIS_E_RANGE;
    if (count == 0) return 0;
    const size_t kvw = s->model->layers[layer].kv_rows;
    std::vector<int32_t> kt;
    try {
        kt.resize(kvw * count);
    } catch (...) {
        return IRIS_E_NOMEM;
    }
    RT_CHECK(hipStreamSynchronize(s->stream));
    RT_CHECK(hipMemcpy2D(kt.data(), (size_t)count * 4, s->k_cache[layer] + pos0, (size_t)s->k_pos_stride * 4,
                         (size_t)count * 4, kvw, hipMemcpyDeviceToHost));
    RT_CHECK(hipMemcpy(v_out, s->v_cache[layer] + (size_t)pos0 * kvw, (size_t)count * kvw * 4,
                       hipMemcpyDeviceToHost));
    for (size_t c = 0; c < kvw; c++)
        for (size_t p = 0; p < count; p++) k_out[p * kvw + c] = kt[c * count + p];
    return 0;
}

int iris_kernel_tracer_loaded(void) { return kernel_tracer_loaded() ? 1 : 0; }

int iris_session_time_pass(IrisSession* s, const int32_t* ids, uint32_t count, double* ms) {
    if (!s || !ids || !ms || count == 0) return IRIS_E_INVALID;
    if (count > s->max_rows || count > s->model->d.max_positions) return IRIS_E_RANGE;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    RT_CHECK(hipEventCreate(&e0));
    RT_CHECK(hipEventCreate(&e1));
    uncover_all(s, 0, count, true);
    int rc = session_reset_and_embed(s, ids, count);
    if (rc == 0) rc = (int)hipEventRecord(e0, s->stream);
    if (rc == 0) rc = session_pass(s, count, nullptr);
    if (rc == 0) rc = (int)hipEventRecord(e1, s->stream);
    float t = 0.f;
    if (rc == 0) rc = (int)hipEventSynchronize(e1);
    if (rc == 0) rc = (int)hipEventElapsedTime(&t, e0, e1);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (rc == 0) {
        *ms = t;
        cover_all(s, 0, count, true);
    }
    return rc;
}

int iris_session_time_decode(IrisSession* s, const int32_t* prompt, uint32_t prompt_len, uint32_t steps,
                             double* ms_per_token, double* prefill_ms, int32_t* out_tokens) {
    return iris_session_time_decode_launches(s, prompt, prompt_len, steps, 1, ms_per_token, prefill_ms, out_tokens);
}

int iris_session_time_decode_launches(IrisSession* s, const int32_t* prompt, uint32_t prompt_len, uint32_t steps,
                                      int use_graph, double* ms_per_token, double* prefill_ms, int32_t* out_tokens) {
    if (!s || !prompt || !ms_per_token || steps == 0) return IRIS_E_INVALID;
    const IrisModelDesc& d = s->model->d;
    if (prompt_len == 0 || prompt_len > s->max_rows) return IRIS_E_RANGE;
    const uint64_t end = (uint64_t)prompt_len + steps;
    if (end > s->max_positions || end > d.max_positions) return IRIS_E_RANGE;
    if (use_graph && kernel_tracer_loaded()) return IRIS_E_TRACED;
    s->keep_logits = false;
    hipEvent_t e0 = nullptr, e1 = nullptr, e2 = nullptr;
    RT_CHECK(hipEventCreate(&e0));
    RT_CHECK(hipEventCreate(&e1));
    RT_CHECK(hipEventCreate(&e2));
    uncover_all(s, 0, (uint32_t)end, true);
    int rc = session_reset_and_embed(s, prompt, prompt_len);
    if (rc == 0) rc = (int)hipEventRecord(e0, s->stream);
    if (rc == 0) rc = session_pass(s, prompt_len, nullptr);
    if (rc == 0) rc = session_head_select(s, prompt_len);
    // Capture (outside the timed region) before timing the replays.
    if (rc == 0) rc = (int)hipEventRecord(e1, s->stream);
    if (rc == 0 && use_graph) rc = ensure_graph(s, true);
    float pre = 0.f, dec = 0.f;
    if (rc == 0) rc = (int)hipEventSynchronize(e1);
    if (rc == 0) rc = (int)hipEventElapsedTime(&pre, e0, e1);
    if (rc == 0) rc = (int)hipEventRecord(e1, s->stream);
    for (uint32_t t = 0; rc == 0 && t < steps; t++)
        rc = use_graph ? (int)hipGraphLaunch(s->graph_exec, s->stream) : session_decode_pass(s, 0);
    if (rc == 0) rc = (int)hipEventRecord(e2, s->stream);
    if (rc == 0) rc = (int)hipEventSynchronize(e2);
    if (rc == 0) rc = (int)hipEventElapsedTime(&dec, e1, e2);
    if (rc == 0 && out_tokens)
        rc = (int)hipMemcpy(out_tokens, s->tokens, (size_t)(steps + 1) * 4, hipMemcpyDeviceToHost);
    if (rc == 0 && (!s->model->embed_bad.empty() || !s->model->ple_bad.empty())) {
        // The selections the timed passes embedded (all but the last).
        std::vector<int32_t> ids(steps + 1);
        rc = (int)hipMemcpy(ids.data(), s->tokens, (size_t)(steps + 1) * 4, hipMemcpyDeviceToHost);
        for (uint32_t t = 0; rc == 0 && t < steps; t++)
            if (embedding_refused(s->model, ids[t])) rc = IRIS_E_SCALE;
    }
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    hipEventDestroy(e2);
    if (rc == 0) {
        *ms_per_token = dec / steps;
        if (prefill_ms) *prefill_ms = pre;
        cover_all(s, 0, (uint32_t)end, true);
    }
    return rc;
}

}  // extern "C"
