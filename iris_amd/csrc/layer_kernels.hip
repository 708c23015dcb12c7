// The non-product kernels of the token loop: exact attention over the
// device KV cache and the prompt embedding gather.
#include "detnum_dev.h"
#include "layer_kernels.h"

namespace {

constexpr int ATTN_MAX_THREADS = 1024;
constexpr int ATTN_MAX_WAVES = ATTN_MAX_THREADS / 64;

struct ArgMax {
    int32_t v;
    uint32_t i;
};

// First maximum: larger value wins, equal values keep the smaller index
// (crates/det-num/src/ops.rs:466-481; crates/inference/direct/src/generation.rs:25-33).
__device__ __forceinline__ ArgMax argmax_combine(ArgMax a, ArgMax b) {
    if (b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
    return a;
}

__device__ __forceinline__ ArgMax wave_argmax(ArgMax a) {
    for (int off = 32; off >= 1; off >>= 1) {
        ArgMax o{__shfl_xor(a.v, off), (uint32_t)__shfl_xor((int)a.i, off)};
        a = argmax_combine(a, o);
    }
    return a;
}

__device__ __forceinline__ int64_t wave_sum_sat64(int64_t v) {
    for (int off = 32; off >= 1; off >>= 1) v = dn::acc_add_sat(v, __shfl_xor(v, off));
    return v;
}

__device__ __forceinline__ int32_t wave_sum_sat32(int32_t v) {
    for (int off = 32; off >= 1; off >>= 1) v = dn::add_sat(v, __shfl_xor(v, off));
    return v;
}

// One (query head, query row) per workgroup of blockDim.x threads (a multiple
// of 256, at most 1024). Scores over the visible keys: each round takes
// 64 * waves/4 keys, one key per lane and a quarter of the head's dimensions
// per wave (independent coalesced loads from the transposed K cache), the four
// quarters summed through LDS. Then the det-num softmax (ops.rs:233-261) and
// the weighted values (ops.rs:339-355; mistral/layer.rs:304-315;
// prefill_range.rs:816-844), one head dimension per thread.
__global__ __launch_bounds__(ATTN_MAX_THREADS) void attention_kernel(const AttnArgs a) {
    constexpr uint32_t QS = 4;  // dimension quarters per key
    __shared__ int32_t s_w[ATTN_MAX_KEYS];
    __shared__ int64_t s_e[ATTN_MAX_KEYS];
    __shared__ int32_t s_q[ATTN_MAX_HEAD_DIM];
    __shared__ int64_t s_part[ATTN_MAX_THREADS];
    __shared__ ArgMax s_am[ATTN_MAX_WAVES];
    __shared__ int64_t s_sum[ATTN_MAX_WAVES];
    __shared__ int32_t s_wsum[ATTN_MAX_WAVES];

    const uint32_t nthreads = blockDim.x, nwaves = nthreads / 64;
    const uint32_t head = blockIdx.x, token = blockIdx.y;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t hd = a.head_dim, dq = hd / QS;
    const uint32_t kvh = head / (a.heads / a.kv_heads);
    const uint32_t pos = (uint32_t)(*a.d_pos) + token;
    const uint32_t start = (a.window == 0 || pos + 1 <= a.window) ? 0 : pos + 1 - a.window;
    const uint32_t n = pos - start + 1;
    const int32_t* q = a.q + (size_t)token * a.q_stride + (size_t)head * hd;
    for (uint32_t d = tid; d < hd; d += nthreads) s_q[d] = q[d];
    __syncthreads();

    // Scores, and the first maximum of the keys this thread finishes.
    const uint32_t per_round = 64 * (nwaves / QS);
    const uint32_t kg = wave / QS, qd = wave % QS;
    const int32_t* kt = a.k_cache + ((size_t)kvh * hd + (size_t)qd * dq) * a.k_pos_stride + start;
    ArgMax best{INT32_MIN, 0xffffffffu};
    for (uint32_t base = 0; base < n; base += per_round) {
        const uint32_t key = base + kg * 64 + lane;
        uint64_t acc = 0;  // wrapping i64 (mac_bits, ops.rs:17-19)
        if (key < n) {
            const int32_t* kk = kt + key;
#pragma unroll 16
            for (uint32_t i = 0; i < dq; i++)
                acc += (uint64_t)((int64_t)s_q[qd * dq + i] * kk[(size_t)i * a.k_pos_stride]);
        }
        s_part[qd * per_round + kg * 64 + lane] = (int64_t)acc;
        __syncthreads();
        if (tid < per_round && base + tid < n) {
            uint64_t sum = 0;
#pragma unroll
            for (uint32_t i = 0; i < QS; i++) sum += (uint64_t)s_part[i * per_round + tid];
            const int32_t sc = a.scaled ? dn::scaled_score_from_sum((int64_t)sum, a.scale_q32)
                                        : dn::requantize((int64_t)sum);
            s_w[base + tid] = sc;
            best = argmax_combine(best, ArgMax{sc, base + tid});
        }
        __syncthreads();
    }
    best = wave_argmax(best);
    if (lane == 0) s_am[wave] = best;
    __syncthreads();
    ArgMax m = s_am[0];
    for (uint32_t i = 1; i < nwaves; i++) m = argmax_combine(m, s_am[i]);

    // exp terms and their saturating sum (non-negative terms: order-free).
    int64_t part = 0;
    for (uint32_t j = tid; j < n; j += nthreads) {
        const int64_t delta = (int64_t)dn::sub_sat(s_w[j], m.v) * 65536;
        const int64_t e = dn::softmax_exp_term(delta);
        s_e[j] = e;
        part = dn::acc_add_sat(part, e);
    }
    part = wave_sum_sat64(part);
    if (lane == 0) s_sum[wave] = part;
    __syncthreads();
    int64_t total = 0;
    for (uint32_t i = 0; i < nwaves; i++) total = dn::acc_add_sat(total, s_sum[i]);

    // weights requantize(div_acc(e, sum)) and their saturating sum.
    int32_t wpart = 0;
    for (uint32_t j = tid; j < n; j += nthreads) {
        const int32_t w = dn::requantize(dn::div_acc_softmax((uint64_t)s_e[j], (uint64_t)total));
        s_w[j] = w;
        wpart = dn::add_sat(wpart, w);
    }
    wpart = wave_sum_sat32(wpart);
    if (lane == 0) s_wsum[wave] = wpart;
    __syncthreads();
    if (tid == 0) {
        int32_t ws = 0;
        for (uint32_t i = 0; i < nwaves; i++) ws = dn::add_sat(ws, s_wsum[i]);
        s_w[m.i] = dn::add_sat(s_w[m.i], dn::sub_sat(dn::ONE_ACT, ws));
    }
    __syncthreads();

    // ctx[d] = requantize(sum_j w_j v_j[d]), wrapping i64; the keys are split
    // over nthreads / head_dim groups of threads.
    const uint32_t groups = nthreads / hd;
    const uint32_t grp = tid / hd, d = tid % hd;
    uint64_t acc = 0;
    if (grp < groups) {
        const int32_t* vb = a.v_cache + (size_t)start * a.kv_stride + (size_t)kvh * hd + d;
#pragma unroll 8
        for (uint32_t j = grp; j < n; j += groups) acc += (uint64_t)((int64_t)s_w[j] * vb[(size_t)j * a.kv_stride]);
    }
    s_part[tid] = (int64_t)acc;
    __syncthreads();
    if (tid < hd) {
        uint64_t t = 0;
        for (uint32_t i = 0; i < groups; i++) t += (uint64_t)s_part[i * hd + tid];
        a.ctx[(size_t)token * a.ctx_stride + (size_t)head * hd + tid] = dn::requantize((int64_t)t);
    }
}

// ---- split decode attention: one query row, each head over key chunks ----

// Scores of one chunk of keys (512 threads: two groups of 64 keys, four
// dimension quarters each), and the chunk's first maximum.
__global__ __launch_bounds__(512) void attn_chunk_scores_kernel(const AttnArgs a) {
    constexpr uint32_t QS = 4;
    __shared__ int32_t s_q[ATTN_MAX_HEAD_DIM];
    __shared__ int64_t s_part[512];
    __shared__ ArgMax s_am[8];
    const uint32_t head = blockIdx.x, chunk = blockIdx.z;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t hd = a.head_dim, dq = hd / QS;
    const uint32_t kvh = head / (a.heads / a.kv_heads);
    const uint32_t pos = (uint32_t)(*a.d_pos);
    const uint32_t start = (a.window == 0 || pos + 1 <= a.window) ? 0 : pos + 1 - a.window;
    const uint32_t n = pos - start + 1;
    const uint32_t c0 = chunk * ATTN_CHUNK;
    if (c0 >= n) return;
    for (uint32_t d = tid; d < hd; d += 512) s_q[d] = a.q[(size_t)head * hd + d];
    __syncthreads();
    const uint32_t kg = wave / QS, qd = wave % QS;
    const uint32_t key = c0 + kg * 64 + lane;
    uint64_t acc = 0;
    if (key < n) {
        const int32_t* kk = a.k_cache + ((size_t)kvh * hd + (size_t)qd * dq) * a.k_pos_stride + start + key;
#pragma unroll 16
        for (uint32_t i = 0; i < dq; i++) acc += (uint64_t)((int64_t)s_q[qd * dq + i] * kk[(size_t)i * a.k_pos_stride]);
    }
    s_part[qd * ATTN_CHUNK + kg * 64 + lane] = (int64_t)acc;
    __syncthreads();
    ArgMax best{INT32_MIN, 0xffffffffu};
    if (tid < ATTN_CHUNK && c0 + tid < n) {
        uint64_t sum = 0;
        for (uint32_t i = 0; i < QS; i++) sum += (uint64_t)s_part[i * ATTN_CHUNK + tid];
        const int32_t sc = a.scaled ? dn::scaled_score_from_sum((int64_t)sum, a.scale_q32) : dn::requantize((int64_t)sum);
        a.scores[(size_t)head * ATTN_MAX_KEYS + c0 + tid] = sc;
        best = ArgMax{sc, c0 + tid};
    }
    best = wave_argmax(best);
    if (lane == 0) s_am[wave] = best;
    __syncthreads();
    if (tid == 0) {
        ArgMax m = s_am[0];
        for (int i = 1; i < 8; i++) m = argmax_combine(m, s_am[i]);
        a.chunk_max[(size_t)head * ATTN_MAX_CHUNKS + chunk] = ((uint64_t)m.i << 32) | (uint32_t)m.v;
    }
}

// Softmax over the head's scores (recomputed in every chunk's workgroup:
// the global first maximum from the chunk records, every exp term for the
// sum), then this chunk's weights, their sum and its weighted values.
__global__ __launch_bounds__(256) void attn_chunk_softmax_pv_kernel(const AttnArgs a) {
    __shared__ int32_t s_w[ATTN_CHUNK];
    __shared__ int64_t s_part[256 * 4];
    __shared__ int64_t s_sum[4];
    __shared__ int32_t s_wsum[4];
    const uint32_t head = blockIdx.x, chunk = blockIdx.z;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t hd = a.head_dim;
    const uint32_t kvh = head / (a.heads / a.kv_heads);
    const uint32_t pos = (uint32_t)(*a.d_pos);
    const uint32_t start = (a.window == 0 || pos + 1 <= a.window) ? 0 : pos + 1 - a.window;
    const uint32_t n = pos - start + 1;
    const uint32_t nchunks = (n + ATTN_CHUNK - 1) / ATTN_CHUNK;
    const uint32_t c0 = chunk * ATTN_CHUNK;
    if (c0 >= n) return;
    const int32_t* sc = a.scores + (size_t)head * ATTN_MAX_KEYS;

    // The first maximum over the chunk records (chunks in key order).
    ArgMax m{INT32_MIN, 0xffffffffu};
    for (uint32_t c = 0; c < nchunks; c++) {
        const uint64_t r = a.chunk_max[(size_t)head * ATTN_MAX_CHUNKS + c];
        m = argmax_combine(m, ArgMax{(int32_t)(uint32_t)r, (uint32_t)(r >> 32)});
    }
    // sum_sat of every exp term (non-negative: order-free).
    int64_t part = 0;
    for (uint32_t j = tid; j < n; j += 256)
        part = dn::acc_add_sat(part, dn::softmax_exp_term((int64_t)dn::sub_sat(sc[j], m.v) * 65536));
    part = wave_sum_sat64(part);
    if (lane == 0) s_sum[wave] = part;
    __syncthreads();
    int64_t total = 0;
    for (int i = 0; i < 4; i++) total = dn::acc_add_sat(total, s_sum[i]);
    // This chunk's weights and their saturating sum.
    const uint32_t cn = min(ATTN_CHUNK, n - c0);
    int32_t wpart = 0;
    if (tid < cn) {
        const int64_t e = dn::softmax_exp_term((int64_t)dn::sub_sat(sc[c0 + tid], m.v) * 65536);
        const int32_t w = dn::requantize(dn::div_acc_softmax((uint64_t)e, (uint64_t)total));
        s_w[tid] = w;
        wpart = w;
        if (c0 + tid == m.i) a.max_weight[head] = w;
    }
    wpart = wave_sum_sat32(wpart);
    if (lane == 0) s_wsum[wave] = wpart;
    __syncthreads();
    // Weighted values of the chunk: four dimensions per thread, keys split
    // over 256 / (head_dim / 4) groups.
    const uint32_t dg = hd / 4, groups = 256 / dg;
    const uint32_t gi = tid / dg, d4 = (tid % dg) * 4;
    uint64_t acc[4] = {0, 0, 0, 0};
    if (gi < groups) {
        const int32_t* vb = a.v_cache + (size_t)(start + c0) * a.kv_stride + (size_t)kvh * hd + d4;
#pragma unroll 8
        for (uint32_t j = gi; j < cn; j += groups) {
            const int4 v = *(const int4*)(vb + (size_t)j * a.kv_stride);
            const int64_t w = s_w[j];
            acc[0] += (uint64_t)(w * v.x);
            acc[1] += (uint64_t)(w * v.y);
            acc[2] += (uint64_t)(w * v.z);
            acc[3] += (uint64_t)(w * v.w);
        }
    }
    for (int i = 0; i < 4; i++) s_part[tid * 4 + i] = (int64_t)acc[i];
    __syncthreads();
    if (tid < hd) {
        const uint32_t t_dg = tid / 4, t_i = tid % 4;
        uint64_t t = 0;
        for (uint32_t g = 0; g < groups; g++) t += (uint64_t)s_part[(g * dg + t_dg) * 4 + t_i];
        a.chunk_acc[((size_t)head * ATTN_MAX_CHUNKS + chunk) * hd + tid] = (int64_t)t;
    }
    if (tid == 0) {
        int32_t ws = 0;
        for (int i = 0; i < 4; i++) ws = dn::add_sat(ws, s_wsum[i]);
        a.chunk_wsum[(size_t)head * ATTN_MAX_CHUNKS + chunk] = ws;
    }
}

// Combines one head's chunk partials: the saturating sum of the chunk weight
// sums, the residual on the first maximum as an exact correction term
// (its weight changes from w to add_sat(w, ONE - sum)), and the rounding.
__global__ __launch_bounds__(256) void attn_chunk_combine_kernel(const AttnArgs a) {
    const uint32_t head = blockIdx.x, tid = threadIdx.x;
    const uint32_t hd = a.head_dim;
    const uint32_t kvh = head / (a.heads / a.kv_heads);
    const uint32_t pos = (uint32_t)(*a.d_pos);
    const uint32_t start = (a.window == 0 || pos + 1 <= a.window) ? 0 : pos + 1 - a.window;
    const uint32_t n = pos - start + 1;
    const uint32_t nchunks = (n + ATTN_CHUNK - 1) / ATTN_CHUNK;
    ArgMax m{INT32_MIN, 0xffffffffu};
    int32_t ws = 0;
    for (uint32_t c = 0; c < nchunks; c++) {
        const uint64_t r = a.chunk_max[(size_t)head * ATTN_MAX_CHUNKS + c];
        m = argmax_combine(m, ArgMax{(int32_t)(uint32_t)r, (uint32_t)(r >> 32)});
        ws = dn::add_sat(ws, a.chunk_wsum[(size_t)head * ATTN_MAX_CHUNKS + c]);
    }
    const int32_t wm = a.max_weight[head];
    const int64_t fix = (int64_t)dn::add_sat(wm, dn::sub_sat(dn::ONE_ACT, ws)) - wm;
    for (uint32_t d = tid; d < hd; d += 256) {
        uint64_t t = 0;
        for (uint32_t c = 0; c < nchunks; c++) t += (uint64_t)a.chunk_acc[((size_t)head * ATTN_MAX_CHUNKS + c) * hd + d];
        t += (uint64_t)fix * (uint64_t)(int64_t)a.v_cache[(size_t)(start + m.i) * a.kv_stride + (size_t)kvh * hd + d];
        a.ctx[(size_t)head * hd + d] = dn::requantize((int64_t)t);
    }
}

// Dequantize one Q8_0 row (reference layout) into out[0..cols) (q8.rs:76-92),
// optionally times a Q16.16 scale (model.rs:316-330).
__device__ __forceinline__ void embed_row(const uint8_t* row, uint32_t cols, int32_t scale, int32_t* out,
                                          uint32_t tid, uint32_t nthreads) {
    for (uint32_t c = tid; c < cols; c += nthreads) {
        const uint8_t* blk = row + (size_t)(c / 32) * 34;
        const int64_t s = dn::scale_q24((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        int32_t v = dn::round_to_i32((dn::i128)((int64_t)(int8_t)blk[2 + c % 32] * s), 8);
        if (scale != 0) v = dn::mul_sat(v, scale);
        out[c] = v;
    }
}

// Embedding rows of `count` token ids (view_kernels.rs:14-35).
__global__ void embed_rows_kernel(const int32_t* ids, const uint8_t* embed_raw, uint32_t row_bytes,
                                  uint32_t hidden, int32_t scale, int32_t* out) {
    const uint32_t t = blockIdx.x;
    embed_row(embed_raw + (size_t)ids[t] * row_bytes, hidden, scale, out + (size_t)t * hidden, threadIdx.x,
              blockDim.x);
}

}  // namespace

int iris_attention_launch(const AttnArgs& a, uint32_t tokens, uint32_t max_keys, hipStream_t stream) {
    if (a.head_dim > ATTN_MAX_HEAD_DIM || a.head_dim % 4 || max_keys > ATTN_MAX_KEYS || a.heads % a.kv_heads)
        return IRIS_E_INVALID;
    if (tokens == 1 && a.scores && a.head_dim <= 256 && a.head_dim % 16 == 0) {
        // One row: every head over chunks of keys, in two launches.
        const uint32_t chunks = (max_keys + ATTN_CHUNK - 1) / ATTN_CHUNK;
        hipLaunchKernelGGL(attn_chunk_scores_kernel, dim3(a.heads, 1, chunks), dim3(512), 0, stream, a);
        hipError_t st = hipGetLastError();
        if (st != hipSuccess) return (int)st;
        hipLaunchKernelGGL(attn_chunk_softmax_pv_kernel, dim3(a.heads, 1, chunks), dim3(256), 0, stream, a);
        st = hipGetLastError();
        if (st != hipSuccess) return (int)st;
        hipLaunchKernelGGL(attn_chunk_combine_kernel, dim3(a.heads), dim3(256), 0, stream, a);
        return (int)hipGetLastError();
    }
    const uint32_t threads = tokens == 1 ? 1024 : 256;
    if (threads < a.head_dim || a.head_dim % 4) return IRIS_E_INVALID;
    hipLaunchKernelGGL(attention_kernel, dim3(a.heads, tokens), dim3(threads), 0, stream, a);
    return (int)hipGetLastError();
}

int iris_embed_rows_launch(const int32_t* d_ids, uint32_t count, const uint8_t* embed_raw, uint32_t row_bytes,
                           uint32_t hidden, int32_t scale, int32_t* out, hipStream_t stream) {
    if (count == 0) return 0;
    hipLaunchKernelGGL(embed_rows_kernel, dim3(count), dim3(256), 0, stream, d_ids, embed_raw, row_bytes, hidden,
                       scale, out);
    return (int)hipGetLastError();
}
