// The non-product kernels of the token loop: exact attention over the
// device KV cache, the greedy select + next-row embedding, and the prompt
// embedding gather.
#include "detnum_dev.h"
#include "layer_kernels.h"

namespace {

constexpr int ATTN_THREADS = 256;

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

// One (query head, query row) per workgroup. Scores over the visible keys,
// the det-num softmax (ops.rs:233-261), and the weighted values
// (ops.rs:339-355; mistral/layer.rs:304-315; prefill_range.rs:816-844).
__global__ __launch_bounds__(ATTN_THREADS) void attention_kernel(const AttnArgs a) {
    __shared__ int32_t s_w[ATTN_MAX_KEYS];
    __shared__ int64_t s_e[ATTN_MAX_KEYS];
    __shared__ int32_t s_q[ATTN_MAX_HEAD_DIM];
    __shared__ ArgMax s_am[ATTN_THREADS / 64];
    __shared__ int64_t s_sum[ATTN_THREADS / 64];
    __shared__ int32_t s_wsum[ATTN_THREADS / 64];
    __shared__ int64_t s_acc[ATTN_THREADS];

    const uint32_t head = blockIdx.x, token = blockIdx.y;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t hd = a.head_dim;
    const uint32_t kvh = head / (a.heads / a.kv_heads);
    const uint32_t pos = (uint32_t)(*a.d_pos) + token;
    const uint32_t start = (a.window == 0 || pos + 1 <= a.window) ? 0 : pos + 1 - a.window;
    const uint32_t n = pos - start + 1;
    const int32_t* q = a.q + (size_t)token * a.q_stride + (size_t)head * hd;
    for (uint32_t d = tid; d < hd; d += ATTN_THREADS) s_q[d] = q[d];
    __syncthreads();

    // Scores, and this thread's first maximum.
    ArgMax best{INT32_MIN, 0xffffffffu};
    for (uint32_t j = tid; j < n; j += ATTN_THREADS) {
        const int32_t* k = a.k_cache + (size_t)(start + j) * a.kv_stride + (size_t)kvh * hd;
        uint64_t sum = 0;  // wrapping i64 (mac_bits, ops.rs:17-19)
        for (uint32_t d = 0; d < hd; d += 4) {
            const int4 kk = *(const int4*)(k + d);
            sum += (uint64_t)((int64_t)s_q[d] * kk.x) + (uint64_t)((int64_t)s_q[d + 1] * kk.y) +
                   (uint64_t)((int64_t)s_q[d + 2] * kk.z) + (uint64_t)((int64_t)s_q[d + 3] * kk.w);
        }
        const int32_t s = a.scaled ? dn::scaled_score_from_sum((int64_t)sum, a.scale_q32)
                                   : dn::requantize((int64_t)sum);
        s_w[j] = s;
        best = argmax_combine(best, ArgMax{s, j});
    }
    best = wave_argmax(best);
    if (lane == 0) s_am[wave] = best;
    __syncthreads();
    ArgMax m = s_am[0];
    for (int i = 1; i < ATTN_THREADS / 64; i++) m = argmax_combine(m, s_am[i]);

    // exp terms and their saturating sum (non-negative terms: order-free).
    int64_t part = 0;
    for (uint32_t j = tid; j < n; j += ATTN_THREADS) {
        const int64_t delta = (int64_t)dn::sub_sat(s_w[j], m.v) * 65536;
        const int64_t e = dn::softmax_exp_term(delta);
        s_e[j] = e;
        part = dn::acc_add_sat(part, e);
    }
    part = wave_sum_sat64(part);
    if (lane == 0) s_sum[wave] = part;
    __syncthreads();
    int64_t total = 0;
    for (int i = 0; i < ATTN_THREADS / 64; i++) total = dn::acc_add_sat(total, s_sum[i]);

    // weights requantize(div_acc(e, sum)) and their saturating sum.
    int32_t wpart = 0;
    for (uint32_t j = tid; j < n; j += ATTN_THREADS) {
        const int32_t w = dn::requantize(dn::div_acc_softmax((uint64_t)s_e[j], (uint64_t)total));
        s_w[j] = w;
        wpart = dn::add_sat(wpart, w);
    }
    wpart = wave_sum_sat32(wpart);
    if (lane == 0) s_wsum[wave] = wpart;
    __syncthreads();
    if (tid == 0) {
        int32_t ws = 0;
        for (int i = 0; i < ATTN_THREADS / 64; i++) ws = dn::add_sat(ws, s_wsum[i]);
        s_w[m.i] = dn::add_sat(s_w[m.i], dn::sub_sat(dn::ONE_ACT, ws));
    }
    __syncthreads();

    // ctx[d] = requantize(sum_j w_j v_j[d]), wrapping i64; the keys are
    // split over ATTN_THREADS / head_dim groups of threads.
    const uint32_t groups = ATTN_THREADS / hd;
    const uint32_t grp = tid / hd, d = tid % hd;
    if (grp < groups) {
        uint64_t acc = 0;
        for (uint32_t j = grp; j < n; j += groups) {
            const int32_t* v = a.v_cache + (size_t)(start + j) * a.kv_stride + (size_t)kvh * hd;
            acc += (uint64_t)((int64_t)s_w[j] * v[d]);
        }
        s_acc[grp * hd + d] = (int64_t)acc;
    }
    __syncthreads();
    if (tid < hd) {
        uint64_t acc = 0;
        for (uint32_t i = 0; i < groups; i++) acc += (uint64_t)s_acc[i * hd + tid];
        a.ctx[(size_t)token * a.ctx_stride + (size_t)head * hd + tid] = dn::requantize((int64_t)acc);
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

constexpr int SELECT_THREADS = 1024;

// Greedy selection (generation.rs:25-57) of the pass's logits, then the next
// pass's input row: the selected token's embedding. Advances the position by
// the rows the pass processed and the step counter by one.
__global__ __launch_bounds__(SELECT_THREADS) void select_embed_kernel(const SelectArgs a) {
    __shared__ ArgMax s_am[SELECT_THREADS / 64];
    __shared__ uint32_t s_token;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t step = *a.d_step;
    ArgMax best{INT32_MIN, 0xffffffffu};
    for (uint32_t i = tid; i < a.vocab; i += SELECT_THREADS) best = argmax_combine(best, ArgMax{a.logits[i], i});
    best = wave_argmax(best);
    if (lane == 0) s_am[wave] = best;
    if (a.logits_keep)
        for (uint32_t i = tid; i < a.vocab; i += SELECT_THREADS)
            a.logits_keep[(size_t)step * a.vocab + i] = a.logits[i];
    __syncthreads();
    if (tid == 0) {
        ArgMax m = s_am[0];
        for (int i = 1; i < SELECT_THREADS / 64; i++) m = argmax_combine(m, s_am[i]);
        s_token = m.i;
        a.tokens_out[step] = (int32_t)m.i;
    }
    __syncthreads();
    const uint32_t token = s_token;
    embed_row(a.embed_raw + (size_t)token * a.row_bytes, a.hidden, a.embed_scale, a.x_next, tid, SELECT_THREADS);
    __syncthreads();
    if (tid == 0) {
        *a.d_step = step + 1;
        *a.d_pos = *a.d_pos + (int32_t)a.rows_in_pass;
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
    hipLaunchKernelGGL(attention_kernel, dim3(a.heads, tokens), dim3(ATTN_THREADS), 0, stream, a);
    return (int)hipGetLastError();
}

int iris_select_embed_launch(const SelectArgs& a, hipStream_t stream) {
    hipLaunchKernelGGL(select_embed_kernel, dim3(1), dim3(SELECT_THREADS), 0, stream, a);
    return (int)hipGetLastError();
}

int iris_embed_rows_launch(const int32_t* d_ids, uint32_t count, const uint8_t* embed_raw, uint32_t row_bytes,
                           uint32_t hidden, int32_t scale, int32_t* out, hipStream_t stream) {
    if (count == 0) return 0;
    hipLaunchKernelGGL(embed_rows_kernel, dim3(count), dim3(256), 0, stream, d_ids, embed_raw, row_bytes, hidden,
                       scale, out);
    return (int)hipGetLastError();
}
