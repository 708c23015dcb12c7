// Shared pieces of the attention kernels: first-maximum and saturating
// reductions, and the scalar attention of one (head, query row) that the
// multi-row paths fall back on.
#pragma once

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

// The LDS one attend_row call uses.
struct AttnRowSmem {
    int32_t w[ATTN_TILE_KEYS];
    int64_t e[ATTN_TILE_KEYS];
    int32_t q[ATTN_MAX_HEAD_DIM];
    int64_t part[ATTN_MAX_THREADS];
    ArgMax am[ATTN_MAX_WAVES];
    int64_t sum[ATTN_MAX_WAVES];
    int32_t wsum[ATTN_MAX_WAVES];
};

// The scores of one round of keys base + [0, per_round) of a view (the
// row's query in s_q): one key per lane and a quarter of the head's
// dimensions per wave (independent coalesced loads from the transposed K
// cache), the quarters summed through LDS; f(index, score) runs on thread
// index < per_round for each key of the view. Two barriers.
template <class F>
__device__ __forceinline__ void attend_round(const AttnArgs& a, const int32_t* kt, const int32_t* s_q, int64_t* s_part,
                                             uint32_t base, uint32_t n, F&& f) {
    constexpr uint32_t QS = 4;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x / 64;
    const uint32_t per_round = 64 * (nwaves / QS), dq = a.head_dim / QS;
    const uint32_t kg = wave / QS, qd = wave % QS;
    const uint32_t key = base + kg * 64 + lane;
    uint64_t acc = 0;  // wrapping i64 (mac_bits, ops.rs:17-19)
    if (key < n) {
        const int32_t* kk = kt + (size_t)qd * dq * a.k_pos_stride + key;
#pragma unroll 16
        for (uint32_t i = 0; i < dq; i++) acc += (uint64_t)((int64_t)s_q[qd * dq + i] * kk[(size_t)i * a.k_pos_stride]);
    }
    s_part[qd * per_round + kg * 64 + lane] = (int64_t)acc;
    __syncthreads();
    if (tid < per_round && base + tid < n) {
        uint64_t sum = 0;
#pragma unroll
        for (uint32_t i = 0; i < QS; i++) sum += (uint64_t)s_part[i * per_round + tid];
        f(tid, a.scaled ? dn::scaled_score_from_sum((int64_t)sum, a.scale_q32) : dn::requantize((int64_t)sum));
    }
    __syncthreads();
}

// attend_row for a view longer than ATTN_TILE_KEYS: the scores are formed
// three times (first maximum; exp sum; weights and weighted values tile by
// tile), and the first maximum's residual is added at the end as resid * v
// (the weighted sum is linear and wraps, so this equals the reference's
// adjusted weight, ops.rs:258-260).
__device__ inline void attend_row_long(const AttnArgs& a, uint32_t head, uint32_t token, AttnRowSmem& sm,
                                       uint32_t start, uint32_t n) {
    const uint32_t nthreads = blockDim.x, nwaves = nthreads / 64;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t hd = a.head_dim, kvh = head / (a.heads / a.kv_heads);
    const uint32_t per_round = 64 * (nwaves / 4);
    const int32_t* kt = a.k_cache + (size_t)kvh * hd * a.k_pos_stride + start;
    ArgMax best{INT32_MIN, 0xffffffffu};
    for (uint32_t base = 0; base < n; base += per_round)
        attend_round(a, kt, sm.q, sm.part, base, n,
                     [&](uint32_t i, int32_t sc) { best = argmax_combine(best, ArgMax{sc, base + i}); });
    best = wave_argmax(best);
    if (lane == 0) sm.am[wave] = best;
    __syncthreads();
    ArgMax m = sm.am[0];
    for (uint32_t i = 1; i < nwaves; i++) m = argmax_combine(m, sm.am[i]);
    auto exp_term = [&](int32_t sc) -> int64_t {
        const int64_t diff = (int64_t)m.v - sc;  // >= 0: m is the maximum
        return (int64_t)dn::softmax_exp_diff((uint32_t)(diff > (1 << 20) ? (1 << 20) : diff));
    };
    int64_t part = 0;
    for (uint32_t base = 0; base < n; base += per_round)
        attend_round(a, kt, sm.q, sm.part, base, n,
                     [&](uint32_t, int32_t sc) { part = dn::acc_add_sat(part, exp_term(sc)); });
    part = wave_sum_sat64(part);
    if (lane == 0) sm.sum[wave] = part;
    __syncthreads();
    int64_t total = 0;
    for (uint32_t i = 0; i < nwaves; i++) total = dn::acc_add_sat(total, sm.sum[i]);
    const double w_scale = 65536.0 / (double)total, q_scale = 4294967296.0 / (double)total;

    const uint32_t groups = nthreads / hd, grp = tid / hd, d = tid % hd;
    const int32_t* vb = a.v_cache + (size_t)start * a.kv_stride + (size_t)kvh * hd + d;
    int32_t wpart = 0;
    uint64_t acc = 0;
    for (uint32_t t0 = 0; t0 < n; t0 += ATTN_TILE_KEYS) {
        const uint32_t tn = min(ATTN_TILE_KEYS, n - t0);
        for (uint32_t base = 0; base < tn; base += per_round)
            attend_round(a, kt + t0, sm.q, sm.part, base, tn, [&](uint32_t i, int32_t sc) {
                const int32_t w = dn::softmax_weight_fast((uint64_t)exp_term(sc), (uint64_t)total, w_scale, q_scale);
                sm.w[base + i] = w;
                wpart = dn::add_sat(wpart, w);
            });
        if (grp < groups)
            for (uint32_t j = grp; j < tn; j += groups)
                acc += (uint64_t)((int64_t)sm.w[j] * vb[(size_t)(t0 + j) * a.kv_stride]);
        __syncthreads();
    }
    wpart = wave_sum_sat32(wpart);
    if (lane == 0) sm.wsum[wave] = wpart;
    sm.part[tid] = (int64_t)acc;
    __syncthreads();
    if (tid < hd) {
        int32_t ws = 0;
        for (uint32_t i = 0; i < nwaves; i++) ws = dn::add_sat(ws, sm.wsum[i]);
        uint64_t t = 0;
        for (uint32_t i = 0; i < groups; i++) t += (uint64_t)sm.part[i * hd + tid];
        const int64_t resid = dn::sub_sat(dn::ONE_ACT, ws);
        t += (uint64_t)(resid * a.v_cache[(size_t)(start + m.i) * a.kv_stride + (size_t)kvh * hd + tid]);
        a.ctx[(size_t)token * a.ctx_stride + (size_t)head * hd + tid] = dn::requantize((int64_t)t);
    }
    __syncthreads();
}

// One (query head, query row) by the whole workgroup of blockDim.x threads (a
// multiple of 256, at most 1024, at least head_dim). Scores over the visible keys: each round takes
// 64 * waves/4 keys, one key per lane and a quarter of the head's dimensions
// per wave (independent coalesced loads from the transposed K cache), the four
// quarters summed through LDS. Then the det-num softmax (ops.rs:233-261) and
// the weighted values (ops.rs:339-355; mistral/layer.rs:304-315;
// prefill_range.rs:816-844), one head dimension per thread.
__device__ inline void attend_row(const AttnArgs& a, uint32_t head, uint32_t token, AttnRowSmem& sm) {
    constexpr uint32_t QS = 4;  // dimension quarters per key
    int32_t* s_w = sm.w;
    int64_t* s_e = sm.e;
    int32_t* s_q = sm.q;
    int64_t* s_part = sm.part;
    ArgMax* s_am = sm.am;
    int64_t* s_sum = sm.sum;
    int32_t* s_wsum = sm.wsum;

    const uint32_t nthreads = blockDim.x, nwaves = nthreads / 64;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t hd = a.head_dim, dq = hd / QS;
    const uint32_t kvh = head / (a.heads / a.kv_heads);
    const uint32_t pos = (uint32_t)(*a.d_pos) + token;
    const uint32_t start = (a.window == 0 || pos + 1 <= a.window) ? 0 : pos + 1 - a.window;
    const uint32_t n = pos - start + 1;
    const int32_t* q = a.q + (size_t)token * a.q_stride + (size_t)head * hd;
    for (uint32_t d = tid; d < hd; d += nthreads) s_q[d] = q[d];
    __syncthreads();
    if (n > ATTN_TILE_KEYS) {  // uniform over the workgroup
        attend_row_long(a, head, token, sm, start, n);
        return;
    }

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
        const int64_t diff = (int64_t)m.v - s_w[j];  // >= 0: m is the maximum
        const int64_t e = (int64_t)dn::softmax_exp_diff((uint32_t)(diff > (1 << 20) ? (1 << 20) : diff));
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
    const double w_scale = 65536.0 / (double)total, q_scale = 4294967296.0 / (double)total;
    for (uint32_t j = tid; j < n; j += nthreads) {
        const int32_t w = dn::softmax_weight_fast((uint64_t)s_e[j], (uint64_t)total, w_scale, q_scale);
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
    __syncthreads();
}

}  // namespace
