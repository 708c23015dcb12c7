// The non-product kernels of the token loop: exact attention over the
// device KV cache and the prompt embedding gather.
#include <algorithm>
#include <map>
#include <numeric>
#include <mutex>

#include "act_planes.h"
#include "attn_common.h"
#include "detnum_dev.h"
#include "layer_kernels.h"
#include "wave_ops.h"

namespace {

// One (query head, query row) per workgroup.
__global__ __launch_bounds__(ATTN_MAX_THREADS) void attention_kernel(const AttnArgs a) {
    __shared__ AttnRowSmem sm;
    attend_row(a, blockIdx.x, blockIdx.y, sm);
}

// One query row in two launches. (1) attn_scores_kernel: one workgroup per
// (query head, 64-position chunk of the cache) forms the chunk's scores
// (wrapping i64 dot, then scaled_score or requantize) into a.scores; each
// workgroup reads only its chunk's keys, so the key bytes a head needs are
// spread over many compute units; each workgroup also leaves the first
// maximum of its keys. (2) attn_values_kernel: one workgroup per (query
// head, 32-dimension slice) takes the head's first maximum from those, reads
// the head's scores, forms the exp terms, their sum and the weights, then
// the weighted values of its slice over every key; the slice's value loads
// are issued right after the scores and stay in flight through the softmax.

// Thread (position quad kq, dimension group grp of 16) holds HD/16 dimensions
// of four consecutive positions: one 16-byte load per dimension from the
// transposed cache (consecutive lanes read consecutive positions of one
// dimension); the groups' partial sums meet by shuffles, then across the
// four waves in LDS.
// The decode kernels' workgroups in XCD order. A data unit is one KV head's
// chunk (scores) or dimension slice (values), read by the `group` query
// heads that share the KV head; workgroup L runs on XCD L % 8 (workgroups are
// dealt to the eight XCDs in turn). When the units fill the XCDs evenly,
// each unit's workgroups go to one XCD, so its keys or values come from
// memory once into that XCD's L2 rather than once per query head. Returns
// (query head, chunk or slice) of workgroup L of heads * per_head.
__device__ __forceinline__ uint2 xcd_head_order(const AttnArgs& a, uint32_t L, uint32_t per_head) {
    const uint32_t group = a.heads / a.kv_heads, units = a.kv_heads * per_head;
    uint32_t u, r;
    if (units % 8 == 0) {
        const uint32_t q = L / 8;
        u = L % 8 + 8 * (q / group);
        r = q % group;
    } else {
        u = L / group;
        r = L % group;
    }
    return make_uint2((u % a.kv_heads) * group + r, u / a.kv_heads);
}

// The first maximum of scores as 64-bit keys: the score with its sign bit
// flipped, then the complemented key index from the view's start, so that
// the larger key is the larger score and, among equal scores, the lower
// index (0 = no key).
__device__ __forceinline__ uint64_t max_key(int32_t score, uint32_t j) {
    return ((uint64_t)((uint32_t)score ^ 0x80000000u) << 32) | (uint32_t)~j;
}
__device__ __forceinline__ ArgMax from_max_key(uint64_t k) {
    return ArgMax{(int32_t)((uint32_t)(k >> 32) ^ 0x80000000u), ~(uint32_t)k};
}
// Each scores workgroup's first maximum, [heads][ATTN_DECODE_CHUNKS], after
// the scores (k_pos_stride is a multiple of 64: 256-byte aligned).
__device__ __forceinline__ uint64_t* chunk_maxima(const AttnArgs& a) {
    return (uint64_t*)(a.scores + (size_t)a.heads * a.k_pos_stride);
}

// Workgroup (head, y) takes the 64-position chunks y, y + chunks, ... of
// the view (one chunk each for views up to 64 * chunks keys), and leaves
// the first maximum of its visible keys in chunk_maxima.
template <uint32_t HD>
__global__ __launch_bounds__(256) void attn_scores_kernel(const AttnArgs a, uint32_t chunks) {
    constexpr uint32_t DPG = HD / 16;
    __shared__ int32_t s_q[HD];
    __shared__ uint64_t s_part[4][64];
    const uint2 hy = xcd_head_order(a, blockIdx.x, chunks);
    const uint32_t head = hy.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t pos = (uint32_t)(*a.d_pos);
    const uint32_t start = (a.window == 0 || pos + 1 <= a.window) ? 0 : pos + 1 - a.window;
    uint64_t* max_out = chunk_maxima(a) + (size_t)head * ATTN_DECODE_CHUNKS + hy.y;
    // The first chunk of this workgroup that holds a visible key (every
    // later one up to the position does too).
    uint32_t c = hy.y;
    if (c * 64 + 63 < start) {
        const uint32_t behind = start - (c * 64 + 63), step = 64 * chunks;
        c += (behind + step - 1) / step * chunks;
    }
    if (c * 64 > pos) {
        if (tid == 0) *max_out = 0;  // no key
        return;
    }
    const uint32_t kvh = head / (a.heads / a.kv_heads);
    // The query elements this thread stages (one, or two for head size 512),
    // loaded first (waiting for them does not wait for the key loads issued
    // after them).
    constexpr uint32_t QPT = HD > 256 ? HD / 256 : 1;
    int32_t qv[QPT];
#pragma unroll
    for (uint32_t u = 0; u < QPT; u++) qv[u] = a.q[(size_t)head * HD + (tid + 256 * u) % HD];
    const uint32_t kq = lane & 15, grp = wave * 4 + (lane >> 4);
    const int32_t* kb = a.k_cache + ((size_t)kvh * HD + grp * DPG) * a.k_pos_stride + 4 * kq;
    int4 kv[DPG];
    auto load_keys = [&](uint32_t chunk) {
#pragma unroll
        for (uint32_t i = 0; i < DPG; i++) kv[i] = *(const int4*)(kb + (size_t)i * a.k_pos_stride + chunk * 64);
    };
    load_keys(c);
#pragma unroll
    for (uint32_t u = 0; u < QPT; u++)
        if (tid + 256 * u < HD) s_q[tid + 256 * u] = qv[u];
    lds_barrier();
    uint64_t best = 0;  // wave 0: the first maximum of the visible keys so far
    for (;;) {
        uint64_t dot[4] = {0, 0, 0, 0};
#pragma unroll
        for (uint32_t i = 0; i < DPG; i++) {
            const int64_t q = s_q[grp * DPG + i];
            dot[0] += (uint64_t)(q * kv[i].x);
            dot[1] += (uint64_t)(q * kv[i].y);
            dot[2] += (uint64_t)(q * kv[i].z);
            dot[3] += (uint64_t)(q * kv[i].w);
        }
        const uint32_t c0 = c * 64;
        c += chunks;
        const bool more = c * 64 <= pos;
        if (more) load_keys(c);
#pragma unroll
        for (uint32_t off = 16; off < 64; off <<= 1)
#pragma unroll
            for (int k = 0; k < 4; k++) dot[k] += __shfl_xor(dot[k], off);
        if (lane < 16)
#pragma unroll
            for (int k = 0; k < 4; k++) s_part[wave][4 * kq + k] = dot[k];
        lds_barrier();
        if (tid < 64) {
            const uint64_t sum = s_part[0][tid] + s_part[1][tid] + s_part[2][tid] + s_part[3][tid];
            const int32_t sc =
                a.scaled ? dn::scaled_score_from_sum((int64_t)sum, a.scale_q32) : dn::requantize((int64_t)sum);
            a.scores[(size_t)head * a.k_pos_stride + c0 + tid] = sc;  // positions outside the view are never read
            const uint32_t p = c0 + tid;
            const uint64_t k = max_key(sc, p - start);
            best = ((p >= start) & (p <= pos) & (k > best)) ? k : best;
        }
        if (!more) break;
        lds_barrier();  // s_part is read before the next chunk overwrites it
    }
    if (wave == 0) {
        best = wave_max_u64(best);
        if (lane == 0) *max_out = best;
    }
}

constexpr uint32_t VAL_NT = 512, VAL_NW = VAL_NT / 64;
constexpr uint32_t VAL_DS = 32;                // dimensions per values workgroup
constexpr uint32_t VAL_TPR = VAL_DS / 4;       // threads per value row, four dimensions each
constexpr uint32_t VAL_RP = VAL_NT / VAL_TPR;  // value rows one pass of the workgroup reads

struct ValuesSmem {
    int32_t w[ATTN_TILE_KEYS];  // weights
    int64_t part[VAL_NW][VAL_DS];
    uint64_t sum[VAL_NW];
    int32_t wsum[VAL_NW];
};

// The head's first maximum from the scores workgroups' maxima, in every
// wave (no barrier): lane i < chunks holds workgroup i's key.
__device__ __forceinline__ ArgMax head_first_max(uint64_t lane_key) {
    return from_max_key(wave_max_u64(lane_key));
}

// Weighted values in f64, exactly: the weights are non-negative, each at
// most 2^16 + 1, and sum to at most 2^16 plus one half per key (under 2^17
// for ATTN_MAX_KEYS keys), and |v| <= 2^31, so every product and every
// partial sum of any subset of keys is an integer below 2^48 in magnitude:
// each fma is exact and the sum equals the reference's wrapping i64 sum
// (which never wraps). v_fma_f64 issues at full rate where the i64
// multiply-add is a quarter-rate instruction.
__device__ __forceinline__ void weigh_values(double (&acc)[4], int32_t w, int4 v) {
    const double wd = (double)w;
    acc[0] = fma(wd, (double)v.x, acc[0]);
    acc[1] = fma(wd, (double)v.y, acc[1]);
    acc[2] = fma(wd, (double)v.z, acc[2]);
    acc[3] = fma(wd, (double)v.w, acc[3]);
}

// The slice's value at the first maximum (thread t: dimension t % VAL_DS),
// loaded as soon as the maximum is known; unconditional, since a
// conditional load is waited for, with every load before it, where its
// branch joins.
template <uint32_t HD>
__device__ __forceinline__ int32_t first_max_value(const AttnArgs& a, ArgMax m, uint32_t slice, uint32_t kvh,
                                                   uint32_t start) {
    return a.v_cache[(size_t)(start + m.i) * a.kv_stride + (size_t)kvh * HD + slice * VAL_DS + threadIdx.x % VAL_DS];
}

// The end of a values workgroup: acc holds this thread's weighted values of
// dimensions d4..d4+3 over its value rows (exact integers, see
// weigh_values), wpart the wave's sum of weights, vmax the first maximum's
// value (first_max_value). The rows meet across the wave's lanes (lanes
// equal modulo VAL_TPR share dimensions), then across the waves in LDS, in
// wrapping i64; thread d < VAL_DS adds the first maximum's residual weight
// times its value (add_sat(w, ONE - sum) at the first maximum: no
// saturation at these magnitudes, so the change is + (ONE - sum) * v) and
// requantizes.
template <uint32_t HD>
__device__ __forceinline__ void values_finish(const AttnArgs& a, ValuesSmem& sm, const double (&accd)[4],
                                              int32_t wpart, int32_t vmax, uint32_t head, uint32_t slice) {
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint64_t acc[4];
#pragma unroll
    for (int c = 0; c < 4; c++) acc[c] = (uint64_t)(int64_t)accd[c];
#pragma unroll
    for (uint32_t off = VAL_TPR; off < 64; off <<= 1)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[c] += __shfl_xor(acc[c], off);
    if (lane < VAL_TPR)
#pragma unroll
        for (int c = 0; c < 4; c++) sm.part[wave][lane * 4 + c] = (int64_t)acc[c];
    if (lane == 0) sm.wsum[wave] = wpart;
    lds_barrier();
    int32_t out = 0;
    if (tid < VAL_DS) {
        // Weights are non-negative and sum to 2^16 plus at most one half per
        // key: the saturating sum never saturates, a plain sum is the same.
        int32_t wsum = 0;
        uint64_t t = 0;
#pragma unroll
        for (uint32_t i = 0; i < VAL_NW; i++) {
            wsum = dn::add_sat(wsum, sm.wsum[i]);
            t += (uint64_t)sm.part[i][tid];
        }
        const int64_t resid = dn::sub_sat(dn::ONE_ACT, wsum);
        t += (uint64_t)(resid * vmax);
        out = dn::requantize((int64_t)t);
        a.ctx[(size_t)head * HD + slice * VAL_DS + tid] = out;
    }
    // The slice is one 32-value block of the context row: its digit planes
    // for the O product, from wave 0 (threads 0..31 hold the values).
    if (a.ctx_planes && wave == 0)
        act_planes_store32(out, lane, head * HD + slice * VAL_DS, a.heads * HD, a.ctx_planes, a.ctx_counts);
}

// The values workgroup for a view longer than ATTN_TILE_KEYS: the exp sum
// from the stored scores, then tile by tile the weights (exp terms formed
// again) and their weighted values.
template <uint32_t HD>
__device__ void values_long(const AttnArgs& a, ValuesSmem& sm, ArgMax m, uint32_t head, uint32_t slice,
                            uint32_t kvh, uint32_t start, uint32_t n) {
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int32_t vmax = first_max_value<HD>(a, m, slice, kvh, start);
    const int32_t* sb = a.scores + (size_t)head * a.k_pos_stride + start;
    auto exp_term = [&](uint32_t j) -> uint64_t {
        const int64_t diff = (int64_t)m.v - sb[j];
        return diff < (1 << 20) ? dn::softmax_exp_diff((uint32_t)diff) : 0;
    };
    // Terms of at most 2^32 each: no saturation below 2^31 keys.
    uint64_t part = 0;
    for (uint32_t j = tid; j < n; j += VAL_NT) part += exp_term(j);
    part = wave_sum_u64(part);
    if (lane == 0) sm.sum[wave] = part;
    __syncthreads();
    uint64_t total = 0;
    for (uint32_t i = 0; i < VAL_NW; i++) total += sm.sum[i];
    const double w_scale = 65536.0 / (double)total, q_scale = 4294967296.0 / (double)total;
    const uint32_t kr = tid / VAL_TPR, d4 = (tid % VAL_TPR) * 4;
    const int32_t* vb = a.v_cache + (size_t)start * a.kv_stride + (size_t)kvh * HD + slice * VAL_DS + d4;
    int32_t wpart = 0;
    double acc[4] = {0, 0, 0, 0};
    for (uint32_t t0 = 0; t0 < n; t0 += ATTN_TILE_KEYS) {
        const uint32_t tn = min(ATTN_TILE_KEYS, n - t0);
        for (uint32_t j = tid; j < tn; j += VAL_NT) {
            const int32_t w = dn::softmax_weight_fast(exp_term(t0 + j), total, w_scale, q_scale);
            sm.w[j] = w;
            wpart += w;
        }
        __syncthreads();
        for (uint32_t key = kr; key < tn; key += VAL_RP)
            weigh_values(acc, sm.w[key], *(const int4*)(vb + (size_t)(t0 + key) * a.kv_stride));
        __syncthreads();
    }
    wpart = (int32_t)wave_sum_u64((uint64_t)(uint32_t)wpart);
    values_finish<HD>(a, sm, acc, wpart, vmax, head, slice);
}

// Workgroup (head, slice) over `chunks` scores workgroups per head.
template <uint32_t HD>
__global__ __launch_bounds__(512) void attn_values_kernel(const AttnArgs a, uint32_t chunks) {
    constexpr uint32_t NT = VAL_NT, NWV = VAL_NW;
    constexpr uint32_t VR = 1024 / VAL_RP;        // value passes loaded before the softmax (1024 rows)
    constexpr uint32_t EPT = ATTN_TILE_KEYS / NT;  // keys per thread, at most
    __shared__ ValuesSmem sm;
    const uint2 hs = xcd_head_order(a, blockIdx.x, HD / VAL_DS);
    const uint32_t head = hs.x, slice = hs.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t kvh = head / (a.heads / a.kv_heads);
    const uint32_t pos = (uint32_t)(*a.d_pos);
    const uint32_t start = (a.window == 0 || pos + 1 <= a.window) ? 0 : pos + 1 - a.window;
    const uint32_t n = pos - start + 1;

    // 1. The scores workgroups' maxima and this thread's scores (keys
    // tid + NT*u, increasing), issued by every wave before any wave's value
    // loads so that they do not queue behind them; then the slice's value
    // rows. Every load is unconditional (indices past the view clamped to
    // the first key): a conditional load would be waited for where its
    // branch joins.
    uint64_t mk = lane < chunks ? chunk_maxima(a)[(size_t)head * ATTN_DECODE_CHUNKS + lane] : 0;
    if (n > ATTN_TILE_KEYS) {  // uniform over the launch
        values_long<HD>(a, sm, head_first_max(mk), head, slice, kvh, start, n);
        return;
    }
    const int32_t* sb = a.scores + (size_t)head * a.k_pos_stride + start;
    int32_t sc[EPT];
#pragma unroll
    for (uint32_t u = 0; u < EPT; u++) {
        const uint32_t j = tid + NT * u;
        sc[u] = sb[j < n ? j : 0];
    }
    asm volatile("s_barrier" ::: "memory");
    const uint32_t kr = tid / VAL_TPR, d4 = (tid % VAL_TPR) * 4;
    const int32_t* vb = a.v_cache + (size_t)start * a.kv_stride + (size_t)kvh * HD + slice * VAL_DS + d4;
    int4 vv[VR];
#pragma unroll
    for (uint32_t r = 0; r < VR; r++) {
        const uint32_t key = kr + VAL_RP * r;
        vv[r] = *(const int4*)(vb + (size_t)(key < n ? key : 0) * a.kv_stride);
    }
    // Every value load issues before the wait for the maxima: mk passes
    // through an ordered statement after them.
    asm volatile("" : "+v"(mk)::"memory");

    // 2. The first maximum, in every wave; 3. the exp terms (non-negative:
    // their sum is order-free and cannot saturate for ATTN_TILE_KEYS keys)
    // and 4. the weights.
    const ArgMax m = head_first_max(mk);
    const int32_t vmax = first_max_value<HD>(a, m, slice, kvh, start);
    uint64_t ev[EPT];
    uint64_t part = 0;
#pragma unroll
    for (uint32_t u = 0; u < EPT; u++) {
        const uint32_t j = tid + NT * u;
        const int64_t diff = (int64_t)m.v - sc[u];
        ev[u] = 0;
        if ((j < n) & (diff < (1 << 20))) ev[u] = dn::softmax_exp_diff((uint32_t)diff);
        part += ev[u];
    }
    part = wave_sum_u64(part);
    if (lane == 0) sm.sum[wave] = part;
    lds_barrier();
    uint64_t total = 0;
#pragma unroll
    for (uint32_t i = 0; i < NWV; i++) total += sm.sum[i];
    const double w_scale = 65536.0 / (double)total, q_scale = 4294967296.0 / (double)total;
    int32_t wpart = 0;
#pragma unroll
    for (uint32_t u = 0; u < EPT; u++) {
        const uint32_t j = tid + NT * u;
        if (j < n) {
            const int32_t w = dn::softmax_weight_fast(ev[u], total, w_scale, q_scale);
            sm.w[j] = w;
            wpart += w;
        }
    }
    wpart = (int32_t)wave_sum_u64((uint64_t)(uint32_t)wpart);
    lds_barrier();

    // 5. Weighted values of the slice (wrapping i64), VAL_RP rows per pass.
    double acc[4] = {0, 0, 0, 0};
#pragma unroll
    for (uint32_t r = 0; r < VR; r++) {
        const uint32_t key = kr + VAL_RP * r;
        if (key < n) weigh_values(acc, sm.w[key], vv[r]);
    }
    for (uint32_t key = kr + VAL_RP * VR; key < n; key += VAL_RP)
        weigh_values(acc, sm.w[key], *(const int4*)(vb + (size_t)key * a.kv_stride));
    values_finish<HD>(a, sm, acc, wpart, vmax, head, slice);
}

template <uint32_t HD>
int attention_decode_launch(const AttnArgs& a, hipStream_t stream) {
    // Up to ATTN_DECODE_CHUNKS chunk workgroups per head (longer views loop
    // over chunks), rounded up so that the KV heads' chunks fill the XCDs
    // evenly (the extra workgroups find no visible key).
    const uint32_t step = 8 / std::gcd(a.kv_heads, 8u);
    const uint32_t chunks = (min(a.k_pos_stride / 64, ATTN_DECODE_CHUNKS) + step - 1) / step * step;
    static_assert(ATTN_DECODE_CHUNKS % 8 == 0 && ATTN_DECODE_CHUNKS <= 64, "chunk maxima: one wave's lanes");
    static_assert(HD % VAL_DS == 0, "whole slices");
    hipLaunchKernelGGL(attn_scores_kernel<HD>, dim3(a.heads * chunks), dim3(256), 0, stream, a, chunks);
    hipLaunchKernelGGL(attn_values_kernel<HD>, dim3(a.heads * (HD / VAL_DS)), dim3(VAL_NT), 0, stream, a, chunks);
    return (int)hipGetLastError();
}

// Dequantize one Q8_0 row (reference layout) into out[0..cols) (q8.rs:76-92),
// times a Q16.16 scale (model.rs:316-330: gemma-dense's embedding scale, any
// value including zero; mistral-dense passes 1.0, which mul_sat leaves exact).
__device__ __forceinline__ void embed_row(const uint8_t* row, uint32_t cols, int32_t scale, int32_t* out,
                                          uint32_t tid, uint32_t nthreads) {
    for (uint32_t c = tid; c < cols; c += nthreads) {
        const uint8_t* blk = row + (size_t)(c / 32) * 34;
        const int64_t s = dn::scale_q24((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        int32_t v = dn::round_to_i32((dn::i128)((int64_t)(int8_t)blk[2 + c % 32] * s), 8);
        out[c] = dn::mul_sat(v, scale);
    }
}

// Embedding rows of `count` token ids (view_kernels.rs:14-35).
__global__ void embed_rows_kernel(const int32_t* ids, const uint8_t* embed_raw, uint32_t row_bytes,
                                  uint32_t hidden, int32_t scale, int32_t* out) {
    const uint32_t t = blockIdx.x;
    embed_row(embed_raw + (size_t)ids[t] * row_bytes, hidden, scale, out + (size_t)t * hidden, threadIdx.x,
              blockDim.x);
}

__global__ __launch_bounds__(256) void rope_table_kernel(const int64_t* inv_freq, uint32_t half, const int32_t* d_pos,
                                                         uint32_t rows, int64_t* out) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * half) return;
    const uint32_t row = i / half, j = i % half;
    int64_t s, c;
    dn::sin_cos_q30((int64_t)((uint32_t)(*d_pos) + row) * inv_freq[j], s, c);
    out[2 * (size_t)i] = s;
    out[2 * (size_t)i + 1] = c;
}

__global__ __launch_bounds__(256) void silu_kernel(const int32_t* x, uint32_t n, int32_t* out) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = dn::silu(x[i]);
}

__global__ __launch_bounds__(256) void silu_table_kernel(int32_t* tab) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < dn::SILU_TAB_N) tab[i] = dn::silu((int32_t)i - (dn::SILU_TAB_HALF - 1));
}

__global__ __launch_bounds__(256) void silu_lookup_kernel(const int32_t* tab, const int32_t* x, uint32_t n,
                                                          int32_t* out) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = dn::silu_from_tab(x[i], tab[dn::silu_tab_index(x[i])]);
}

// The pass position and the selection step of a session, set on its stream.
__global__ void set_counters_kernel(int32_t* d_pos, int32_t pos, int32_t* d_step, int32_t step) {
    if (threadIdx.x == 0) {
        *d_pos = pos;
        *d_step = step;
    }
}

}  // namespace

int iris_set_counters_launch(int32_t* d_pos, int32_t pos, int32_t* d_step, int32_t step, hipStream_t stream) {
    hipLaunchKernelGGL(set_counters_kernel, dim3(1), dim3(64), 0, stream, d_pos, pos, d_step, step);
    return (int)hipGetLastError();
}

extern "C" int iris_silu_device(const int32_t* d_x, uint32_t n, int32_t* d_out) {
    if (n == 0) return 0;
    if (!d_x || !d_out) return IRIS_E_INVALID;
    hipLaunchKernelGGL(silu_kernel, dim3((n + 255) / 256), dim3(256), 0, nullptr, d_x, n, d_out);
    hipError_t st = hipGetLastError();
    if (st == hipSuccess) st = hipDeviceSynchronize();
    return (int)st;
}

int iris_silu_table(const int32_t** out) {
    // One table per device, made on first use and kept until the process ends.
    static std::mutex mu;
    static std::map<int, int32_t*> tables;
    *out = nullptr;
    int dev = 0;
    hipError_t st = hipGetDevice(&dev);
    if (st != hipSuccess) return (int)st;
    std::lock_guard<std::mutex> lock(mu);
    auto it = tables.find(dev);
    if (it != tables.end()) {
        *out = it->second;
        return 0;
    }
    int32_t* tab = nullptr;
    st = hipMalloc((void**)&tab, (size_t)dn::SILU_TAB_N * 4);
    if (st != hipSuccess) return IRIS_E_NOMEM;
    hipLaunchKernelGGL(silu_table_kernel, dim3((dn::SILU_TAB_N + 255) / 256), dim3(256), 0, nullptr, tab);
    st = hipGetLastError();
    if (st == hipSuccess) st = hipDeviceSynchronize();
    if (st != hipSuccess) {
        hipFree(tab);
        return (int)st;
    }
    tables[dev] = tab;
    *out = tab;
    return 0;
}

extern "C" int iris_silu_table_device(const int32_t* d_x, uint32_t n, int32_t* d_out) {
    if (n == 0) return 0;
    if (!d_x || !d_out) return IRIS_E_INVALID;
    const int32_t* tab = nullptr;
    int rc = iris_silu_table(&tab);
    if (rc) return rc;
    hipLaunchKernelGGL(silu_lookup_kernel, dim3((n + 255) / 256), dim3(256), 0, nullptr, tab, d_x, n, d_out);
    hipError_t st = hipGetLastError();
    if (st == hipSuccess) st = hipDeviceSynchronize();
    return (int)st;
}

int iris_rope_table_launch(const int64_t* inv_freq, uint32_t half, const int32_t* d_pos, uint32_t rows, int64_t* out,
                           hipStream_t stream) {
    if (rows == 0 || half == 0) return 0;
    hipLaunchKernelGGL(rope_table_kernel, dim3((rows * half + 255) / 256), dim3(256), 0, stream, inv_freq, half, d_pos,
                       rows, out);
    return (int)hipGetLastError();
}

bool iris_attention_decode_applies(const AttnArgs& a, uint32_t tokens, uint32_t max_keys) {
    const uint32_t hd = a.head_dim;
    return tokens == 1 && a.scores && a.k_pos_stride % 64 == 0 && max_keys <= a.k_pos_stride &&
           (hd == 32 || hd == 64 || hd == 128 || hd == 256 || hd == 512);
}

int iris_attention_launch(const AttnArgs& a, uint32_t tokens, uint32_t max_keys, hipStream_t stream) {
    if (a.head_dim > ATTN_MAX_HEAD_DIM || a.head_dim % 4 || max_keys > ATTN_MAX_KEYS || a.heads % a.kv_heads)
        return IRIS_E_INVALID;
    if ((a.ctx_planes || a.ctx_counts) && !(iris_attention_decode_applies(a, tokens, max_keys) && a.ctx_planes &&
                                            a.ctx_counts))
        return IRIS_E_INVALID;
    if (iris_attention_decode_applies(a, tokens, max_keys)) {
        // One row: the chunked scores, then HD/32 workgroups per head.
        switch (a.head_dim) {
            case 32: return attention_decode_launch<32>(a, stream);
            case 64: return attention_decode_launch<64>(a, stream);
            case 128: return attention_decode_launch<128>(a, stream);
            case 256: return attention_decode_launch<256>(a, stream);
            case 512: return attention_decode_launch<512>(a, stream);
            default: break;  // other head sizes: the one-workgroup-per-head kernel
        }
    }
    if (tokens >= 2 && iris_attention_prefill_applies(a, tokens, max_keys))
        return iris_attention_prefill_launch(a, tokens, max_keys, stream);
    // attend_row takes a multiple of 256 threads, at least one per head dimension.
    const uint32_t threads = tokens == 1 ? 1024 : std::max(256u, (a.head_dim + 255) / 256 * 256);
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
