// Exact multi-row attention on gfx950's int8 matrix cores.
//
// The reference attends one query row at a time (mistral/layer.rs:274-318,
// prefill_range.rs:755-845): wrapping-i64 scores q.k, the det-num softmax
// (ops.rs:233-261) and wrapping-i64 weighted values, each requantized. Both
// sums are exact integers modulo 2^64, so they may be formed in any order.
// Here queries, keys and values are split into signed byte digits
// (v = sum_l 256^l d_l, d_l in [-128, 127]) and every pair of digit planes
// is an int8 MFMA with exact int32 accumulation; the planes are recombined
// modulo 2^64 (planes whose digit sums share l1 + l2 share an accumulator:
// |sum| <= 4 * 128 * 2^14 < 2^31 for scores, 2 * 4096 * 2^14 for values).
//
// The softmax needs each row's first maximum before any exp term and the
// full sum before any weight, so each workgroup walks its keys three times:
// (1) scores and the first maximum, the scores kept in an HBM store; (2) the
// exp terms of the stored scores and their sum, the terms overwriting the
// scores; (3) the weights from the stored terms and the weighted values. The
// weights never leave registers: the score tile's lane layout is, up to a
// fixed permutation of the keys inside each 64-key step, the A operand of
// the value product, and the value planes are written in that permuted key
// order. A weight w <= 2^16 is two digits unless w >= 32640; those (at most
// two per row: the weights sum to 2^16 plus rounding) are carried as
// w - 65536 plus 65536 * v added at the end, with the residual of the first
// maximum (ops.rs:258-260).
//
// Workgroup: one 16-row query tile of four consecutive query heads (any
// number of them per KV head), one wave per head. A tile whose queries or keys need five digits (|v|
// near i32::MAX), or whose values need four (|v| >= 2^23), takes the scalar
// one-row routine instead.
#include <type_traits>

#include "attn_common.h"
#include "detnum_dev.h"
#include "layer_kernels.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int AP_PLANES = 4;             // digit planes kept per value
constexpr int AP_V_PLANES = 3;           // value digits the matrix-core path takes (more: scalar path)
constexpr int32_t BIG_WEIGHT = 32640;    // first weight that needs a third digit
constexpr uint32_t FRAG = 1024;          // one 16 x 64 MFMA operand

__device__ __forceinline__ uint64_t digits5(int32_t v) {
    return (uint64_t)((int64_t)v + 0x8080808080LL) ^ 0x8080808080ULL;
}

__device__ __forceinline__ int limbs_needed(uint64_t d) {
    return (d >> 32) ? 5 : (d >> 24) ? 4 : (d >> 16) ? 3 : (d >> 8) ? 2 : 1;
}

// Byte l of the digits of four values, as one dword.
__device__ __forceinline__ uint32_t digit_dword(const uint64_t (&d)[4], int l) {
    const int sh = 8 * l;
    return (uint32_t)((d[0] >> sh) & 0xff) | ((uint32_t)((d[1] >> sh) & 0xff) << 8) |
           ((uint32_t)((d[2] >> sh) & 0xff) << 16) | ((uint32_t)((d[3] >> sh) & 0xff) << 24);
}

__device__ __forceinline__ int wave_max_int(int v) {
    for (int off = 32; off >= 1; off >>= 1) v = max(v, __shfl_xor(v, off));
    return v;
}

// Query planes: one wave per (16-row tile, head). Lane l takes row l % 16
// and dims 16 * (l / 16) .. + 16 of each 64-dim step.
template <uint32_t HD>
__global__ __launch_bounds__(64) void attn_q_planes_kernel(const AttnArgs a, uint32_t tokens) {
    constexpr uint32_t DS = HD / 64;
    const AttnPlanes& p = a.planes;
    const uint32_t qt = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const uint32_t t = qt * 16 + (lane & 15), dq = (lane >> 4) * 16;
    const bool valid = t < tokens;
    const int32_t* q = a.q + (size_t)(valid ? t : 0) * a.q_stride + (size_t)h * HD;
    const size_t lstride = (size_t)a.heads * p.qt_cap * DS * FRAG;
    int need = 1;
#pragma unroll
    for (uint32_t ds = 0; ds < DS; ds++) {
        uint32_t out[AP_PLANES][4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            int4 v = make_int4(0, 0, 0, 0);
            if (valid) v = *(const int4*)(q + ds * 64 + dq + 4 * c);
            const uint64_t d[4] = {digits5(v.x), digits5(v.y), digits5(v.z), digits5(v.w)};
            need = max(need, max(max(limbs_needed(d[0]), limbs_needed(d[1])), max(limbs_needed(d[2]), limbs_needed(d[3]))));
#pragma unroll
            for (int l = 0; l < AP_PLANES; l++) out[l][c] = digit_dword(d, l);
        }
        int8_t* dst = p.q + (((size_t)h * p.qt_cap + qt) * DS + ds) * FRAG + lane * 16;
#pragma unroll
        for (int l = 0; l < AP_PLANES; l++)
            *(uint4*)(dst + l * lstride) = make_uint4(out[l][0], out[l][1], out[l][2], out[l][3]);
    }
    need = wave_max_int(need);
    if (lane == 0) p.q_limbs[h * p.qt_cap + qt] = (uint8_t)need;
}

// Key and value planes of one 64-key step of one KV head (keys past the
// last position are zero). Wave w writes key tile w: lane l takes key
// l % 16 and dims 16 * (l / 16) .. of each 64-dim step. Value d-tiles
// w, w + 4, ...: lane l takes dim l % 16 and, as byte 4t + i, the key
// 16t + 4(l / 16) + i of the step.
template <uint32_t HD>
__global__ __launch_bounds__(256) void attn_kv_planes_kernel(const AttnArgs a, uint32_t tokens) {
    constexpr uint32_t DS = HD / 64, DT = HD / 16;
    __shared__ int s_need[2];
    const AttnPlanes& p = a.planes;
    const uint32_t ks = blockIdx.x, g = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t nkeys = (uint32_t)(*a.d_pos) + tokens;
    if (ks * 64 >= nkeys) return;
    if (tid < 2) s_need[tid] = 1;
    __syncthreads();

    const uint32_t key = ks * 64 + wave * 16 + (lane & 15), dq = (lane >> 4) * 16;
    const bool kvalid = key < nkeys;
    const size_t kl = (size_t)a.kv_heads * p.ks_cap * 4 * DS * FRAG;
    int kneed = 1;
#pragma unroll
    for (uint32_t ds = 0; ds < DS; ds++) {
        uint32_t out[AP_PLANES][4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            int32_t v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t dim = ds * 64 + dq + 4 * c + j;
                v[j] = kvalid ? a.k_cache[((size_t)g * HD + dim) * a.k_pos_stride + key] : 0;
            }
            const uint64_t d[4] = {digits5(v[0]), digits5(v[1]), digits5(v[2]), digits5(v[3])};
            kneed = max(kneed, max(max(limbs_needed(d[0]), limbs_needed(d[1])), max(limbs_needed(d[2]), limbs_needed(d[3]))));
#pragma unroll
            for (int l = 0; l < AP_PLANES; l++) out[l][c] = digit_dword(d, l);
        }
        int8_t* dst = p.k + (((size_t)g * p.ks_cap * 4 + ks * 4 + wave) * DS + ds) * FRAG + lane * 16;
#pragma unroll
        for (int l = 0; l < AP_PLANES; l++)
            *(uint4*)(dst + l * kl) = make_uint4(out[l][0], out[l][1], out[l][2], out[l][3]);
    }

    const size_t vl = (size_t)a.kv_heads * p.ks_cap * DT * FRAG;
    const uint32_t gk = lane >> 4;
    int vneed = 1;
    for (uint32_t dt = wave; dt < DT; dt += 4) {
        const uint32_t dim = dt * 16 + (lane & 15);
        uint32_t out[AP_PLANES][4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            int32_t v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t k = ks * 64 + 16 * t + 4 * gk + i;
                v[i] = k < nkeys ? a.v_cache[(size_t)k * a.kv_stride + (size_t)g * HD + dim] : 0;
            }
            const uint64_t d[4] = {digits5(v[0]), digits5(v[1]), digits5(v[2]), digits5(v[3])};
            vneed = max(vneed, max(max(limbs_needed(d[0]), limbs_needed(d[1])), max(limbs_needed(d[2]), limbs_needed(d[3]))));
#pragma unroll
            for (int l = 0; l < AP_PLANES; l++) out[l][t] = digit_dword(d, l);
        }
        int8_t* dst = p.v + (((size_t)g * p.ks_cap + ks) * DT + dt) * FRAG + lane * 16;
#pragma unroll
        for (int l = 0; l < AP_PLANES; l++)
            *(uint4*)(dst + l * vl) = make_uint4(out[l][0], out[l][1], out[l][2], out[l][3]);
    }
    kneed = wave_max_int(kneed);
    vneed = wave_max_int(vneed);
    if (lane == 0) {
        atomicMax(&s_need[0], kneed);
        atomicMax(&s_need[1], vneed);
    }
    __syncthreads();
    if (tid < 2) p.kv_limbs[((size_t)g * p.ks_cap + ks) * 2 + tid] = (uint8_t)s_need[tid];
}

struct PrefillSmem {
    int32_t info[4][16][2];   // per wave and query row: first-maximum key, residual
    int32_t big[4][16][8];    // per wave and query row: large-weight keys (two per lane group, -1 none)
};

template <uint32_t HD, int LQK>
__device__ __forceinline__ void load_key_tile(const int8_t* kb, size_t kl, v4i (&kf)[LQK][HD / 64]) {
#pragma unroll
    for (int l = 0; l < LQK; l++)
#pragma unroll
        for (uint32_t ds = 0; ds < HD / 64; ds++) kf[l][ds] = *(const v4i*)(kb + l * kl + ds * FRAG);
}

// The scores of one 16-key tile against the wave's 16 query rows, from LQK
// digit planes of each: lane l holds query l % 16 and keys 4 * (l / 16) + i
// of the tile.
template <uint32_t HD, int LQK>
__device__ __forceinline__ void tile_scores(const AttnArgs& a, const v4i (&kf)[LQK][HD / 64],
                                            const v4i (&qf)[LQK][HD / 64], int32_t (&sc)[4]) {
    constexpr int NS = 2 * LQK - 1;
    v4i acc[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) acc[s] = v4i{0, 0, 0, 0};
#pragma unroll
    for (uint32_t ds = 0; ds < HD / 64; ds++)
#pragma unroll
        for (int l = 0; l < LQK; l++)
#pragma unroll
            for (int b = 0; b < LQK; b++)
                acc[l + b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf[l][ds], qf[b][ds], acc[l + b], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint64_t s = 0;  // the wrapping i64 dot product
#pragma unroll
        for (int j = 0; j < NS; j++) s += (uint64_t)(int64_t)acc[j][i] << (8 * j);
        sc[i] = a.scaled ? dn::scaled_score_from_sum((int64_t)s, a.scale_q32) : dn::requantize((int64_t)s);
    }
}

// One wave: 16 query rows of one head over key steps [ks0, ks1), queries
// and keys of LQK digits, values of AP_V_PLANES.
template <uint32_t HD, int LQK>
__device__ __forceinline__ void prefill_wave(const AttnArgs& a, uint32_t tokens, PrefillSmem& sm, uint32_t g,
                                             uint32_t head, uint32_t qt, uint32_t ks0, uint32_t ks1) {
    constexpr uint32_t DS = HD / 64, DT = HD / 16;
    const AttnPlanes& p = a.planes;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t pos0 = (uint32_t)(*a.d_pos);

    // This lane's query row for the scores, and its visible keys.
    const uint32_t qrow = qt * 16 + (lane & 15), grp = lane >> 4;
    const bool qvalid = qrow < tokens;
    const uint32_t qpos = pos0 + qrow;
    const uint32_t qstart = (a.window == 0 || qpos + 1 <= a.window) ? 0 : qpos + 1 - a.window;
    const uint32_t span = qpos - qstart;  // qstart <= key <= qpos, as one unsigned comparison
    auto visible = [&](uint32_t key) { return qvalid & (key - qstart <= span); };
    v4i qf[LQK][DS];
    {
        const int8_t* qb = p.q + ((size_t)head * p.qt_cap + qt) * DS * FRAG + lane * 16;
        const size_t ql = (size_t)a.heads * p.qt_cap * DS * FRAG;
#pragma unroll
        for (int b = 0; b < LQK; b++)
#pragma unroll
            for (uint32_t ds = 0; ds < DS; ds++) qf[b][ds] = *(const v4i*)(qb + b * ql + ds * FRAG);
    }
    const size_t kl = (size_t)a.kv_heads * p.ks_cap * 4 * DS * FRAG;
    const int8_t* kbase = p.k + (size_t)g * p.ks_cap * 4 * DS * FRAG + lane * 16;
    const uint32_t kt0 = ks0 * 4, kt1 = ks1 * 4;  // 16-key tiles
    // The next key tile is loaded during the current one's scores where the
    // registers allow (head sizes up to 128).
    constexpr bool KEY_PREFETCH = HD <= 128;
    v4i kf[LQK][DS], kn[KEY_PREFETCH ? LQK : 1][KEY_PREFETCH ? DS : 1];

    // (1) the scores, kept in the exp store (one 16-byte slot per lane and
    // tile), and the first maximum: keys run in increasing order in each lane.
    uint32_t* estore = p.e_store + ((size_t)head * p.qt_cap + qt) * p.ks_cap * 4 * 256 + lane * 4;
    int32_t best = INT32_MIN;
    uint32_t best_key = 0xffffffffu;
    if constexpr (KEY_PREFETCH) {
        load_key_tile<HD, LQK>(kbase + (size_t)kt0 * DS * FRAG, kl, kf);
        // Waited for here, where the compiler sees it (s_waitcnt vmcnt(0)):
        // a load into kf still pending at the loop's entry made its wait
        // insertion, which merges the loop's entry with its back edge,
        // wait for every load before each tile's products, the next tile's
        // prefetch included. With none pending, each tile waits for its
        // prefetch only where kn is copied into kf, after its products.
        __builtin_amdgcn_s_waitcnt(0x0f70);
    }
#pragma unroll 1
    for (uint32_t kt = kt0; kt < kt1; kt++) {
        if constexpr (KEY_PREFETCH) {
            if (kt + 1 < kt1) load_key_tile<HD, LQK>(kbase + (size_t)(kt + 1) * DS * FRAG, kl, kn);
        } else {
            load_key_tile<HD, LQK>(kbase + (size_t)kt * DS * FRAG, kl, kf);
        }
        int32_t sc[4];
        tile_scores<HD, LQK>(a, kf, qf, sc);
        *(uint4*)(estore + (size_t)kt * 256) = make_uint4((uint32_t)sc[0], (uint32_t)sc[1], (uint32_t)sc[2], (uint32_t)sc[3]);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t key = kt * 16 + 4 * grp + i;
            const bool take = visible(key) & (sc[i] > best);
            best = take ? sc[i] : best;
            best_key = take ? key : best_key;
        }
        if constexpr (KEY_PREFETCH) {
#pragma unroll
            for (int l = 0; l < LQK; l++)
#pragma unroll
                for (uint32_t ds = 0; ds < DS; ds++) kf[l][ds] = kn[l][ds];
        }
    }
#pragma unroll
    for (int off = 16; off <= 32; off <<= 1) {
        const int32_t ov = __shfl_xor(best, off);
        const uint32_t ok = (uint32_t)__shfl_xor((int)best_key, off);
        if (ov > best || (ov == best && ok < best_key)) {
            best = ov;
            best_key = ok;
        }
    }

    // (2) the sum of exp terms (non-negative, so no order and no saturation)
    // from the stored scores; each lane overwrites a tile's scores with its
    // terms for (3) (2^32, the maximum's term, as 0xffffffff: every other
    // term is below 2^32 - 2^15).
    uint64_t sum = 0;
    uint4 sn = *(const uint4*)(estore + (size_t)kt0 * 256);
    // Waited for here, visibly (as the first key tile above): otherwise
    // each tile's wait for its prefetched scores also covered the previous
    // tile's store of its terms.
    __builtin_amdgcn_s_waitcnt(0x0f70);
#pragma unroll 1
    for (uint32_t kt = kt0; kt < kt1; kt++) {
        const uint4 scv = sn;
        if (kt + 1 < kt1) sn = *(const uint4*)(estore + (size_t)(kt + 1) * 256);
        const int32_t sc[4] = {(int32_t)scv.x, (int32_t)scv.y, (int32_t)scv.z, (int32_t)scv.w};
        uint32_t ev[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t key = kt * 16 + 4 * grp + i;
            const int64_t diff = (int64_t)best - sc[i];
            uint64_t e = 0;
            if (visible(key) & (diff < (1 << 20))) e = dn::softmax_exp_diff((uint32_t)diff);
            sum += e;
            ev[i] = e > 0xffffffffull ? 0xffffffffu : (uint32_t)e;
        }
        *(uint4*)(estore + (size_t)kt * 256) = make_uint4(ev[0], ev[1], ev[2], ev[3]);
    }
    sum += __shfl_xor(sum, 16);
    sum += __shfl_xor(sum, 32);
    const double q_scale = qvalid ? 4294967296.0 / (double)sum : 0.0;
    const double w_scale = qvalid ? 65536.0 / (double)sum : 0.0;

    // (3) weights from the stored terms (zero for keys out of view), their
    // sum, and the weighted values, for value d-tiles [D0, D0 + DN): head
    // size 256 takes several such passes (the weights formed again from the
    // stored terms), so that the value sums fit the registers.
    auto values_pass = [&](auto d0c, auto dnc) __attribute__((always_inline)) {
        constexpr uint32_t D0 = decltype(d0c)::value, DN = decltype(dnc)::value;
        v4i pacc[DN][AP_V_PLANES + 1];
#pragma unroll
        for (uint32_t dt = 0; dt < DN; dt++)
#pragma unroll
            for (int s = 0; s < AP_V_PLANES + 1; s++) pacc[dt][s] = v4i{0, 0, 0, 0};
        const size_t vl = (size_t)a.kv_heads * p.ks_cap * DT * FRAG;
        const int8_t* vbase = p.v + (size_t)g * p.ks_cap * DT * FRAG + lane * 16;
        int32_t wsum = 0;
        int32_t big[2] = {-1, -1};
        uint4 en = *(const uint4*)(estore + (size_t)kt0 * 256);
#pragma unroll 1
        for (uint32_t ks = ks0; ks < ks1; ks++) {
            // The step's value operands, needed after its four weight tiles.
            const int8_t* vb = vbase + (size_t)ks * DT * FRAG;
            // The two weight digits of this lane's 16 keys: byte 4t + i of
            // wf0/wf1 (tile t is shifted in as the last component).
            v4i wf0 = v4i{0, 0, 0, 0}, wf1 = v4i{0, 0, 0, 0};
#pragma unroll
            for (uint32_t t = 0; t < 4; t++) {
                const uint32_t kt = ks * 4 + t;
                const uint4 ec = en;
                if (kt + 1 < kt1) en = *(const uint4*)(estore + (size_t)(kt + 1) * 256);
                const uint32_t ev[4] = {ec.x, ec.y, ec.z, ec.w};
                // Weights by the double estimate of softmax_weight_fast; a key
                // whose estimate lies near a rounding tie, or whose weight
                // needs the large-weight carry, is flagged and redone below
                // (rare: the lanes skip that code together when none is
                // flagged).
                int32_t w[4];
                uint32_t slow = 0;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const double ed = ev[i] == 0xffffffffu ? 4294967296.0 : (double)ev[i];
                    const double tt = ed * w_scale + 0.5;
                    const double fl = floor(tt);
                    w[i] = (int32_t)fl;
                    slow |= (uint32_t)((fabs(tt - fl - 0.5) > 0.5 - 0x1p-15) | (w[i] >= BIG_WEIGHT)) << i;
                }
                if (slow) {
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        if (!((slow >> i) & 1)) continue;
                        const uint64_t e = ev[i] == 0xffffffffu ? (uint64_t)dn::ONE_ACC : ev[i];
                        w[i] = dn::softmax_weight_fast(e, sum, w_scale, q_scale);
                        if (w[i] >= BIG_WEIGHT) {
                            const int32_t key = (int32_t)(kt * 16 + 4 * grp + i);
                            if (big[0] < 0) big[0] = key;
                            else big[1] = key;
                            w[i] -= 65536;
                            wsum += 65536;
                        }
                    }
                }
                wsum += w[0] + w[1] + w[2] + w[3];
                // Two signed digits per weight: (w + 0x8080) ^ 0x8080 holds
                // digit 0 in byte 0 and digit 1 in byte 1; byte i of b0 (b1)
                // is digit 0 (1) of key i.
                uint32_t d[4];
#pragma unroll
                for (int i = 0; i < 4; i++) d[i] = (uint32_t)(w[i] + 0x8080) ^ 0x8080u;
                const uint32_t lo = __builtin_amdgcn_perm(d[1], d[0], 0x05010400u);
                const uint32_t hi = __builtin_amdgcn_perm(d[3], d[2], 0x05010400u);
                const uint32_t b0 = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
                const uint32_t b1 = __builtin_amdgcn_perm(hi, lo, 0x07060302u);
                wf0 = v4i{wf0[1], wf0[2], wf0[3], (int)b0};
                wf1 = v4i{wf1[1], wf1[2], wf1[3], (int)b1};
            }
#pragma unroll
            for (uint32_t dt = 0; dt < DN; dt++) {
                v4i vf[AP_V_PLANES];
#pragma unroll
                for (int b = 0; b < AP_V_PLANES; b++) vf[b] = *(const v4i*)(vb + b * vl + (D0 + dt) * FRAG);
#pragma unroll
                for (int b = 0; b < AP_V_PLANES; b++) {
                    pacc[dt][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf0, vf[b], pacc[dt][b], 0, 0, 0);
                    pacc[dt][b + 1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf1, vf[b], pacc[dt][b + 1], 0, 0, 0);
                }
            }
        }
        wsum += __shfl_xor(wsum, 16);
        wsum += __shfl_xor(wsum, 32);

        // Per query row: the residual goes to the first maximum; every large
        // weight adds 65536 * v back. (Each wave reads only its own rows'
        // entries; a second pass rewrites them with the same values.)
        if (lane < 16) {
            sm.info[wave][lane][0] = (int32_t)best_key;
            sm.info[wave][lane][1] = dn::sub_sat(dn::ONE_ACT, wsum);
        }
        sm.big[wave][lane & 15][2 * grp] = big[0];
        sm.big[wave][lane & 15][2 * grp + 1] = big[1];
        __syncthreads();

        // Lane l of the value product holds dim l % 16 of each d-tile for
        // query rows 4 * (l / 16) + i.
        const int32_t* vcache = a.v_cache + (size_t)g * HD;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t qq = 4 * grp + i, row = qt * 16 + qq;
            if (row >= tokens) continue;
            const uint32_t mkey = (uint32_t)sm.info[wave][qq][0];
            const int64_t resid = sm.info[wave][qq][1];
#pragma unroll
            for (uint32_t dt = 0; dt < DN; dt++) {
                const uint32_t dim = (D0 + dt) * 16 + (lane & 15);
                uint64_t tot = 0;
#pragma unroll
                for (int s = 0; s < AP_V_PLANES + 1; s++) tot += (uint64_t)(int64_t)pacc[dt][s][i] << (8 * s);
                tot += (uint64_t)(resid * vcache[(size_t)mkey * a.kv_stride + dim]);
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const int32_t bk = sm.big[wave][qq][j];
                    if (bk >= 0) tot += (uint64_t)((int64_t)65536 * vcache[(size_t)bk * a.kv_stride + dim]);
                }
                a.ctx[(size_t)row * a.ctx_stride + (size_t)head * HD + dim] = dn::requantize((int64_t)tot);
            }
        }
    };
    // Head size 256: four passes of four d-tiles (two of eight spill);
    // 512 (one wave per SIMD): four passes of eight.
    constexpr uint32_t VPASS = HD >= 512 ? 8 : HD >= 256 ? 4 : DT;
    auto passes = [&](auto self, auto pc) __attribute__((always_inline)) {
        constexpr uint32_t P = decltype(pc)::value;
        values_pass(std::integral_constant<uint32_t, P * VPASS>{}, std::integral_constant<uint32_t, VPASS>{});
        if constexpr (P + 1 < DT / VPASS) self(self, std::integral_constant<uint32_t, P + 1>{});
    };
    passes(passes, std::integral_constant<uint32_t, 0>{});
}

// Workgroup: query heads h0..h0+3 (four consecutive heads, one wave each,
// each with its own KV head) over one 16-row query tile, the longest rows
// first. Two waves per SIMD up to head size 256; one at 512, whose query and
// key-tile fragments (LQK x 8 each) take 256 registers together.
template <uint32_t HD>
__global__ __launch_bounds__(256, HD >= 512 ? 1 : 2) void attn_prefill_kernel(const AttnArgs a, uint32_t tokens) {
    __shared__ union {
        AttnRowSmem row;
        PrefillSmem pre;
    } sm;
    __shared__ int s_limbs;
    const AttnPlanes& p = a.planes;
    const uint32_t tid = threadIdx.x, wave = tid >> 6;
    const uint32_t group = a.heads / a.kv_heads, per_qt = a.heads / 4;
    const uint32_t QT = (tokens + 15) / 16;
    const uint32_t qt = QT - 1 - blockIdx.x / per_qt;
    const uint32_t h0 = (blockIdx.x % per_qt) * 4;
    const uint32_t pos0 = (uint32_t)(*a.d_pos);
    const uint32_t rows = min(16u, tokens - qt * 16);
    const uint32_t first_pos = pos0 + qt * 16, last_pos = first_pos + rows - 1;
    const uint32_t first_key = (a.window == 0 || first_pos + 1 <= a.window) ? 0 : first_pos + 1 - a.window;
    const uint32_t ks0 = first_key / 64, ks1 = last_pos / 64 + 1;
    const uint32_t g_first = h0 / group, g_last = (h0 + 3) / group;

    // Digits the block's queries and keys need (values: at most three);
    // 5 or more sends the block to the one-row routine.
    if (tid == 0) s_limbs = 1;
    __syncthreads();
    if (tid < 4) atomicMax(&s_limbs, (int)p.q_limbs[(h0 + tid) * p.qt_cap + qt]);
    for (uint32_t g = g_first; g <= g_last; g++) {
        const uint8_t* kvl = p.kv_limbs + (size_t)g * p.ks_cap * 2;
        for (uint32_t ks = ks0 + tid; ks < ks1; ks += 256)
            atomicMax(&s_limbs, kvl[2 * ks + 1] > AP_V_PLANES ? AP_PLANES + 1 : (int)kvl[2 * ks]);
    }
    __syncthreads();
    const int limbs = s_limbs;
    if (limbs > AP_PLANES) {
        for (uint32_t i = 0; i < 4 * rows; i++) attend_row(a, h0 + i / rows, qt * 16 + i % rows, sm.row);
    } else if (limbs <= 3) {
        prefill_wave<HD, 3>(a, tokens, sm.pre, (h0 + wave) / group, h0 + wave, qt, ks0, ks1);
    } else {
        prefill_wave<HD, 4>(a, tokens, sm.pre, (h0 + wave) / group, h0 + wave, qt, ks0, ks1);
    }
}

template <uint32_t HD>
int prefill_launch(const AttnArgs& a, uint32_t tokens, hipStream_t stream) {
    const uint32_t QT = (tokens + 15) / 16;
    hipLaunchKernelGGL(attn_q_planes_kernel<HD>, dim3(QT, a.heads), dim3(64), 0, stream, a, tokens);
    hipLaunchKernelGGL(attn_kv_planes_kernel<HD>, dim3(a.planes.ks_cap, a.kv_heads), dim3(256), 0, stream, a, tokens);
    const uint32_t wgs = QT * (a.heads / 4);
    hipLaunchKernelGGL(attn_prefill_kernel<HD>, dim3(wgs), dim3(256), 0, stream, a, tokens);
    return (int)hipGetLastError();
}

__global__ void attention_numerics_kernel(const uint32_t* diff, const uint64_t* e, const uint64_t* sum,
                                          const int64_t* dot, uint32_t scale_q32, uint32_t n, uint64_t* e_out,
                                          int32_t* w_out, int32_t* score_out) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    e_out[i] = dn::softmax_exp_diff(diff[i]);
    w_out[i] = dn::softmax_weight_fast(e[i], sum[i], 65536.0 / (double)sum[i], 4294967296.0 / (double)sum[i]);
    score_out[i] = dn::scaled_score_from_sum(dot[i], scale_q32);
}

}  // namespace

int iris_attention_numerics(const uint32_t* d_diff, const uint64_t* d_e, const uint64_t* d_sum, const int64_t* d_dot,
                            uint32_t scale_q32, uint32_t n, uint64_t* d_exp, int32_t* d_weight, int32_t* d_score) {
    if (n == 0) return 0;
    if (!d_diff || !d_e || !d_sum || !d_dot || !d_exp || !d_weight || !d_score) return IRIS_E_INVALID;
    hipLaunchKernelGGL(attention_numerics_kernel, dim3((n + 255) / 256), dim3(256), 0, nullptr, d_diff, d_e, d_sum,
                       d_dot, scale_q32, n, d_exp, d_weight, d_score);
    hipError_t st = hipGetLastError();
    if (st == hipSuccess) st = hipDeviceSynchronize();
    return (int)st;
}

bool iris_attention_prefill_applies(const AttnArgs& a, uint32_t tokens, uint32_t max_keys) {
    const AttnPlanes& p = a.planes;
    // Head size 256 (four value passes) pays off from about 128 workgroups
    // (Gemma-2B shape: 93 against 117 ms for a 2048-row pass, 15.2 against
    // 12.8 ms for 128 rows on the one-row routine), and so does 512 (one
    // wave per SIMD; the scaled gemma-4 shape: 12.5 against 16.7 ms for 2048
    // rows, 5.2 against 4.9 ms for 600).
    if (a.head_dim >= 256 && (tokens + 15) / 16 * (a.heads / 4) < 128) return false;
    return tokens >= 2 && p.q && p.k && p.v && p.q_limbs && p.kv_limbs && p.e_store &&
           (a.head_dim == 64 || a.head_dim == 128 || a.head_dim == 256 || a.head_dim == 512) &&
           a.heads % a.kv_heads == 0 && a.heads % 4 == 0 && (tokens + 15) / 16 <= p.qt_cap &&
           max_keys <= p.ks_cap * 64 && max_keys <= ATTN_MAX_KEYS;
}

int iris_attention_prefill_launch(const AttnArgs& a, uint32_t tokens, uint32_t max_keys, hipStream_t stream) {
    if (!iris_attention_prefill_applies(a, tokens, max_keys)) return IRIS_E_INVALID;
    switch (a.head_dim) {
        case 64: return prefill_launch<64>(a, tokens, stream);
        case 128: return prefill_launch<128>(a, tokens, stream);
        case 256: return prefill_launch<256>(a, tokens, stream);
        default: return prefill_launch<512>(a, tokens, stream);
    }
}
