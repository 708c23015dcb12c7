// Exact Q8_0 products on gfx950: the tile packing of an uploaded matrix and
// the bandwidth-bound product kernel (decode GEMV; also any token count).
//
// Every output is det_num::q8::dot_row (crates/det-num/src/q8.rs:56-72):
// exact block sums, each times the block's Q.24 scale, summed without
// overflow, rounded once (ties to even) and saturated.
//
// Activations are staged in LDS as signed byte digits: a Q16.16 value v is
// sum_l d_l * 256^l with d_l in [-128, 127], taken as the bytes of
// v + 0x8080808080 each xor 0x80. The representation is unique, so the digits
// do not depend on how many are kept; a chunk keeps as many as its largest
// value needs (1 to 5). Each digit plane times the int8 weights is an exact
// v_dot4_i32_i8 sum (|sum| < 2^19 per block), and the planes recombine into
// the exact 64-bit block sum.
#include "detnum_dev.h"
#include "q8_internal.h"
#include "act_planes.h"
#include "q8_epilogue.h"
#include "wave_ops.h"

namespace {

constexpr int KC_BLOCKS = 128;            // blocks staged per chunk (4096 values)
constexpr int KC_WORDS = KC_BLOCKS * 8;   // dwords per digit plane per chunk
constexpr int MAX_LIMBS = 5;
constexpr int GEMV_WAVES = 8;             // waves per workgroup
constexpr int GEMV_THREADS = GEMV_WAVES * 64;

__device__ __forceinline__ uint64_t digits5(int32_t v) {
    return (uint64_t)((int64_t)v + 0x8080808080LL) ^ 0x8080808080ULL;
}

__device__ __forceinline__ int limbs_needed(uint64_t d) {
    return (d >> 32) ? 5 : (d >> 24) ? 4 : (d >> 16) ? 3 : (d >> 8) ? 2 : 1;
}

__device__ __forceinline__ int wave_max_int(int v) {
    for (int off = 32; off >= 1; off >>= 1) v = max(v, __shfl_xor(v, off));
    return v;
}

// Sum of the four kgroups (lanes r, r+16, r+32, r+48) of a wave.
__device__ __forceinline__ dn::i128 kgroup_sum(dn::i128 v) {
    for (int off = 16; off <= 32; off <<= 1) {
        uint64_t lo = (uint64_t)v, hi = (uint64_t)(v >> 64);
        uint64_t olo = __shfl_xor(lo, off), ohi = __shfl_xor(hi, off);
        v += (dn::i128)(((dn::u128)ohi << 64) | olo);
    }
    return v;
}

// Planes l0 .. l0+N-1 of one block's sum: their 16-byte LDS reads are all
// issued before the first dot product, and each plane's sum is two
// independent chains (|half| < 2^18, so the i32 sums are exact).
template <int L0, int N>
__device__ __forceinline__ int64_t plane_sums(const uint4 q0, const uint4 q1, const uint32_t* lb, uint32_t pw) {
    uint4 p[N][2];
#pragma unroll
    for (int l = 0; l < N; l++) {
        p[l][0] = *(const uint4*)(lb + (L0 + l) * pw);
        p[l][1] = *(const uint4*)(lb + (L0 + l) * pw + 4);
    }
    int64_t bs = 0;
#pragma unroll
    for (int l = 0; l < N; l++) {
        int s0 = 0, s1 = 0;
        s0 = __builtin_amdgcn_sdot4((int)q0.x, (int)p[l][0].x, s0, false);
        s1 = __builtin_amdgcn_sdot4((int)q1.x, (int)p[l][1].x, s1, false);
        s0 = __builtin_amdgcn_sdot4((int)q0.y, (int)p[l][0].y, s0, false);
        s1 = __builtin_amdgcn_sdot4((int)q1.y, (int)p[l][1].y, s1, false);
        s0 = __builtin_amdgcn_sdot4((int)q0.z, (int)p[l][0].z, s0, false);
        s1 = __builtin_amdgcn_sdot4((int)q1.z, (int)p[l][1].z, s1, false);
        s0 = __builtin_amdgcn_sdot4((int)q0.w, (int)p[l][0].w, s0, false);
        s1 = __builtin_amdgcn_sdot4((int)q1.w, (int)p[l][1].w, s1, false);
        bs += (int64_t)(s0 + s1) << (8 * (L0 + l));
    }
    return bs;
}

// Exact sum of one block's 32 int8 weights (q0: bytes 0-15, q1: 16-31)
// times the values whose L digit planes start at lb (plane stride pw
// dwords, 32-byte aligned), the planes read three at a time.
template <int L>
__device__ __forceinline__ int64_t block_sum_pw(const uint4 q0, const uint4 q1, const uint32_t* lb, uint32_t pw) {
    if constexpr (L <= 3) return plane_sums<0, L>(q0, q1, lb, pw);
    else return plane_sums<0, 3>(q0, q1, lb, pw) + plane_sums<3, L - 3>(q0, q1, lb, pw);
}

// block_sum_pw for a digit count that is uniform over the wave (held in a
// scalar register): one scalar branch per block picks the unrolled body.
__device__ __forceinline__ int64_t block_sum_planes(const uint4 q0, const uint4 q1, const uint32_t* lb, uint32_t pw,
                                                    int L) {
    switch (L) {
        case 1: return block_sum_pw<1>(q0, q1, lb, pw);
        case 2: return block_sum_pw<2>(q0, q1, lb, pw);
        case 3: return block_sum_pw<3>(q0, q1, lb, pw);
        case 4: return block_sum_pw<4>(q0, q1, lb, pw);
        default: return block_sum_pw<5>(q0, q1, lb, pw);
    }
}

// The blocks of one chunk this lane owns, accumulated into acc (i64 sum of
// block sums in row-scale mode, exact 128-bit sum of scaled block sums else).
template <int L, int MODE>
__device__ __forceinline__ void chunk_blocks(const Q8View& w, uint32_t tile, uint32_t cb0, uint32_t cb1,
                                             uint32_t slot, uint32_t r, const uint32_t* lds, int64_t& acc64,
                                             dn::i128& acc128) {
    const uint8_t* qrow = w.qs + (size_t)tile * w.nb * Q8_TILE_BLOCK_BYTES + r * 16;
    const size_t sbase = (size_t)tile * w.nb * Q8_TILE_ROWS + r;
    for (uint32_t b = cb0 + slot; b < cb1; b += 4 * GEMV_WAVES) {
        const uint8_t* qp = qrow + (size_t)b * Q8_TILE_BLOCK_BYTES;
        const uint4 q0 = *(const uint4*)qp;
        const uint4 q1 = *(const uint4*)(qp + 256);
        const int64_t bs = block_sum_pw<L>(q0, q1, lds + (b - cb0) * 8, KC_WORDS);
        if constexpr (MODE == Q8_SCALE_ROW) {
            acc64 += bs;  // |bs| < 2^44 and at most 2^17 blocks: no overflow
        } else if constexpr (MODE == Q8_SCALE_F16) {
            const uint32_t bits = w.sc16[sbase + (size_t)b * Q8_TILE_ROWS];
            const uint32_t e = (bits >> 10) & 0x1f;
            const int64_t m = (int64_t)(bits & 0x3ff) | (e ? 1024 : 0);
            int64_t p = bs * m;  // < 2^55
            if (bits & 0x8000) p = -p;
            acc128 += (dn::i128)p << (e ? e - 1 : 0);
        } else {
            acc128 += (dn::i128)bs * (dn::i128)w.sc64[sbase + (size_t)b * Q8_TILE_ROWS];
        }
    }
}

// First maximum of (value, index) pairs: larger value, then smaller index
// (crates/inference/direct/src/generation.rs:25-33).
__device__ __forceinline__ void argmax_combine(int32_t& v, uint32_t& i, int32_t ov, uint32_t oi) {
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

// The head's epilogue, run by the wave finishing a tile: logits out
// (softcapped) and the tile's first maximum to the partials; the selection
// itself is the next kernel's (iris_select_launch).
__device__ __forceinline__ void head_select(const GemvArgs& a, int32_t v, uint32_t row, uint32_t lane, uint32_t tile) {
    const uint32_t step = (uint32_t)*a.d_step;
    int32_t best = INT32_MIN;
    uint32_t best_i = 0xffffffffu;
    if (lane < Q8_TILE_ROWS && row < a.w.rows) {
        const int32_t logit = dn::softcap(v, a.softcap);
        a.out[row] = logit;
        if (a.logits_keep) a.logits_keep[(size_t)step * a.w.rows + row] = logit;
        best = logit;
        best_i = row;
    }
    for (int off = 8; off >= 1; off >>= 1) argmax_combine(best, best_i, __shfl_xor(best, off), __shfl_xor(best_i, off));
    if (lane == 0) a.sel_partial[tile] = ((uint64_t)best_i << 32) | (uint32_t)best;
}

// Greedy selection (generation.rs:25-57) over the head's tile partials, in
// tile (= token id) order with the first maximum kept, then the selected
// token's embedding as the next pass's row (view_kernels.rs:37-57,
// model.rs:316-330), and the step and position advanced. With rope_next,
// threads past the embedding's also form the next one-row pass's RoPE
// (sin, cos) pairs (mistral.rs:84-109) at the advanced position, while the
// partials are on their way.
constexpr uint32_t SELECT_THREADS = 1024;

__global__ __launch_bounds__(SELECT_THREADS) void select_embed_kernel(const GemvArgs a) {
    __shared__ int32_t s_v[SELECT_THREADS / 64];
    __shared__ uint32_t s_i[SELECT_THREADS / 64];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int32_t pos0 = *a.d_pos_rw;
    int32_t best = INT32_MIN;
    uint32_t best_i = 0xffffffffu;
    for (uint32_t t = tid; t < a.w.tiles; t += SELECT_THREADS) {
        const uint64_t p = a.sel_partial[t];
        argmax_combine(best, best_i, (int32_t)(uint32_t)p, (uint32_t)(p >> 32));
    }
    if (a.rope_next && tid >= SELECT_THREADS - a.rope_half) {
        const uint32_t j = tid - (SELECT_THREADS - a.rope_half);
        int64_t sn, cs;
        dn::sin_cos_q30((int64_t)(uint32_t)(pos0 + (int32_t)a.rows_in_pass) * a.inv_freq[j], sn, cs);
        a.rope_next[2 * j] = sn;
        a.rope_next[2 * j + 1] = cs;
    }
    for (int off = 32; off >= 1; off >>= 1) argmax_combine(best, best_i, __shfl_xor(best, off), __shfl_xor(best_i, off));
    if (lane == 0) {
        s_v[wave] = best;
        s_i[wave] = best_i;
    }
    __syncthreads();
    best = s_v[0];
    best_i = s_i[0];
    for (uint32_t i = 1; i < SELECT_THREADS / 64; i++) argmax_combine(best, best_i, s_v[i], s_i[i]);
    const uint32_t token = best_i;
    const uint8_t* er = a.embed_raw + (size_t)token * a.embed_row_bytes;
    for (uint32_t c = tid; c < a.hidden; c += SELECT_THREADS) {
        const uint8_t* blk = er + (size_t)(c / 32) * 34;
        const int64_t sc = dn::scale_q24((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        int32_t e = dn::round_to_i32((dn::i128)((int64_t)(int8_t)blk[2 + c % 32] * sc), 8);
        a.x_next[c] = dn::mul_sat(e, a.embed_scale);
    }
    if (tid == 0) {
        const int32_t step = *a.d_step;
        a.tokens_out[step] = (int32_t)token;
        if (a.ids_next) a.ids_next[0] = (int32_t)token;
        *a.d_step = step + 1;
        *a.d_pos_rw = pos0 + (int32_t)a.rows_in_pass;
    }
}

// The row a lane finishes (lanes 16..63 repeat rows 0..15), clamped to the
// matrix, and what its epilogue needs: the row's scale (row-scale mode) and
// the epilogue's other inputs.
struct TileIn {
    int64_t row_scale;
    EpiIn epi;
};

template <int MODE>
__device__ __forceinline__ TileIn tile_inputs(const GemvArgs& a, uint32_t tile, uint32_t token, uint32_t lane) {
    const uint32_t row = min(tile * Q8_TILE_ROWS + (lane & (Q8_TILE_ROWS - 1)), a.w.rows - 1);
    TileIn in;
    in.row_scale = MODE == Q8_SCALE_ROW ? a.w.row_scale[row] : 0;
    in.epi = epilogue_inputs(a, row, token);
    return in;
}

template <int MODE>
__device__ __forceinline__ void finish_tile(const GemvArgs& a, uint32_t tile, uint32_t token, dn::i128 t, uint32_t lane,
                            const TileIn& in) {
    const Q8View& w = a.w;
    const uint32_t row = tile * Q8_TILE_ROWS + lane;
    int32_t v = 0;
    if (lane < Q8_TILE_ROWS) {
        if (MODE == Q8_SCALE_ROW) t = t * (dn::i128)in.row_scale;
        v = dn::round_to_i32(t, 24);
    }
    const int32_t partner = __shfl_xor(v, 1);  // the other row of an even/odd pair
    if (a.epilogue == EPI_HEAD_SELECT) {
        head_select(a, v, row, lane, tile);
        return;
    }
    if (a.ssq_out) {
        // The tile's rows as stored (add_sat with the residual, or as they
        // are), squared and summed with saturation over the 16 lanes.
        const bool own = lane < Q8_TILE_ROWS && row < w.rows;
        const int32_t o = a.epilogue == EPI_RESIDUAL ? dn::add_sat(v, in.epi.res) : v;
        const int64_t sq = row16_sum_sat_nonneg(own ? (int64_t)o * o : 0);
        if (lane == 0) a.ssq_out[tile] = sq;
    }
    if (a.out_planes) {
        // One gated row (EPI_SWIGLU / EPI_GEGLU, one token): each even lane's
        // output stored, and the tile's eight outputs as digit planes for the
        // product that reads them.
        const bool own = lane < Q8_TILE_ROWS && (lane & 1) == 0 && row < w.rows;
        int32_t o = 0;
        if (own) {
            const int32_t act = a.epilogue == EPI_SWIGLU ? dn::silu(v) : dn::gelu(v);
            o = dn::mul_sat(act, partner);
            a.out[row >> 1] = o;
        }
        act_planes_store8_even(o, lane, tile * (Q8_TILE_ROWS / 2), w.rows / 2, a.out_planes, a.out_counts);
        return;
    }
    if (lane >= Q8_TILE_ROWS || row >= w.rows) return;
    store_output_in(a, row, token, v, partner, in.epi);
}

// Stages x[4*i0 .. 4*i1) (after the optional rms_norm: mul_sat(mul_sat(v,
// scale), w)) as MAX_LIMBS digit planes of dwords at planes[l*pw + i - i0];
// returns the most digits any value needs.
__device__ __forceinline__ int stage_planes(const int32_t* x, const int32_t* norm_w, int32_t scale, uint32_t i0,
                                            uint32_t i1, uint32_t* planes, uint32_t pw, uint32_t tid) {
    int need = 1;
    for (uint32_t i = i0 + tid; i < i1; i += GEMV_THREADS) {
        const uint32_t k = i * 4;
        int4 v = *(const int4*)(x + k);
        if (norm_w) {
            const int4 nw = *(const int4*)(norm_w + k);
            v.x = dn::mul_sat(dn::mul_sat(v.x, scale), nw.x);
            v.y = dn::mul_sat(dn::mul_sat(v.y, scale), nw.y);
            v.z = dn::mul_sat(dn::mul_sat(v.z, scale), nw.z);
            v.w = dn::mul_sat(dn::mul_sat(v.w, scale), nw.w);
        }
        const uint64_t d0 = digits5(v.x), d1 = digits5(v.y), d2 = digits5(v.z), d3 = digits5(v.w);
        need = max(need, max(max(limbs_needed(d0), limbs_needed(d1)), max(limbs_needed(d2), limbs_needed(d3))));
#pragma unroll
        for (int l = 0; l < MAX_LIMBS; l++) {
            const int sh = 8 * l;
            planes[l * pw + (i - i0)] = (uint32_t)((d0 >> sh) & 0xff) | ((uint32_t)((d1 >> sh) & 0xff) << 8) |
                                        ((uint32_t)((d2 >> sh) & 0xff) << 16) | ((uint32_t)((d3 >> sh) & 0xff) << 24);
        }
    }
    return need;
}

// Digit planes of the four values at dword index i (after the optional
// norm: mul_sat(mul_sat(v, scale), w)); returns the digits the largest needs.
__device__ __forceinline__ int stage_int4(int4 v, bool norm, int4 nw, int32_t scale, uint32_t i, uint32_t* planes,
                                          uint32_t pw) {
    if (norm) {
        v.x = dn::mul_sat(dn::mul_sat(v.x, scale), nw.x);
        v.y = dn::mul_sat(dn::mul_sat(v.y, scale), nw.y);
        v.z = dn::mul_sat(dn::mul_sat(v.z, scale), nw.z);
        v.w = dn::mul_sat(dn::mul_sat(v.w, scale), nw.w);
    }
    const uint64_t d0 = digits5(v.x), d1 = digits5(v.y), d2 = digits5(v.z), d3 = digits5(v.w);
    const int need = max(max(limbs_needed(d0), limbs_needed(d1)), max(limbs_needed(d2), limbs_needed(d3)));
#pragma unroll
    for (int l = 0; l < MAX_LIMBS; l++) {
        const int sh = 8 * l;
        planes[l * pw + i] = (uint32_t)((d0 >> sh) & 0xff) | ((uint32_t)((d1 >> sh) & 0xff) << 8) |
                             ((uint32_t)((d2 >> sh) & 0xff) << 16) | ((uint32_t)((d3 >> sh) & 0xff) << 24);
    }
    return need;
}

// add_sat(mul_sat(mul_sat(v, scale), w), r), then mul_sat(., scalar) when
// scalar is set: a post-norm with its residual and layer scalar.
__device__ __forceinline__ int4 norm_res4(int4 v, int4 w, int4 r, int32_t scale, int32_t scalar) {
    int4 y;
    y.x = dn::add_sat(dn::mul_sat(dn::mul_sat(v.x, scale), w.x), r.x);
    y.y = dn::add_sat(dn::mul_sat(dn::mul_sat(v.y, scale), w.y), r.y);
    y.z = dn::add_sat(dn::mul_sat(dn::mul_sat(v.z, scale), w.z), r.z);
    y.w = dn::add_sat(dn::mul_sat(dn::mul_sat(v.w, scale), w.w), r.w);
    if (scalar != 0) {
        y.x = dn::mul_sat(y.x, scalar);
        y.y = dn::mul_sat(y.y, scalar);
        y.z = dn::mul_sat(y.z, scalar);
        y.w = dn::mul_sat(y.w, scalar);
    }
    return y;
}

__device__ __forceinline__ int64_t sumsq4(int64_t s, int4 v) {
    s = dn::acc_add_sat(s, (int64_t)v.x * v.x);
    s = dn::acc_add_sat(s, (int64_t)v.y * v.y);
    s = dn::acc_add_sat(s, (int64_t)v.z * v.z);
    return dn::acc_add_sat(s, (int64_t)v.w * v.w);
}

constexpr uint32_t XROUND = 4;  // int4 loads a thread has in flight per staging round
constexpr uint32_t NRN_ROUND = 2;  // int4 of the row per thread under PRO_NORM_RES_NORM

// The persistent kernel's prologue: the row's rms_norm scale when asked
// (sum of squares: saturating, non-negative terms, so order-free) and every
// digit plane of the row in LDS. A thread issues XROUND 16-byte loads (with
// their norm weights) before it uses any of them; a row of at most
// XROUND * GEMV_THREADS dwords is read once and kept in registers between
// the two steps. issue() runs once, right after the first round's loads are
// issued: the weight loads it issues queue behind the row's, and only LDS
// barriers follow, so they stay in flight through the staging. Returns the
// digits the row needs.
//
// PRO_NORM_RES_NORM (a row of at most XROUND * NT dwords, the launcher's
// check): the row is first y = norm_res4(x, res_norm_w, res_in) with the
// scale from the producer's slots, then rms_norm'ed as above; workgroup 0
// stores y.
template <int NT, int PRO, typename Issue>
__device__ __forceinline__ int stage_row(const GemvArgs& a, const int32_t* x, uint32_t pw, uint32_t* planes, int64_t* ssq,
                         uint32_t tid, Issue&& issue) {
    const uint32_t lane = tid & 63, wave = tid >> 6;
    constexpr bool NORM = PRO != PRO_NONE;
    constexpr bool norm = NORM;
    const int4* x4 = (const int4*)x;
    const int4* n4 = (const int4*)a.norm_w;
    // Out-of-range slots load the row's last dword (always valid) and are
    // dropped afterwards: no load sits behind a branch, so the counted waits
    // for them stay exact and the weight loads issued next stay in flight.
    auto load_round = [&](uint32_t i0, int4 (&v)[XROUND], int4 (&nw)[XROUND]) {
#pragma unroll
        for (uint32_t u = 0; u < XROUND; u++) v[u] = x4[min(i0 + u * NT + tid, pw - 1)];
#pragma unroll
        for (uint32_t u = 0; u < XROUND; u++) nw[u] = NORM ? n4[min(i0 + u * NT + tid, pw - 1)] : make_int4(0, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    };
    auto round_sumsq = [&](uint32_t i0, const int4 (&v)[XROUND], int64_t s) {
#pragma unroll
        for (uint32_t u = 0; u < XROUND; u++) {
            const bool ok = i0 + u * NT + tid < pw;
            const int4 m = make_int4(ok ? v[u].x : 0, ok ? v[u].y : 0, ok ? v[u].z : 0, ok ? v[u].w : 0);
            s = sumsq4(s, m);
        }
        return s;
    };
    auto round_stage = [&](uint32_t i0, const int4 (&v)[XROUND], const int4 (&nw)[XROUND], int32_t scale, int need) {
#pragma unroll
        for (uint32_t u = 0; u < XROUND; u++) {
            const uint32_t i = i0 + u * NT + tid;
            if (i < pw) need = max(need, stage_int4(v[u], norm, nw[u], scale, i, planes, pw));
        }
        return need;
    };
    // Every wave forms the sum of the wave totals itself: one barrier.
    auto finish_scale = [&](int64_t s) -> int32_t {
        s = wave_sum_sat_nonneg(s);
        if (lane == 0) ssq[wave] = s;
        lds_barrier();
        int64_t t = 0;
        for (int i = 0; i < NT / 64; i++) t = dn::acc_add_sat(t, ssq[i]);
        return dn::rms_scale_from_sum(t, pw * 4, a.norm_eps);
    };
    int4 v[XROUND], nw[XROUND];
    constexpr uint32_t SPL = GEMV_SSQ_SLOTS / 64;
    if constexpr (PRO == PRO_NORM_RES_NORM) {
        // At most NRN_ROUND dwords per thread (the launcher's limit): x, its
        // norm weights, the residual and both norms' weights in registers.
        int4 xv[NRN_ROUND], wv[NRN_ROUND], rv[NRN_ROUND], mv[NRN_ROUND];
        const int4* r4 = (const int4*)a.res_in;
        const int4* rw4 = (const int4*)a.res_norm_w;
#pragma unroll
        for (uint32_t u = 0; u < NRN_ROUND; u++) xv[u] = x4[min(u * NT + tid, pw - 1)];
#pragma unroll
        for (uint32_t u = 0; u < NRN_ROUND; u++) rv[u] = r4[min(u * NT + tid, pw - 1)];
#pragma unroll
        for (uint32_t u = 0; u < NRN_ROUND; u++) wv[u] = rw4[min(u * NT + tid, pw - 1)];
#pragma unroll
        for (uint32_t u = 0; u < NRN_ROUND; u++) mv[u] = n4[min(u * NT + tid, pw - 1)];
        int64_t sl[SPL];
#pragma unroll
        for (uint32_t u = 0; u < SPL; u++) sl[u] = a.ssq_in[min(lane + 64 * u, a.ssq_n - 1)];
        __builtin_amdgcn_sched_barrier(0);
        issue();
        int64_t t = 0;
#pragma unroll
        for (uint32_t u = 0; u < SPL; u++)
            if (lane + 64 * u < a.ssq_n) t = dn::acc_add_sat(t, sl[u]);
        const int32_t scale1 = dn::rms_scale_from_sum(wave_sum_sat_nonneg(t), pw * 4, a.norm_eps);
        const bool store = a.res_out != nullptr && blockIdx.x == 0;
        int64_t s = 0;
#pragma unroll
        for (uint32_t u = 0; u < NRN_ROUND; u++) {
            const uint32_t i = u * NT + tid;
            xv[u] = norm_res4(xv[u], wv[u], rv[u], scale1, a.res_scalar);
            if (i < pw) {
                if (store) ((int4*)a.res_out)[i] = xv[u];
                s = sumsq4(s, xv[u]);
            }
        }
        const int32_t scale2 = finish_scale(s);
        int need = 1;
#pragma unroll
        for (uint32_t u = 0; u < NRN_ROUND; u++) {
            const uint32_t i = u * NT + tid;
            if (i < pw) need = max(need, stage_int4(xv[u], true, mv[u], scale2, i, planes, pw));
        }
        return need;
    }
    if (pw <= XROUND * NT) {
        load_round(0, v, nw);
        // The producer's per-tile sums of squares, when given: loaded with
        // the row (unconditionally: the row itself stands in when unused),
        // summed by every wave on its own, so no barrier waits for the
        // slowest wave's row before the planes.
        const bool slots = norm && a.ssq_in != nullptr;
        int64_t sl[SPL];
#pragma unroll
        for (uint32_t u = 0; u < SPL; u++)
            sl[u] = slots ? a.ssq_in[min(lane + 64 * u, a.ssq_n - 1)] : ((const int64_t*)x)[u];
        issue();
        int32_t scale = 0;
        if (slots) {
            int64_t t = 0;
#pragma unroll
            for (uint32_t u = 0; u < SPL; u++)
                if (lane + 64 * u < a.ssq_n) t = dn::acc_add_sat(t, sl[u]);
            scale = dn::rms_scale_from_sum(wave_sum_sat_nonneg(t), pw * 4, a.norm_eps);
        } else if (norm) {
            scale = finish_scale(round_sumsq(0, v, 0));
        }
        return round_stage(0, v, nw, scale, 1);
    }
    int32_t scale = 0;
    bool issued = false;
    if (norm) {
        int64_t s = 0;
        for (uint32_t i0 = 0; i0 < pw; i0 += XROUND * NT) {
            load_round(i0, v, nw);
            if (!issued) issue();
            issued = true;
            s = round_sumsq(i0, v, s);
        }
        scale = finish_scale(s);
    }
    int need = 1;
    for (uint32_t i0 = 0; i0 < pw; i0 += XROUND * NT) {
        load_round(i0, v, nw);
        if (!issued) issue();
        issued = true;
        need = round_stage(i0, v, nw, scale, need);
    }
    return need;
}

// The persistent kernel's prologue staged by each wave on its own (PRO_NONE,
// or PRO_RMSNORM from the producer's slots). A wave's blocks are
// tile_blocks' slots part * 4 + g of nslots: the runs of four consecutive
// blocks starting at part * 4 + j * nslots, 32 plane dwords each. The wave
// stages the digit planes of those dwords only, at their places in planes,
// and returns the digits its own values need: no wave waits for another's
// row, and the digit count may differ between waves (the digits of a value
// do not depend on how many are kept). Waves of one part write the same
// values to the same places. issue() runs right after the first round's
// row loads are issued, as in stage_row.
template <int PRO, typename Issue>
__device__ __forceinline__ int stage_wave(const GemvArgs& a, const int32_t* x, uint32_t pw, uint32_t* planes,
                                          uint32_t part, uint32_t nslots, uint32_t lane, Issue&& issue) {
    constexpr bool NORM = PRO == PRO_RMSNORM;
    const int4* x4 = (const int4*)x;
    const int4* n4 = (const int4*)a.norm_w;
    const uint32_t span = nslots * 8, first = part * 32;
    const uint32_t runs = first < pw ? (pw - first + span - 1) / span : 0;
    const uint32_t n = runs * 32;  // the wave's dwords, some of the last run past the row
    auto at = [&](uint32_t q) { return first + (q >> 5) * span + (q & 31); };
    int4 v[XROUND], nw[XROUND];
    auto load_round = [&](uint32_t q0) {
#pragma unroll
        for (uint32_t u = 0; u < XROUND; u++) {
            const uint32_t q = q0 + 64 * u + lane;
            const uint32_t i = q < n ? min(at(q), pw - 1) : pw - 1;
            v[u] = x4[i];
            nw[u] = NORM ? n4[i] : make_int4(0, 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    load_round(0);
    constexpr uint32_t SPL = GEMV_SSQ_SLOTS / 64;
    int64_t sl[SPL];
    if constexpr (NORM) {
#pragma unroll
        for (uint32_t u = 0; u < SPL; u++) sl[u] = a.ssq_in[min(lane + 64 * u, a.ssq_n - 1)];
    }
    issue();
    int32_t scale = 0;
    if constexpr (NORM) {
        int64_t t = 0;
#pragma unroll
        for (uint32_t u = 0; u < SPL; u++)
            if (lane + 64 * u < a.ssq_n) t = dn::acc_add_sat(t, sl[u]);
        scale = dn::rms_scale_from_sum(wave_sum_sat_nonneg(t), pw * 4, a.norm_eps);
    }
    int need = 1;
    for (uint32_t q0 = 0;;) {
#pragma unroll
        for (uint32_t u = 0; u < XROUND; u++) {
            const uint32_t q = q0 + 64 * u + lane;
            const uint32_t i = at(q);
            if (q < n && i < pw) need = max(need, stage_int4(v[u], NORM, nw[u], scale, i, planes, pw));
        }
        q0 += 64 * XROUND;
        if (q0 >= n) break;
        load_round(q0);
    }
    return need;
}

// One block's contribution to the lane's accumulator (L digit planes,
// uniform over the wave).
template <int MODE>
__device__ __forceinline__ void accumulate_block(const uint4 q0, const uint4 q1, uint32_t sbits, int64_t sc64,
                                                 const uint32_t* lb, uint32_t pw, int L, int64_t& acc64,
                                                 dn::i128& acc128) {
    const int64_t bs = block_sum_planes(q0, q1, lb, pw, L);
    if constexpr (MODE == Q8_SCALE_ROW) {
        acc64 += bs;  // |bs| < 2^44 and at most 2^17 blocks: no overflow
    } else if constexpr (MODE == Q8_SCALE_F16) {
        const uint32_t e = (sbits >> 10) & 0x1f;
        const int64_t m = (int64_t)(sbits & 0x3ff) | (e ? 1024 : 0);
        int64_t p = bs * m;  // < 2^55
        if (sbits & 0x8000) p = -p;
        acc128 += (dn::i128)p << (e ? e - 1 : 0);
    } else {
        acc128 += (dn::i128)bs * (dn::i128)sc64;
    }
}

constexpr int BATCH = 2;  // blocks a lane has in flight while it computes the previous batch

// A batch of one lane's blocks: weights and the scale each needs.
struct BlockBatch {
    uint4 q[BATCH][2];
    uint32_t s[BATCH];
    int64_t w[BATCH];
};

// Loads blocks slot + (k0 + u) * nslots of a tile; an index past the lane's
// last block re-reads that block (its result is not used).
template <int MODE>
__device__ __forceinline__ void fetch_batch(const Q8View& w, uint32_t tile, uint32_t slot, uint32_t nslots,
                                            uint32_t last, uint32_t r, uint32_t k0, BlockBatch& bb) {
    const uint8_t* qrow = w.qs + (size_t)tile * w.nb * Q8_TILE_BLOCK_BYTES + r * 16;
    const size_t sbase = (size_t)tile * w.nb * Q8_TILE_ROWS + r;
#pragma unroll
    for (int u = 0; u < BATCH; u++) {
        const uint32_t b = min(slot + (k0 + u) * nslots, last);
        const uint8_t* qp = qrow + (size_t)b * Q8_TILE_BLOCK_BYTES;
        bb.q[u][0] = *(const uint4*)qp;
        bb.q[u][1] = *(const uint4*)(qp + 256);
        if constexpr (MODE == Q8_SCALE_F16) bb.s[u] = w.sc16[sbase + (size_t)b * Q8_TILE_ROWS];
        if constexpr (MODE == Q8_SCALE_I64) bb.w[u] = w.sc64[sbase + (size_t)b * Q8_TILE_ROWS];
    }
}

__device__ __forceinline__ uint32_t lane_block_count(uint32_t nb, uint32_t slot, uint32_t nslots) {
    return slot < nb ? (nb - slot + nslots - 1) / nslots : 0;
}

// One batch's blocks (k0, k0 + 1, ... of the lane's) into the accumulator.
// Slots past the lane's last block were fetched as that block again; their
// planes are read at the same clamped index and their sums dropped, so no
// read waits on a branch.
template <int MODE>
__device__ __forceinline__ void consume_batch(const BlockBatch& bb, uint32_t k0, uint32_t cnt, uint32_t slot,
                                              uint32_t nslots, uint32_t last, const uint32_t* planes, uint32_t pw,
                                              int L, int64_t& acc64, dn::i128& acc128) {
#pragma unroll
    for (int u = 0; u < BATCH; u++) {
        const uint32_t b = min(slot + (k0 + u) * nslots, last);
        int64_t a64 = 0;
        dn::i128 a128 = 0;
        accumulate_block<MODE>(bb.q[u][0], bb.q[u][1], bb.s[u], bb.w[u], planes + b * 8, pw, L, a64, a128);
        if (k0 + u < cnt) {
            acc64 += a64;
            acc128 += a128;
        }
    }
}

// All of one tile's blocks this lane owns (slot, slot + nslots, ...), against
// L digit planes covering the whole row (plane stride pw dwords). Two
// batches are in flight while one is summed; the caller may already have
// issued the first `prefetched` of them (0, 1 or 2) into b0 and b1.
template <int MODE>
__device__ __forceinline__ void tile_blocks(const Q8View& w, uint32_t tile, uint32_t slot, uint32_t nslots, uint32_t r,
                                            const uint32_t* planes, uint32_t pw, int L, int64_t& acc64,
                                            dn::i128& acc128, BlockBatch& b0, BlockBatch& b1, uint32_t prefetched) {
    const uint32_t cnt = lane_block_count(w.nb, slot, nslots);
    if (cnt == 0) return;
    const uint32_t last = slot + (cnt - 1) * nslots;
    if (prefetched < 1) fetch_batch<MODE>(w, tile, slot, nslots, last, r, 0, b0);
    if (prefetched < 2) fetch_batch<MODE>(w, tile, slot, nslots, last, r, BATCH, b1);
    for (uint32_t k0 = 0; k0 < cnt; k0 += 2 * BATCH) {
        consume_batch<MODE>(b0, k0, cnt, slot, nslots, last, planes, pw, L, acc64, acc128);
        if (k0 + 2 * BATCH < cnt) fetch_batch<MODE>(w, tile, slot, nslots, last, r, k0 + 2 * BATCH, b0);
        if (k0 + BATCH < cnt) {
            consume_batch<MODE>(b1, k0 + BATCH, cnt, slot, nslots, last, planes, pw, L, acc64, acc128);
            if (k0 + 3 * BATCH < cnt) fetch_batch<MODE>(w, tile, slot, nslots, last, r, k0 + 3 * BATCH, b1);
        }
    }
}

template <int MODE>
__global__ __launch_bounds__(GEMV_THREADS) void q8_gemv_kernel(const GemvArgs a) {
    __shared__ __align__(16) uint32_t lds[MAX_LIMBS * KC_WORDS];
    __shared__ dn::i128 red[GEMV_WAVES][Q8_TILE_ROWS];
    __shared__ int64_t ssq[GEMV_WAVES];
    __shared__ int32_t s_scale;
    __shared__ int s_limbs;

    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6, lane = tid & 63;
    const uint32_t r = lane & 15, g = lane >> 4;
    const uint32_t slot = wave * 4 + g;
    const uint32_t tile = blockIdx.x;
    const uint32_t token = blockIdx.y;
    const Q8View& w = a.w;
    const uint32_t K = w.cols;
    const int32_t* x = a.x + (size_t)token * a.x_stride;

    int32_t scale = 0;
    if (a.prologue == PRO_RMSNORM) {
        int64_t s = 0;
        for (uint32_t k = tid; k < K; k += GEMV_THREADS) s = dn::acc_add_sat(s, (int64_t)x[k] * x[k]);
        s = wave_sum_sat_nonneg(s);
        if (lane == 0) ssq[wave] = s;
        __syncthreads();
        if (tid == 0) {
            int64_t t = 0;
            for (int i = 0; i < GEMV_WAVES; i++) t = dn::acc_add_sat(t, ssq[i]);
            s_scale = dn::rms_scale_from_sum(t, K, a.norm_eps);
        }
        __syncthreads();
        scale = s_scale;
    }

    int64_t acc64 = 0;
    dn::i128 acc128 = 0;
    for (uint32_t cb0 = 0; cb0 < w.nb; cb0 += KC_BLOCKS) {
        const uint32_t cb1 = min(cb0 + KC_BLOCKS, w.nb);
        if (tid == 0) s_limbs = 1;
        __syncthreads();  // also: the previous chunk's readers are done
        int need = 1;
        const uint32_t words = (cb1 - cb0) * 8;
        for (uint32_t i = tid; i < words; i += GEMV_THREADS) {
            const uint32_t k = cb0 * 32 + i * 4;
            int4 v = *(const int4*)(x + k);
            if (a.prologue == PRO_RMSNORM) {
                const int4 nw = *(const int4*)(a.norm_w + k);
                v.x = dn::mul_sat(dn::mul_sat(v.x, scale), nw.x);
                v.y = dn::mul_sat(dn::mul_sat(v.y, scale), nw.y);
                v.z = dn::mul_sat(dn::mul_sat(v.z, scale), nw.z);
                v.w = dn::mul_sat(dn::mul_sat(v.w, scale), nw.w);
            }
            const uint64_t d0 = digits5(v.x), d1 = digits5(v.y), d2 = digits5(v.z), d3 = digits5(v.w);
            need = max(need, max(max(limbs_needed(d0), limbs_needed(d1)), max(limbs_needed(d2), limbs_needed(d3))));
#pragma unroll
            for (int l = 0; l < MAX_LIMBS; l++) {
                const int sh = 8 * l;
                lds[l * KC_WORDS + i] = (uint32_t)((d0 >> sh) & 0xff) | ((uint32_t)((d1 >> sh) & 0xff) << 8) |
                                        ((uint32_t)((d2 >> sh) & 0xff) << 16) |
                                        ((uint32_t)((d3 >> sh) & 0xff) << 24);
            }
        }
        need = wave_max_int(need);  // one LDS atomic per wave, not per lane
        if (lane == 0) atomicMax(&s_limbs, need);
        __syncthreads();
        switch (s_limbs) {
            case 1: chunk_blocks<1, MODE>(w, tile, cb0, cb1, slot, r, lds, acc64, acc128); break;
            case 2: chunk_blocks<2, MODE>(w, tile, cb0, cb1, slot, r, lds, acc64, acc128); break;
            case 3: chunk_blocks<3, MODE>(w, tile, cb0, cb1, slot, r, lds, acc64, acc128); break;
            case 4: chunk_blocks<4, MODE>(w, tile, cb0, cb1, slot, r, lds, acc64, acc128); break;
            default: chunk_blocks<5, MODE>(w, tile, cb0, cb1, slot, r, lds, acc64, acc128); break;
        }
    }

    dn::i128 total = MODE == Q8_SCALE_ROW ? (dn::i128)acc64 : acc128;
    total = kgroup_sum(total);
    if (g == 0) red[wave][r] = total;
    __syncthreads();
    if (wave != 0) return;
    // Wave 0 finishes the tile: lanes 0..15 own its rows.
    dn::i128 t = 0;
    if (lane < Q8_TILE_ROWS)
#pragma unroll
        for (int i = 0; i < GEMV_WAVES; i++) t += red[i][lane];
    finish_tile<MODE>(a, tile, token, t, lane, tile_inputs<MODE>(a, tile, token, lane));
}

// W waves per workgroup: 8 (two workgroups per CU) for matrices with many
// tiles, 16 (one per CU, the same 16 waves) when a matrix has at most one
// tile per CU, so that its few tiles still keep every wave slot busy.
template <int MODE, int W, int PRO>
__global__ __launch_bounds__(W * 64, 4) void q8_gemv_persistent(const GemvArgs a, const uint32_t split,
                                                                 const uint32_t ahead, const uint32_t wave_stage) {
    extern __shared__ __align__(16) uint32_t planes[];  // MAX_LIMBS planes of K/4 dwords
    __shared__ dn::i128 red[W][Q8_TILE_ROWS];
    __shared__ TileIn s_in[W * Q8_TILE_ROWS];  // the first group's epilogue inputs, by tile and row
    __shared__ int64_t ssq[W];
    __shared__ int s_need[W];

    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6, lane = tid & 63;
    const uint32_t r = lane & 15, g = lane >> 4;
    const uint32_t token = blockIdx.y;
    const Q8View& w = a.w;
    const uint32_t K = w.cols, pw = K / 4;
    const int32_t* x = a.x + (size_t)token * a.x_stride;

    // Tiles in groups of W / split; split waves share a tile's blocks.
    const uint32_t per_group = W / split;
    const uint32_t groups = (w.tiles + per_group - 1) / per_group;
    const uint32_t part = wave % split;
    const uint32_t slot = part * 4 + g, nslots = split * 4;

    // The first `ahead` batches (one or two, the launcher's choice; with one
    // the second goes out right after the staging) of this wave's first tile
    // go out right after the row's own loads (the weights do not depend on
    // the row), so the weight latency runs under the staging. The fewer
    // weight loads queue in front of the other waves' row loads on the CU,
    // the sooner those rows arrive: one batch ahead is faster wherever a
    // workgroup streams less than 192 KB (N=14336, K=4096: 15.71 -> 15.30
    // us; Gemma-2B decode 1.758 -> 1.728 ms per token), two where it
    // streams more (Mistral-7B gate/up and head; decode 2.668 -> 2.653 ms).
    // Unconditional, from clamped indices (a wave past the last tile or a
    // lane without blocks reads valid blocks it never uses): a load behind a
    // branch would make the counted waits of the staging wait for it.
    //
    // A barrier first lets every wave's row loads reach the memory pipeline
    // ahead of any wave's weight loads. Behind the weights, the first
    // group's epilogue inputs (row scales, residuals, rotations): one entry
    // per thread (clamped likewise), waited for only when the sums are done
    // and parked in LDS for the lanes that finish each row.
    BlockBatch b0, b1;
    const uint32_t nin = per_group * Q8_TILE_ROWS;
    TileIn in_mine;
    auto issue = [&]() __attribute__((always_inline)) {
        __builtin_amdgcn_s_barrier();
        const uint32_t tile0 = min(blockIdx.x * per_group + wave / split, w.tiles - 1);
        const uint32_t cnt = lane_block_count(w.nb, slot, nslots);
        const uint32_t last = cnt ? slot + (cnt - 1) * nslots : w.nb - 1;
        fetch_batch<MODE>(w, tile0, slot, nslots, last, r, 0, b0);
        if (ahead > 1) fetch_batch<MODE>(w, tile0, slot, nslots, last, r, BATCH, b1);
        in_mine = tile_inputs<MODE>(a, min(blockIdx.x * per_group + (tid % nin) / Q8_TILE_ROWS, w.tiles - 1), token,
                                    tid % nin);
    };

    // Once per workgroup: the norm scale and every digit plane of the row;
    // or (wave_stage) each wave's own blocks' planes, staged by the wave.
    int limbs;
    if (PRO != PRO_NORM_RES_NORM && wave_stage) {
        limbs = wave_max_int(stage_wave<PRO>(a, x, pw, planes, part, nslots, lane, issue));
        // The wave reads only what its own lanes wrote: LDS keeps one wave's
        // accesses in order, the fence keeps the compiler from moving them.
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
    } else {
        const int need = stage_row<W * 64, PRO>(a, x, pw, planes, ssq, tid, issue);
        const int wave_need = wave_max_int(need);
        if (lane == 0) s_need[wave] = wave_need;
        lds_barrier();
        limbs = s_need[0];
#pragma unroll
        for (int i = 1; i < W; i++) limbs = max(limbs, s_need[i]);
    }

    // One group of tiles; the first group is the workgroup's own (its
    // weights and epilogue inputs already issued), further ones (more groups
    // than workgroups) come after it.
    const int L = __builtin_amdgcn_readfirstlane(limbs);
    auto group = [&](uint32_t grp, bool first) __attribute__((always_inline)) {
        const uint32_t tile = grp * per_group + wave / split;
        int64_t acc64 = 0;
        dn::i128 acc128 = 0;
        if (tile < w.tiles)
            tile_blocks<MODE>(w, tile, slot, nslots, r, planes, pw, L, acc64, acc128, b0, b1, first ? ahead : 0);
        dn::i128 total = MODE == Q8_SCALE_ROW ? (dn::i128)acc64 : acc128;
        total = kgroup_sum(total);
        if (first) {
            if (tid < nin) s_in[tid] = in_mine;
            __syncthreads();
        }
        if (split == 1) {
            if (tile < w.tiles)
                finish_tile<MODE>(a, tile, token, total, lane,
                                  first ? s_in[(wave / split) * Q8_TILE_ROWS + r] : tile_inputs<MODE>(a, tile, token, lane));
            return;
        }
        if (g == 0) red[wave][r] = total;
        __syncthreads();
        if (part == 0 && tile < w.tiles) {
            // Every partial of the workgroup is read (all loads in flight
            // together); those of the tile's split waves are summed.
            dn::i128 t = 0;
#pragma unroll
            for (uint32_t i = 0; i < W; i++) {
                const dn::i128 e = red[(wave + i) % W][r];
                if (i < split) t += e;
            }
            finish_tile<MODE>(a, tile, token, t, lane,
                              first ? s_in[(wave / split) * Q8_TILE_ROWS + r] : tile_inputs<MODE>(a, tile, token, lane));
        }
        __syncthreads();
    };
    group(blockIdx.x, true);
#pragma unroll 1
    for (uint32_t grp = blockIdx.x + gridDim.x; grp < groups; grp += gridDim.x) group(grp, false);
}

// One thread per (row, block): copies the 32 weights into the tile layout
// and the scale bits into sc16; flags bit 0 = a non-finite scale.
// With interleave_half = h > 0, device row 2i reads source row i and row
// 2i+1 source row h + i.
__global__ void q8_pack_kernel(const uint8_t* raw, uint32_t rows, uint32_t nb, uint8_t* qs, uint16_t* sc16,
                               int* flags, uint32_t interleave_half) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)rows * nb) return;
    const uint32_t row = (uint32_t)(idx / nb), b = (uint32_t)(idx % nb);
    const uint32_t src_row = interleave_half ? ((row & 1) ? interleave_half + (row >> 1) : (row >> 1)) : row;
    const uint8_t* src = raw + ((size_t)src_row * nb + b) * 34;
    const uint32_t tile = row / Q8_TILE_ROWS, r = row % Q8_TILE_ROWS;
    uint8_t* dst = qs + ((size_t)tile * nb + b) * Q8_TILE_BLOCK_BYTES + r * 16;
#pragma unroll
    for (int j = 0; j < 16; j++) dst[j] = src[2 + j];
#pragma unroll
    for (int j = 0; j < 16; j++) dst[256 + j] = src[18 + j];
    const uint32_t bits = (uint32_t)src[0] | ((uint32_t)src[1] << 8);
    sc16[((size_t)tile * nb + b) * Q8_TILE_ROWS + r] = (uint16_t)bits;
    if (((bits >> 10) & 0x1f) == 0x1f) atomicOr(flags, 1);
}

// One thread per row: the row's common scale, or flags bit 1 when its blocks
// differ in value.
__global__ void q8_row_scale_kernel(const uint16_t* sc16, uint32_t rows, uint32_t nb, int64_t* row_scale,
                                    int* flags) {
    const uint32_t row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    const uint32_t tile = row / Q8_TILE_ROWS, r = row % Q8_TILE_ROWS;
    const uint16_t* s = sc16 + (size_t)tile * nb * Q8_TILE_ROWS + r;
    const int64_t first = dn::scale_q24(s[0]);
    bool same = true;
    for (uint32_t b = 1; b < nb; b++) same &= dn::scale_q24(s[(size_t)b * Q8_TILE_ROWS]) == first;
    row_scale[row] = first;
    if (!same) atomicOr(flags, 2);
}

}  // namespace

namespace {

constexpr uint32_t PERSISTENT_MAX_K = 24576;  // digit planes of a whole row: 5*K bytes of LDS
constexpr uint32_t WGS_PER_CU = 2;

int g_num_cus = 0;

void gemv_prepare_once() {
    static bool done = false;
    if (done) return;
    done = true;
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
        g_num_cus = prop.multiProcessorCount;
    if (g_num_cus <= 0) g_num_cus = 256;
    const int bytes = MAX_LIMBS * PERSISTENT_MAX_K;
#define IRIS_PERSISTENT_W(M, P) (const void*)&q8_gemv_persistent<M, 8, P>, (const void*)&q8_gemv_persistent<M, 16, P>
#define IRIS_PERSISTENT_P(P) \
    IRIS_PERSISTENT_W(Q8_SCALE_ROW, P), IRIS_PERSISTENT_W(Q8_SCALE_F16, P), IRIS_PERSISTENT_W(Q8_SCALE_I64, P)
    for (const void* f : {IRIS_PERSISTENT_P(PRO_NONE), IRIS_PERSISTENT_P(PRO_RMSNORM),
                          IRIS_PERSISTENT_P(PRO_NORM_RES_NORM)})
        hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
#undef IRIS_PERSISTENT_P
#undef IRIS_PERSISTENT_W
}

// Waves sharing one tile (of a workgroup's W): the most that still give a
// single round of tile groups (at most wgs), so every tile's blocks are
// spread as thin as one round allows; when even two waves per tile need
// more than one round, the fewest that cover 7/8 of the workgroups.
// Measured: a second, mostly empty round costs more than leaving slots
// idle (N=14336, K=4096: split 4 at 448 of 512 groups is 10% faster than
// split 8 at 1.75 rounds); one wave per tile is slower at every size.
uint32_t choose_split(uint32_t tiles, uint32_t w, uint64_t wgs) {
    uint32_t best = 0;
    for (uint32_t s = 2; s <= w; s *= 2)
        if ((uint64_t)tiles * s / w <= wgs) best = s;
    if (best) return best;
    for (uint32_t s = 2; s < w; s *= 2)
        if ((uint64_t)tiles * s / w >= wgs * 7 / 8) return s;
    return w;
}

// Resident 8-wave workgroups to aim for: two per CU when each CU's share of
// the matrix is large (the weight stream sets the time), one when it is
// small: a second workgroup on a CU gets its row only behind the first
// one's weight loads, and with little streaming to hide that it sets the
// kernel's end (N=6144, K=4096: 192 workgroups 17% faster than 384).
uint64_t gemv_workgroups(const Q8View& w) {
    const uint64_t share = (uint64_t)w.rows * w.cols / (uint64_t)g_num_cus;
    return share <= (128u << 10) ? (uint64_t)g_num_cus : (uint64_t)WGS_PER_CU * g_num_cus;
}

template <int W>
int launch_persistent(const GemvArgs& a, hipStream_t stream, uint64_t resident) {
    const uint32_t split = choose_split(a.w.tiles, W, resident);
    const uint32_t groups = (a.w.tiles + W / split - 1) / (W / split);
    const uint32_t wgs = min(groups, (uint32_t)resident);
    const size_t shmem = (size_t)MAX_LIMBS * a.w.cols;
    // Two weight batches ahead where an 8-wave workgroup streams at least
    // 192 KB (Mistral-7B gate/up 28.3 -> 27.7 us, head 30.0 -> 28.7 us), one
    // elsewhere (two put q/k/v at 13.4 -> 13.9 us and slow the short rows).
    const uint64_t wg_bytes = (uint64_t)(W / split) * Q8_TILE_ROWS * a.w.cols;
    const uint32_t ahead = W == 8 && wg_bytes >= (192u << 10) ? 2 : 1;
    // Each wave stages its own blocks' planes when the prologue allows it
    // (no norm, or a norm from the producer's slots).
    const bool eligible = a.prologue == PRO_NONE || (a.prologue == PRO_RMSNORM && a.ssq_in != nullptr);
    // Per wave where every split part has one wave and rows are at least
    // 4096 long (K=2048, Gemma-2B's O: 7.8 -> 8.3 us per wave; K=4096 and
    // K=14336, 16384: faster).
    const uint32_t wave_stage = eligible && split == W && a.w.cols >= 4096 ? 1 : 0;
    dim3 grid(wgs, a.tokens);
    switch (a.w.scale_mode * 3 + a.prologue) {
#define IRIS_PERSISTENT(M, P)                                                                                   \
    case M * 3 + P:                                                                                             \
        hipLaunchKernelGGL((q8_gemv_persistent<M, W, P>), grid, dim3(W * 64), shmem, stream, a, split, ahead, \
                           wave_stage);                                                                      \
        break;
#define IRIS_PERSISTENT_M(M) IRIS_PERSISTENT(M, PRO_NONE) IRIS_PERSISTENT(M, PRO_RMSNORM) IRIS_PERSISTENT(M, PRO_NORM_RES_NORM)
        IRIS_PERSISTENT_M(Q8_SCALE_ROW)
        IRIS_PERSISTENT_M(Q8_SCALE_F16)
        IRIS_PERSISTENT_M(Q8_SCALE_I64)
#undef IRIS_PERSISTENT_M
#undef IRIS_PERSISTENT
        default: return IRIS_E_INVALID;
    }
    return (int)hipGetLastError();
}

}  // namespace

void iris_gemv_prepare() { gemv_prepare_once(); }

int iris_device_cus() {
    gemv_prepare_once();
    return g_num_cus;
}

int iris_select_launch(const GemvArgs& a, hipStream_t stream) {
    if (a.rope_next && (a.rope_half == 0 || a.rope_half > SELECT_THREADS / 2 || !a.inv_freq)) return IRIS_E_INVALID;
    hipLaunchKernelGGL(select_embed_kernel, dim3(1), dim3(SELECT_THREADS), 0, stream, a);
    return (int)hipGetLastError();
}

int iris_gemv_launch(const GemvArgs& a, hipStream_t stream) {
    if (a.tokens == 0 || a.w.rows == 0) return 0;
    if (iris_gemv_bcast_applies(a)) return iris_gemv_bcast_launch(a, stream);
    // (Planes given where the broadcast product does not apply, e.g. a
    // per-block scale matrix: the row is staged from x as usual.)
    if (a.out_planes && (a.tokens != 1 || !a.out_counts || (a.epilogue != EPI_SWIGLU && a.epilogue != EPI_GEGLU) ||
                         a.w.rows % 64))
        return IRIS_E_INVALID;
    if (iris_gemm_applies(a)) return iris_gemm_launch(a, stream);
    if (a.w.cols % 32 || a.x_stride % 4 || ((uintptr_t)a.x & 15)) return IRIS_E_INVALID;
    if (a.prologue < PRO_NONE || a.prologue > PRO_NORM_RES_NORM) return IRIS_E_INVALID;
    if (a.prologue != PRO_NONE && ((uintptr_t)a.norm_w & 15)) return IRIS_E_INVALID;
    if (a.tokens > 65535) return IRIS_E_INVALID;
    if ((a.ssq_out || a.ssq_in) && a.tokens != 1) return IRIS_E_INVALID;
    if (a.ssq_out && a.epilogue != EPI_RESIDUAL && a.epilogue != EPI_STORE) return IRIS_E_INVALID;
    if (a.ssq_in && (a.prologue == PRO_NONE || a.ssq_n == 0 || a.ssq_n > GEMV_SSQ_SLOTS)) return IRIS_E_INVALID;
    if (a.prologue == PRO_NORM_RES_NORM) {
        // One row of at most NRN_ROUND dwords per thread of an 8-wave
        // workgroup, staged from the producer's slots; y is written apart
        // from every buffer the launch reads.
        if (!a.ssq_in || a.tokens != 1 || a.w.cols > NRN_ROUND * 8 * 64 * 4) return IRIS_E_INVALID;
        if (((uintptr_t)a.res_in & 15) || ((uintptr_t)a.res_norm_w & 15) || ((uintptr_t)a.res_out & 15))
            return IRIS_E_INVALID;
        if (a.res_out && (a.res_out == a.res_in || a.res_out == a.x)) return IRIS_E_INVALID;
    }
    gemv_prepare_once();
    if (a.w.cols <= PERSISTENT_MAX_K) {
        // Long rows (K >= 8192) of a matrix with at most one tile per CU: one
        // 16-wave workgroup per CU (measured faster there; slower for short rows).
        if (a.w.tiles <= (uint32_t)g_num_cus && a.w.cols >= 8192)
            return launch_persistent<16>(a, stream, (uint64_t)g_num_cus);
        return launch_persistent<8>(a, stream, gemv_workgroups(a.w));
    }
    dim3 grid(a.w.tiles, a.tokens);
    switch (a.w.scale_mode) {
        case Q8_SCALE_ROW: hipLaunchKernelGGL(q8_gemv_kernel<Q8_SCALE_ROW>, grid, dim3(GEMV_THREADS), 0, stream, a); break;
        case Q8_SCALE_F16: hipLaunchKernelGGL(q8_gemv_kernel<Q8_SCALE_F16>, grid, dim3(GEMV_THREADS), 0, stream, a); break;
        default: hipLaunchKernelGGL(q8_gemv_kernel<Q8_SCALE_I64>, grid, dim3(GEMV_THREADS), 0, stream, a); break;
    }
    return (int)hipGetLastError();
}

int iris_q8_pack_device(const uint8_t* d_raw, Q8GpuMatrix* m, hipStream_t stream, uint32_t interleave_half) {
    int* d_flags = nullptr;
    int flags = 0;
    hipError_t st = hipMalloc(&d_flags, sizeof(int));
    if (st != hipSuccess) return (int)st;
    st = hipMemsetAsync(d_flags, 0, sizeof(int), stream);
    const size_t n = (size_t)m->rows * m->nb;
    if (st == hipSuccess && n) {
        hipLaunchKernelGGL(q8_pack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, d_raw, m->rows,
                           m->nb, m->qs, m->sc16, d_flags, interleave_half);
        st = hipGetLastError();
    }
    if (st == hipSuccess && m->rows) {
        hipLaunchKernelGGL(q8_row_scale_kernel, dim3((m->rows + 255) / 256), dim3(256), 0, stream, m->sc16, m->rows,
                           m->nb, m->row_scale, d_flags);
        st = hipGetLastError();
    }
    if (st == hipSuccess) st = hipMemcpyAsync(&flags, d_flags, sizeof(int), hipMemcpyDeviceToHost, stream);
    if (st == hipSuccess) st = hipStreamSynchronize(stream);
    hipFree(d_flags);
    if (st != hipSuccess) return (int)st;
    if (flags & 1) return IRIS_E_SCALE;
    m->scale_mode = (flags & 2) ? Q8_SCALE_F16 : Q8_SCALE_ROW;
    return 0;
}
