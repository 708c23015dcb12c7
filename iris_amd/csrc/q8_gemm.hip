// Multi-token Q8_0 products on gfx950's int8 matrix cores, exact.
//
// When every block of a row shares one scale (the row-scale layout),
// det_num::q8::dot_row (crates/det-num/src/q8.rs:56-72) of a token is the
// single ties-to-even rounding of scale[row] * sum_b blocksum_b, and the
// block sums add up to the full-row integer dot product sum_k q[row][k] *
// x[k] (|.| < K * 2^38). So the product is an integer GEMM followed by the
// GEMV's rounding and epilogue. The activations are split into signed byte
// digits, x = sum_l 256^l d_l with d_l in [-128, 127] (the bytes of
// x + 0x8080808080, each xor 0x80; five digits only for x >= 0x7F7F7F80),
// and every digit plane is an int8 GEMM with exact int32 accumulation
// (|sum| <= K * 2^14 < 2^31 for K < 2^17) on v_mfma_i32_32x32x32_i8.
//
// Operand layout. One v_mfma_i32_32x32x32_i8 takes, in lane l, 16 bytes of
// row (A) or column (B) l % 32 at reduction offset 16 * (l / 32), and
// leaves output i of lane l at row 8 * (i / 4) + 4 * (l / 32) + i % 4,
// column l % 32. (On gfx950 this instruction runs at about twice the rate
// of the 16x16x64 one.) A weight operand, 32 rows by 32 k, is four 256-byte
// runs of the Q8_0 tile layout (two 16-row tiles, two 16-byte halves of a
// 32-wide block); the digit planes are written directly in operand shape:
// plane l, 32-token tile tt and 32-wide k block kb form one 1 KB block at
// ((l * TT + tt) * KB + kb) * 1024. Every operand is copied from global
// memory straight into LDS (global_load_lds_dwordx4: each lane fetches its
// own 16 bytes, the wave writes one contiguous kilobyte, no registers in
// between) through a four-deep ring of 64-wide k steps, and read back by
// each lane as one conflict-free 16-byte LDS load.
#include <mutex>

#include "detnum_dev.h"
#include "q8_epilogue.h"
#include "q8_internal.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int PL_MAX = 5;                   // digit planes of an i32
constexpr uint32_t GM_TT = 4;               // 32-token tiles per workgroup (128 tokens)
constexpr uint32_t FRAG = 1024;             // bytes of one 32 x 32 operand
constexpr uint32_t GM_BAND = 8;             // row groups per band of the launch order

// The two workgroup shapes: W waves in a (W/2) x 2 grid over 32 * W rows and
// 128 tokens (W = 8: two waves per SIMD, 256 rows, for launches that fill
// the chip; W = 4: one wave per SIMD, 128 rows, for smaller ones). A stage
// is one 64-wide k step: 2W weight operands and up to 24 digit-plane ones.
//
// SPLIT = 2 (four-wave shape only): the workgroup holds two such groups of
// W waves (two waves per SIMD), each walking half of the k steps through a
// two-stage ring of its own; the second group's int32 plane sums are then
// added into the first's (exact: the whole row's sum fits int32), and both
// groups store the block.
template <uint32_t W, uint32_t SPLIT = 1>
struct GemmShape {
    static constexpr uint32_t WAVES = W, RT = W;                     // per k group; RT: 32-row tiles
    static constexpr uint32_t SPLITS = SPLIT, THREADS = 64 * W * SPLIT;
    static constexpr int RI = 2;                                      // row tiles per wave
    static constexpr uint32_t STAGE = (2 * W + 24) * FRAG;
    static constexpr uint32_t STAGES = SPLIT == 2 ? 2 : W == 8 ? 3 : 4;
    static constexpr uint32_t RING = STAGES * STAGE;                  // per k group
    static constexpr uint32_t OUT = 32 * W * 129 * 4;  // the output block, [row][128 tokens + 1]
    static constexpr uint32_t SMEM = SPLIT * RING > OUT ? SPLIT * RING : OUT;
};

__device__ __forceinline__ uint64_t digits5(int32_t v) {
    return (uint64_t)((int64_t)v + 0x8080808080LL) ^ 0x8080808080ULL;
}

__device__ __forceinline__ int limbs_needed(uint64_t d) {
    return (d >> 32) ? 5 : (d >> 24) ? 4 : (d >> 16) ? 3 : (d >> 8) ? 2 : 1;
}

__device__ __forceinline__ uint32_t plane_byte4(uint64_t d0, uint64_t d1, uint64_t d2, uint64_t d3, int l) {
    const int sh = 8 * l;
    return (uint32_t)((d0 >> sh) & 0xff) | ((uint32_t)((d1 >> sh) & 0xff) << 8) | ((uint32_t)((d2 >> sh) & 0xff) << 16) |
           ((uint32_t)((d3 >> sh) & 0xff) << 24);
}

// Per token, one wave each, under the rms_norm prologue only: the token's
// scale (ops.rs:98-114, rms_norm_scale of the order-free saturating sum of
// squares) at token_limbs[t].
__global__ __launch_bounds__(256) void token_prep_kernel(const GemvArgs a) {
    const uint32_t t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (t >= a.tokens) return;
    {
        const uint32_t K = a.w.cols;
        const int32_t* x = a.x + (size_t)t * a.x_stride;
        int64_t s = 0;
        for (uint32_t k = lane * 4; k < K; k += 256) {
            const int4 v = *(const int4*)(x + k);
            s = dn::acc_add_sat(s, (int64_t)v.x * v.x);
            s = dn::acc_add_sat(s, (int64_t)v.y * v.y);
            s = dn::acc_add_sat(s, (int64_t)v.z * v.z);
            s = dn::acc_add_sat(s, (int64_t)v.w * v.w);
        }
        for (int off = 32; off >= 1; off >>= 1) s = dn::acc_add_sat(s, __shfl_xor(s, off));
        if (lane == 0) a.token_limbs[t] = dn::rms_scale_from_sum(s, K, a.norm_eps);
    }
}

constexpr uint32_t PLANE_KB = GEMM_PLANE_KB;

__global__ __launch_bounds__(256) void fill_ints_kernel(int32_t* p, uint32_t n, int32_t v) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = v;
}

// The digit planes of one 32-token tile over PLANE_KB k blocks (one k
// chunk) per workgroup, after the optional rms_norm (mul_sat(mul_sat(v,
// scale), w)), in the operand layout above, and the digits the chunk's
// values need, stored for the (chunk, tile) at token_limbs[M + chunk * TT +
// tile]: every launch writes each of its counts, so none needs a reset.
// Tokens past the end of the last tile get zero digits.
__global__ __launch_bounds__(256) void digit_planes_kernel(const GemvArgs a) {
    __shared__ int s_need;
    const uint32_t tt = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t K = a.w.cols, M = a.tokens, TT = (M + 31) / 32, KB = K / 32;
    const uint32_t kb0 = blockIdx.y * PLANE_KB, kb1 = min(kb0 + PLANE_KB, KB);
    const bool norm = a.prologue == PRO_RMSNORM;
    if (tid == 0) s_need = 1;
    __syncthreads();
    // Lane l writes the 16 bytes of token l % 32 at k-offset 16 * (l / 32)
    // of each 32-wide block the wave takes.
    const uint32_t tl = lane & 31, q = lane >> 5, t = tt * 32 + tl;
    const bool valid = t < M;
    const int32_t scale = norm && valid ? a.token_limbs[t] : 0;
    const int32_t* x = a.x + (size_t)(valid ? t : 0) * a.x_stride;
    const size_t lstride = (size_t)TT * KB * FRAG;
    int need = 1;
    for (uint32_t kb = kb0 + wave; kb < kb1; kb += 4) {
        const uint32_t k0 = kb * 32 + q * 16;
        uint32_t out[PL_MAX][4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            int4 v = make_int4(0, 0, 0, 0);
            if (valid) v = *(const int4*)(x + k0 + 4 * c);
            if (norm) {
                const int4 nw = *(const int4*)(a.norm_w + k0 + 4 * c);
                v.x = dn::mul_sat(dn::mul_sat(v.x, scale), nw.x);
                v.y = dn::mul_sat(dn::mul_sat(v.y, scale), nw.y);
                v.z = dn::mul_sat(dn::mul_sat(v.z, scale), nw.z);
                v.w = dn::mul_sat(dn::mul_sat(v.w, scale), nw.w);
            }
            const uint64_t d0 = digits5(v.x), d1 = digits5(v.y), d2 = digits5(v.z), d3 = digits5(v.w);
            need = max(need, max(max(limbs_needed(d0), limbs_needed(d1)), max(limbs_needed(d2), limbs_needed(d3))));
#pragma unroll
            for (int l = 0; l < PL_MAX; l++) out[l][c] = plane_byte4(d0, d1, d2, d3, l);
        }
        int8_t* dst = a.planes + ((size_t)tt * KB + kb) * FRAG + lane * 16;
#pragma unroll
        for (int l = 0; l < PL_MAX; l++)
            *(uint4*)(dst + l * lstride) = make_uint4(out[l][0], out[l][1], out[l][2], out[l][3]);
    }
    for (int off = 32; off >= 1; off >>= 1) need = max(need, __shfl_xor(need, off));
    if (lane == 0) atomicMax(&s_need, need);  // the largest of four: any order
    __syncthreads();
    if (tid == 0) a.token_limbs[M + blockIdx.y * TT + tt] = s_need;
}

// The digits a workgroup's token tiles tt0 .. tt0 + tg - 1 need: the most
// any k chunk of them needs, from digit_planes_kernel's counts.
__device__ __forceinline__ int tiles_limbs(const GemvArgs& a, uint32_t tt0, uint32_t tg, int& s_limbs) {
    const uint32_t tid = threadIdx.x, TT = (a.tokens + 31) / 32;
    const uint32_t chunks = (a.w.cols / 32 + PLANE_KB - 1) / PLANE_KB;
    const int32_t* need = a.token_limbs + a.tokens;
    if (tid == 0) s_limbs = 1;
    __syncthreads();
    for (uint32_t i = tid; i < tg * chunks; i += blockDim.x) {
        const uint32_t t = tt0 + i % tg;
        if (t < TT) atomicMax(&s_limbs, need[(i / tg) * TT + t]);
    }
    __syncthreads();
    const int limbs = s_limbs;
    __syncthreads();
    return limbs;
}

template <int N>
__device__ __forceinline__ void wait_vmem() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// 16 bytes per lane from src into LDS at byte offset lds (the wave's base,
// the same in every lane; lane i writes lds + 16i): global_load_lds_dwordx4.
// Written out here because the compiler, lacking alias information, treats
// every copy still in flight as a write to any LDS address a later ds_read
// touches, and in some shapes waited for all of them (vmcnt(0)) before each
// k step's reads, so the next step's copies, issued just before, no longer
// overlapped the step's matrix work. The k loops' own waits (wait_vmem, then
// the barrier) order each copy before the reads of its stage, and the
// compiler's waits for its own loads stay correct: the copies only make its
// vmcnt counts more conservative.
__device__ __forceinline__ void copy_to_lds16(const int8_t* src, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory");
}

// The LDS byte offset of a pointer into LDS: a flat address of LDS is the
// aperture above the offset, so its low 32 bits.
__device__ __forceinline__ uint32_t lds_offset(const void* p) { return (uint32_t)(uintptr_t)p; }

// One pass of the workgroup over the whole k range: RT weight tiles of 32
// rows (from 32-row tile rt0) times 2*TTW token tiles of 32 (from tt0) times
// LG digit planes. Wave (wr, wt) accumulates weight tiles wr*2, wr*2+1
// against token tiles wt*TTW..: acc[i][j][l] is the int32 sum of plane l
// for its 32 x 32 block. A stage holds, for its two 32-wide k blocks s, the
// weight operand of tile r at chunk 2r + s and the plane-l operand of token
// tile j at 2RT + 2(l * 2TTW + j) + s (padded to a whole number of chunks
// per wave with copies of chunk 0). Operands past the last tile are clamped
// onto it (read, never stored).
template <class G, int LG, int TTW, bool DEEP = false>
__device__ __forceinline__ void gemm_mainloop(const GemvArgs& a, int8_t* smem, uint32_t rt0, uint32_t tt0,
                                              v16i (&acc)[2][TTW][LG]) {
    constexpr uint32_t TTWG = 2 * TTW;                      // token tiles per pass
    constexpr uint32_t CHUNKS = 2 * G::RT + 2 * LG * TTWG;  // 1 KB operands per stage
    constexpr uint32_t PER_WAVE = (CHUNKS + G::WAVES - 1) / G::WAVES;
    static_assert(PER_WAVE * G::WAVES * FRAG <= G::STAGE && PER_WAVE >= 2, "stage layout");
    // The ring's stages are as large as this pass's operands, so fewer
    // digit planes leave room for more stages in the same LDS: four where
    // four fit, else the shape's own count; with DEEP (long rows), as many
    // as fit up to four. At three planes and 64 tokens the split four-wave
    // shape then runs three stages instead of two: faster over the 112 k
    // steps of a K=14336 down product (the 512-row prompt pass 20.1-20.2 ->
    // 19.6-19.75 ms), slower over K=4096 (the M=512 product 48.4 -> 49.6 us).
    constexpr uint32_t GM_RT = G::RT, GM_STAGE = PER_WAVE * G::WAVES * FRAG;
    constexpr uint32_t FIT = G::RING / GM_STAGE;
    constexpr uint32_t GM_STAGES = FIT >= 4 ? 4 : DEEP && FIT > G::STAGES ? FIT : G::STAGES;
    static_assert(GM_STAGES * GM_STAGE <= G::RING, "ring layout");
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    // The wave within its k group, the group's ring and k steps [ks0, ks1).
    // The k group through readfirstlane: uniform, so the k loop's control
    // stays in scalar registers.
    const uint32_t half = __builtin_amdgcn_readfirstlane((tid >> 6) / G::WAVES), wave = (tid >> 6) % G::WAVES;
    const uint32_t wr = wave % (G::WAVES / 2), wt = wave / (G::WAVES / 2);
    const Q8View& w = a.w;
    const uint32_t KS = w.cols / 64, KB = w.cols / 32, TT = (a.tokens + 31) / 32;
    const uint32_t ks0 = half * (KS / G::SPLITS), ks1 = ks0 + KS / G::SPLITS;
    smem += half * G::RING;
    const size_t lstride = (size_t)TT * KB * FRAG;

    // Wave w copies chunks w, w + W, ...: the first two are weight operands
    // (advancing 1 KB of the tile layout per k step), the rest plane
    // operands (advancing 2 KB).
    const int8_t* src[PER_WAVE];
    uint32_t step[PER_WAVE];
#pragma unroll
    for (uint32_t i = 0; i < PER_WAVE; i++) {
        const uint32_t c0 = wave + G::WAVES * i, c = c0 < CHUNKS ? c0 : 0;
        step[i] = c < 2 * GM_RT ? FRAG : 2 * FRAG;
        if (c < 2 * GM_RT) {
            const uint32_t r = lane & 31, h = lane >> 5, sub = c & 1;
            const uint32_t tile16 = min(2 * (rt0 + c / 2) + r / 16, w.tiles - 1);
            src[i] = (const int8_t*)w.qs + ((size_t)tile16 * w.nb + sub) * Q8_TILE_BLOCK_BYTES + h * 256 + (r % 16) * 16;
        } else {
            const uint32_t b = c - 2 * GM_RT, sub = b & 1, rest = b >> 1, l = rest / TTWG;
            const uint32_t tile = min(tt0 + rest % TTWG, TT - 1);
            src[i] = a.planes + l * lstride + ((size_t)tile * KB + sub) * FRAG + lane * 16;
        }
    }
    const uint32_t ring = lds_offset(smem);
    auto issue = [&](uint32_t ks) {
        const uint32_t base = ring + (ks % GM_STAGES) * GM_STAGE;
#pragma unroll
        for (uint32_t i = 0; i < PER_WAVE; i++)
            copy_to_lds16(src[i] + (size_t)ks * step[i], base + (wave + G::WAVES * i) * FRAG);
    };

#pragma unroll
    for (uint32_t s = 0; s < GM_STAGES - 1; s++)
        if (ks0 + s < ks1) issue(ks0 + s);
    // Both k groups take the same number of steps (the launcher's even KS),
    // so their barriers pair up.
    for (uint32_t ks = ks0; ks < ks1; ks++) {
        // This wave's copies for step ks are in LDS once at most the later
        // steps' copies are outstanding; the barrier makes every wave's
        // visible and frees the slot the next copy overwrites (read at ks-1).
        if (GM_STAGES == 2) wait_vmem<0>();
        else if (GM_STAGES >= 4 && ks + 2 < ks1) wait_vmem<(GM_STAGES >= 4 ? 2 : 1) * PER_WAVE>();
        else if (ks + 1 < ks1) wait_vmem<PER_WAVE>();
        else wait_vmem<0>();
        lds_barrier();
        if (ks + GM_STAGES - 1 < ks1) issue(ks + GM_STAGES - 1);
        const int8_t* st = smem + (ks % GM_STAGES) * GM_STAGE + lane * 16;
#pragma unroll
        for (uint32_t sub = 0; sub < 2; sub++) {
            v4i fa[2];
#pragma unroll
            for (int i = 0; i < 2; i++) fa[i] = *(const v4i*)(st + (2 * (wr * 2 + i) + sub) * FRAG);
#pragma unroll
            for (int l = 0; l < LG; l++) {
                v4i fb[TTW];
#pragma unroll
                for (int j = 0; j < TTW; j++)
                    fb[j] = *(const v4i*)(st + (2 * GM_RT + 2 * (l * TTWG + wt * TTW + j) + sub) * FRAG);
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < TTW; j++)
                        acc[i][j][l] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j][l], 0, 0, 0);
            }
        }
    }
    lds_barrier();  // every wave is done with the ring before it is reused
}

// Output e of lane l of a 32 x 32 block is row 8(e/4) + 4(l/32) + e%4,
// token l % 32. Each wave's blocks (row tiles wr*2 + i, token tiles wt*TTW
// + j) get their values from `block_values(i, j, v)`, rounded once (and,
// for the gated activations, each gate/up row pair combined in registers);
// the blocks are parked in LDS as [row][token], then the epilogue runs
// row-fastest.
// The block's gated values (parked in LDS, pair p of token tl at
// sC[p * step * STRIDE + tl]) as the next product's digit planes: each
// thread takes 16 consecutive pairs of one token (16 bytes of one operand
// lane per plane, as digit_planes_kernel writes them; tokens past the last
// of the launch, up to the end of its last 32-token tile, get zero digits),
// and the digits each 32-token tile needs meet in LDS, then in the launch's
// counts by atomicMax (the largest wins in any order). A block's pairs lie
// in one k chunk (its first pair is a multiple of ROWS / 2 <= 256).
template <class G, uint32_t NTOK>
__device__ __forceinline__ void gated_planes(const GemvArgs& a, const int32_t* sC, uint32_t rt0, uint32_t tt0,
                                             uint32_t step) {
    constexpr uint32_t ROWS = G::RT * 32, STRIDE = NTOK + 1, NG = ROWS / 2 / 16, NTT = NTOK / 32;
    static_assert(ROWS / 2 <= 32 * PLANE_KB && NTT <= 4, "one k chunk, at most four token tiles");
    __shared__ int s_need[4];
    const uint32_t tid = threadIdx.x;
    const uint32_t K = a.w.rows / 2, KB = K / 32, M = a.tokens, TT = (M + 31) / 32;
    const size_t lstride = (size_t)TT * KB * FRAG;
    if (tid < 4) s_need[tid] = 1;
    __syncthreads();
    for (uint32_t c = tid; c < NTOK * NG; c += G::THREADS) {
        const uint32_t tl = c % NTOK, gi = c / NTOK;
        const uint32_t pair0 = rt0 * 16 + gi * 16, token = tt0 * 32 + tl;
        if (pair0 >= K || token / 32 >= TT) continue;
        const bool valid = token < M;
        uint64_t d[16];
        int need = 1;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            d[j] = digits5(valid ? sC[(gi * 16 + j) * step * STRIDE + tl] : 0);
            need = max(need, limbs_needed(d[j]));
        }
        int8_t* dst = a.out_gemm_planes + ((size_t)(token / 32) * KB + pair0 / 32) * FRAG +
                      ((token % 32) + 32 * ((pair0 % 32) / 16)) * 16;
#pragma unroll
        for (int l = 0; l < PL_MAX; l++)
            *(uint4*)(dst + l * lstride) = make_uint4(plane_byte4(d[0], d[1], d[2], d[3], l),
                                                      plane_byte4(d[4], d[5], d[6], d[7], l),
                                                      plane_byte4(d[8], d[9], d[10], d[11], l),
                                                      plane_byte4(d[12], d[13], d[14], d[15], l));
        atomicMax(&s_need[tl / 32], need);
    }
    __syncthreads();
    const uint32_t chunk = rt0 * 16 / (32 * PLANE_KB);
    if (tid < NTT && tt0 + tid < TT && rt0 * 16 < K) atomicMax(&a.out_gemm_limbs[M + chunk * TT + tt0 + tid], s_need[tid]);
}

template <class G, int TTW, class Values>
__device__ __forceinline__ void park_and_store(const GemvArgs& a, int8_t* smem, uint32_t rt0, uint32_t tt0,
                                               Values&& block_values) {
    constexpr uint32_t NTOK = 64 * TTW, ROWS = G::RT * 32, STRIDE = NTOK + 1;
    static_assert(ROWS * STRIDE * 4 <= G::SMEM, "output block must fit the LDS");
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t wr = wave % (G::WAVES / 2), wt = wave / (G::WAVES / 2);
    const Q8View& w = a.w;
    const bool pairs = a.epilogue == EPI_SWIGLU || a.epilogue == EPI_GEGLU;
    const bool table = a.epilogue == EPI_SWIGLU && a.silu_tab != nullptr;
    int32_t* sC = (int32_t*)smem;
#pragma unroll
    for (int i = 0; i < G::RI; i++) {
        if (wave >= G::WAVES) break;  // a second k group's sums are in the first's
#pragma unroll
        for (int j = 0; j < TTW; j++) {
            const uint32_t tl = (wt * TTW + j) * 32 + (lane & 31);
            int32_t v[16];
            block_values(i, j, v);
            if (pairs && !table) {
                // Rows e and e + 1 (e even) are a gate/up pair in this lane:
                // the activation runs here, once per pair, every lane busy.
#pragma unroll
                for (int e = 0; e < 16; e += 2) {
                    const uint32_t rl = (wr * G::RI + i) * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
                    const int32_t act = a.epilogue == EPI_SWIGLU ? dn::silu(v[e]) : dn::gelu(v[e]);
                    sC[(rl >> 1) * STRIDE + tl] = dn::mul_sat(act, v[e + 1]);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 16; e++)
                    sC[((wr * G::RI + i) * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4)) * STRIDE + tl] = v[e];
            }
        }
    }
    __syncthreads();
    if (table) {
        // out[token][row / 2] = mul_sat(silu(gate), up) from the parked
        // [row][token] block, TB pairs per thread at a time: their table
        // loads (tab[gate], exact: dn::silu of every input that needs it)
        // are in flight together.
        constexpr uint32_t PAIRS = ROWS / 2 * NTOK, TB = 8;
        static_assert(PAIRS % (G::THREADS * TB) == 0, "whole batches");
        for (uint32_t c0 = tid; c0 < PAIRS; c0 += G::THREADS * TB) {
            int32_t gate[TB], up[TB], looked[TB];
#pragma unroll
            for (uint32_t u = 0; u < TB; u++) {
                const uint32_t c = c0 + u * G::THREADS, pl = c % (ROWS / 2), tl = c / (ROWS / 2);
                gate[u] = sC[2 * pl * STRIDE + tl];
                up[u] = sC[(2 * pl + 1) * STRIDE + tl];
            }
#pragma unroll
            for (uint32_t u = 0; u < TB; u++) looked[u] = a.silu_tab[dn::silu_tab_index(gate[u])];
#pragma unroll
            for (uint32_t u = 0; u < TB; u++) {
                const uint32_t c = c0 + u * G::THREADS, pl = c % (ROWS / 2), tl = c / (ROWS / 2);
                const uint32_t pair = rt0 * 16 + pl, token = tt0 * 32 + tl;
                const int32_t o = dn::mul_sat(dn::silu_from_tab(gate[u], looked[u]), up[u]);
                if (a.out && 2 * pair < w.rows && token < a.tokens) a.out[(size_t)token * a.out_stride + pair] = o;
                if (a.out_gemm_planes) sC[2 * pl * STRIDE + tl] = o;  // this thread's own slot, read above
            }
        }
    } else if (pairs) {
        // out[token][row / 2] for the block's ROWS / 2 pairs (none when the
        // gated rows are kept only as planes).
        for (uint32_t c = tid; a.out && c < ROWS / 2 * NTOK; c += G::THREADS) {
            const uint32_t pl = c % (ROWS / 2), tl = c / (ROWS / 2);
            const uint32_t pair = rt0 * 16 + pl, token = tt0 * 32 + tl;
            if (2 * pair < w.rows && token < a.tokens) a.out[(size_t)token * a.out_stride + pair] = sC[pl * STRIDE + tl];
        }
    } else {
        // One loop per epilogue (the choice is uniform), each reading only
        // what its epilogue uses.
        auto each = [&](auto&& f) __attribute__((always_inline)) {
            for (uint32_t c = tid; c < ROWS * NTOK; c += G::THREADS) {
                const uint32_t rl = c % ROWS, tl = c / ROWS;
                const uint32_t row = rt0 * 32 + rl, token = tt0 * 32 + tl;
                if (row < w.rows && token < a.tokens) f(row, token, sC[rl * STRIDE + tl], sC[(rl ^ 1) * STRIDE + tl]);
            }
        };
        if (a.epilogue == EPI_RESIDUAL) {
            each([&](uint32_t row, uint32_t token, int32_t v, int32_t) __attribute__((always_inline)) {
                a.out[(size_t)token * a.out_stride + row] =
                    dn::add_sat(v, a.residual[(size_t)token * a.residual_stride + row]);
            });
        } else if (a.epilogue == EPI_ROPE_KV) {
            each([&](uint32_t row, uint32_t token, int32_t v, int32_t partner) __attribute__((always_inline)) {
                store_output(a, row, token, v, partner);
            });
        } else {
            each([&](uint32_t row, uint32_t token, int32_t v, int32_t partner) __attribute__((always_inline)) {
                store_output_in(a, row, token, v, partner, EpiIn{0, 0, 0, 0});
            });
        }
    }
    __syncthreads();
    if (pairs && a.out_gemm_planes) gated_planes<G, NTOK>(a, sC, rt0, tt0, table ? 2 : 1);
}

// Row-scale matrices: the planes recombine into the row's integer dot
// product, then round_to_i32(tot * scale, 24) (q8.rs:94-104) through one
// 64-bit product where the operands' bit lengths show it cannot overflow
// (the usual case); if any lane of the wave has a larger product, the wave
// redoes the block with 128-bit ones.
template <class G, int LG, int TTW>
__device__ __forceinline__ void gemm_epilogue(const GemvArgs& a, int8_t* smem, uint32_t rt0, uint32_t tt0,
                                              const v16i (&acc)[2][TTW][LG]) {
    const uint32_t lane = threadIdx.x & 63, wr = (threadIdx.x >> 6) % (G::WAVES / 2);
    const Q8View& w = a.w;
    park_and_store<G, TTW>(a, smem, rt0, tt0, [&](int i, int j, int32_t (&v)[16]) __attribute__((always_inline)) {
        bool fits = true;
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const uint32_t row = rt0 * 32 + (wr * 2 + i) * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
            int64_t tot = 0;  // the row's integer dot product, |tot| < K * 2^38
#pragma unroll
            for (int l = 0; l < LG; l++) tot += (int64_t)acc[i][j][l][e] * ((int64_t)1 << (8 * l));
            const int64_t sc = row < w.rows ? w.row_scale[row] : 0;
            const uint64_t at = tot < 0 ? 0 - (uint64_t)tot : (uint64_t)tot;
            const uint64_t as = sc < 0 ? 0 - (uint64_t)sc : (uint64_t)sc;
            fits &= (128 - __clzll(at) - __clzll(as)) <= 63;  // |tot * sc| < 2^63
            v[e] = dn::clamp_i64_to_i32(dn::rshift_rte((int64_t)((uint64_t)tot * (uint64_t)sc), 24));
        }
        if (!__all(fits)) {
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const uint32_t row = rt0 * 32 + (wr * 2 + i) * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
                int64_t tot = 0;
#pragma unroll
                for (int l = 0; l < LG; l++) tot += (int64_t)acc[i][j][l][e] * ((int64_t)1 << (8 * l));
                v[e] = row < w.rows ? dn::round_to_i32((dn::i128)tot * (dn::i128)w.row_scale[row], 24) : 0;
            }
        }
    });
}

template <class G, int LG, int TTW, bool DEEP>
__device__ __forceinline__ void gemm_pass(const GemvArgs& a, int8_t* smem, uint32_t rt0, uint32_t tt0) {
    v16i acc[2][TTW][LG];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < TTW; j++)
#pragma unroll
            for (int l = 0; l < LG; l++) acc[i][j][l] = v16i{};
    gemm_mainloop<G, LG, TTW, DEEP>(a, smem, rt0, tt0, acc);
    if constexpr (G::SPLITS == 2) {
        // The second k group's sums into the first's, one row tile at a
        // time through LDS (TTW * LG * 16 KB each), lane-contiguous.
        const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63, hw = wave % G::WAVES;
        static_assert(G::WAVES * TTW * LG * 16 * 64 * 4 <= G::SMEM, "combine fits the LDS");
        int32_t* buf = (int32_t*)smem;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            if (wave >= G::WAVES) {
#pragma unroll
                for (int j = 0; j < TTW; j++)
#pragma unroll
                    for (int l = 0; l < LG; l++)
#pragma unroll
                        for (int e = 0; e < 16; e++)
                            buf[(((hw * TTW + j) * LG + l) * 16 + e) * 64 + lane] = acc[i][j][l][e];
            }
            lds_barrier();
            if (wave < G::WAVES) {
#pragma unroll
                for (int j = 0; j < TTW; j++)
#pragma unroll
                    for (int l = 0; l < LG; l++)
#pragma unroll
                        for (int e = 0; e < 16; e++)
                            acc[i][j][l][e] += buf[(((hw * TTW + j) * LG + l) * 16 + e) * 64 + lane];
            }
            lds_barrier();
        }
    }
    gemm_epilogue<G, LG, TTW>(a, smem, rt0, tt0, acc);
}

// 32W weight rows x 128 tokens per workgroup. Up to three digit planes (the
// usual case) are accumulated side by side in one pass; a block whose
// tokens need four or five takes two passes of 64 tokens. Workgroups are
// ordered so that each XCD (blocks are dealt to the 8 XCDs in turn) takes a
// contiguous range, walked in bands of 8 row groups with the token groups
// inside a band, so blocks in flight together share operands in their XCD's
// L2.
template <uint32_t W, uint32_t TG, uint32_t SPLIT = 1, bool DEEP = false>
__global__ __launch_bounds__(64 * W * SPLIT, 1) void q8_gemm_row_kernel(const GemvArgs a) {
    static_assert(TG == 2 || TG == 4, "64 or 128 tokens per workgroup");
    using G = GemmShape<W, SPLIT>;
    __shared__ __attribute__((aligned(1024))) int8_t smem[G::SMEM];
    int& s_limbs = *(int*)smem;  // read before the ring is first filled
    const uint32_t tid = threadIdx.x;
    const uint32_t TT = (a.tokens + 31) / 32;
    const uint32_t n_rg = (a.w.tiles + 2 * G::RT - 1) / (2 * G::RT), n_tg = (TT + TG - 1) / TG;
    const uint32_t total = n_rg * n_tg;
    uint32_t b = blockIdx.x;
    if (total % 8 == 0) b = (b % 8) * (total / 8) + b / 8;
    const uint32_t band = b / (GM_BAND * n_tg), first = band * GM_BAND, rows_in_band = min(GM_BAND, n_rg - first);
    const uint32_t r = b - band * GM_BAND * n_tg;
    const uint32_t rt0 = (first + r % rows_in_band) * G::RT, tt0 = (r / rows_in_band) * TG;

    const int limbs = tiles_limbs(a, tt0, TG, s_limbs);
    constexpr int TTW = TG / 2;  // token tiles per wave for up to three planes
    switch (limbs) {
        case 1: gemm_pass<G, 1, TTW, DEEP>(a, smem, rt0, tt0); break;
        case 2: gemm_pass<G, 2, TTW, DEEP>(a, smem, rt0, tt0); break;
        case 3: gemm_pass<G, 3, TTW, DEEP>(a, smem, rt0, tt0); break;
        case 4:
            gemm_pass<G, 4, 1, DEEP>(a, smem, rt0, tt0);
            if constexpr (TG == 4) gemm_pass<G, 4, 1, DEEP>(a, smem, rt0, tt0 + 2);
            break;
        default:
            gemm_pass<G, 5, 1, DEEP>(a, smem, rt0, tt0);
            if constexpr (TG == 4) gemm_pass<G, 5, 1, DEEP>(a, smem, rt0, tt0 + 2);
            break;
    }
}


// ---- per-block scales on the matrix cores ----
//
// A per-block scale matrix is first folded (iris_q8_prepare_fold): with
// s_b = sign_b * m_b * 2^sh_b the exact Q.24 value of block b's f16 scale
// (m_b the integer significand, under 2^11) and R the least sh_b of the
// row's non-zero scales, w' = q * sign_b * (m_b << (sh_b - R)) are integers,
// and dot_row's total sum_b s_b * sum_j q_j x_j equals 2^R * sum_k w'_k x_k
// (crates/det-num/src/q8.rs:56-72). Each w' is split into WP signed byte
// digits like the activations, so every (weight digit p, activation digit
// l) pair is an int8 GEMM with exact int32 sums, and pairs with the same
// p + l share an accumulator (at most five terms of |.| <= K * 2^14 each:
// 5 * 2^28 < 2^31 for K <= 16384). The epilogue recombines the shifts in 128
// bits, shifts by R and rounds once at 24 fraction bits.

// The signed byte digits of |v| < 2^47 (six bytes, d_l = byte l as int8,
// v = sum_l 256^l d_l) and how many of them v needs.
__device__ __forceinline__ uint64_t digits6(int64_t v) {
    return (uint64_t)(v + 0x808080808080LL) ^ 0x808080808080ULL;
}
__device__ __forceinline__ int digits6_needed(uint64_t d) {
    return (d >> 40) ? 6 : (d >> 32) ? 5 : (d >> 24) ? 4 : (d >> 16) ? 3 : (d >> 8) ? 2 : 1;
}

// Per row: R (the least exponent shift of its non-zero block scales; 0 for
// an all-zero row) into shift[row], and the digits its largest |w'| needs
// raised into *need (at most 6: sh_b - R <= 29, so |w'| < 2^47).
__global__ __launch_bounds__(256) void fold_rows_kernel(const uint8_t* qs, const uint16_t* sc16, uint32_t rows,
                                                        uint32_t nb, int32_t* shift, int* need) {
    const uint32_t row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    const uint32_t tile = row / Q8_TILE_ROWS, r = row % Q8_TILE_ROWS;
    const uint16_t* sc = sc16 + (size_t)tile * nb * Q8_TILE_ROWS + r;
    int least = 64;
    for (uint32_t b = 0; b < nb; b++) {
        const uint32_t bits = sc[(size_t)b * Q8_TILE_ROWS], e = (bits >> 10) & 0x1f, mant = bits & 0x3ff;
        if (e == 0 && mant == 0) continue;
        least = min(least, e ? (int)e - 1 : 0);
    }
    if (least == 64) least = 0;
    shift[row] = least;
    int digits = 1;
    const uint8_t* q = qs + (size_t)tile * nb * Q8_TILE_BLOCK_BYTES + r * 16;
    for (uint32_t b = 0; b < nb; b++) {
        const uint32_t bits = sc[(size_t)b * Q8_TILE_ROWS], e = (bits >> 10) & 0x1f, mant = bits & 0x3ff;
        const int64_t m = (int64_t)(e ? 1024 + mant : mant);
        if (m == 0) continue;
        const int d = (e ? (int)e - 1 : 0) - least;  // 0..29
        // The largest |q| of the block (both signs: digits are asymmetric).
        int qmax = 0, qmin = 0;
        const uint8_t* qb = q + (size_t)b * Q8_TILE_BLOCK_BYTES;
        for (int h = 0; h < 2; h++)
            for (int j = 0; j < 16; j++) {
                const int v = (int8_t)qb[h * 256 + j];
                qmax = max(qmax, v);
                qmin = min(qmin, v);
            }
        const int64_t f = (bits & 0x8000) ? -(m << d) : (m << d);
        for (int64_t wv : {f * qmax, f * qmin}) digits = max(digits, digits6_needed(digits6(wv)));
    }
    atomicMax(need, digits);
}

// One thread per (row, block): the block's w' as `nplanes` digit planes in
// the qs tile layout.
__global__ __launch_bounds__(256) void fold_planes_kernel(const uint8_t* qs, const uint16_t* sc16, uint32_t rows,
                                                          uint32_t nb, const int32_t* shift, uint32_t nplanes,
                                                          size_t plane_bytes, int8_t* planes) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)rows * nb) return;
    const uint32_t row = (uint32_t)(idx / nb), b = (uint32_t)(idx % nb);
    const uint32_t tile = row / Q8_TILE_ROWS, r = row % Q8_TILE_ROWS;
    const uint32_t bits = sc16[((size_t)tile * nb + b) * Q8_TILE_ROWS + r], e = (bits >> 10) & 0x1f,
                   mant = bits & 0x3ff;
    const int64_t m = (int64_t)(e ? 1024 + mant : mant);
    const int d = m ? (e ? (int)e - 1 : 0) - shift[row] : 0;
    const int64_t f = (bits & 0x8000) ? -(m << d) : (m << d);
    const size_t off = ((size_t)tile * nb + b) * Q8_TILE_BLOCK_BYTES + r * 16;
    for (int h = 0; h < 2; h++) {
        const uint4 qv = *(const uint4*)(qs + off + h * 256);
        const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w};
        uint32_t out[Q8_FOLD_MAX_PLANES][4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            uint64_t dg[4];
#pragma unroll
            for (int k = 0; k < 4; k++) dg[k] = digits6((int64_t)(int8_t)(qw[c] >> (8 * k)) * f);
#pragma unroll
            for (uint32_t p = 0; p < Q8_FOLD_MAX_PLANES; p++) out[p][c] = plane_byte4(dg[0], dg[1], dg[2], dg[3], p);
        }
        for (uint32_t p = 0; p < nplanes; p++)
            *(uint4*)(planes + p * plane_bytes + off + h * 256) = make_uint4(out[p][0], out[p][1], out[p][2], out[p][3]);
    }
}

// Workgroup shape of the folded product: four waves in a 2 x 2 grid over
// 128 weight rows and 64 tokens (one wave per SIMD: the shared-shift
// accumulators, 2 x (WP + LG - 1) blocks per wave, may need the
// accumulation registers); a stage is one 64-wide k step of WP weight
// planes and LG activation planes.
template <int WP, int LG>
struct FoldShape {
    // Two row tiles per wave up to three weight planes; one for four to six
    // (whose accumulators would not fit twice).
    static constexpr int RI = WP <= 3 ? 2 : 1;
    static constexpr uint32_t WAVES = 4, THREADS = 256, RT = 2 * RI;
    static constexpr uint32_t CHUNKS = 2 * RT * WP + 2 * LG * 2;
    static constexpr uint32_t PER_WAVE = (CHUNKS + WAVES - 1) / WAVES;
    static constexpr uint32_t STAGE = PER_WAVE * WAVES * FRAG;
    static constexpr uint32_t STAGES = 3 * STAGE <= 160 * 1024 ? 3 : 2;
    static constexpr uint32_t OUT = 32 * RT * 65 * 4;
    static constexpr uint32_t SMEM = STAGES * STAGE > OUT ? STAGES * STAGE : OUT;
    static constexpr int NS = WP + LG - 1;
};

template <class G, int WP, int LG>
__device__ __forceinline__ void fold_mainloop(const GemvArgs& a, int8_t* smem, uint32_t rt0, uint32_t tt0,
                                              v16i (&acc)[G::RI][G::NS]) {
    constexpr uint32_t TTWG = 2, RT = G::RT, CHUNKS = G::CHUNKS, PER_WAVE = G::PER_WAVE;
    constexpr uint32_t STAGES = G::STAGES, STAGE = G::STAGE;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t wr = wave % 2, wt = wave / 2;
    const Q8View& w = a.w;
    const uint32_t KS = w.cols / 64, KB = w.cols / 32, TT = (a.tokens + 31) / 32;
    const size_t lstride = (size_t)TT * KB * FRAG;
    const size_t pstride = (size_t)w.tiles * w.nb * Q8_TILE_BLOCK_BYTES;
    // Wave w copies chunks w, w + 4, ...: weight-plane operands (1 KB of the
    // tile layout per k step) first, then digit-plane operands (2 KB).
    const int8_t* src[PER_WAVE];
    uint32_t step[PER_WAVE];
#pragma unroll
    for (uint32_t i = 0; i < PER_WAVE; i++) {
        const uint32_t c0 = wave + G::WAVES * i, c = c0 < CHUNKS ? c0 : 0;
        if (c < 2 * RT * WP) {
            const uint32_t p = c / (2 * RT), cw = c % (2 * RT), rr = lane & 31, h = lane >> 5, sub = cw & 1;
            const uint32_t tile16 = min(2 * (rt0 + cw / 2) + rr / 16, w.tiles - 1);
            src[i] = w.fold_planes + p * pstride + ((size_t)tile16 * w.nb + sub) * Q8_TILE_BLOCK_BYTES + h * 256 +
                     (rr % 16) * 16;
            step[i] = FRAG;
        } else {
            const uint32_t b = c - 2 * RT * WP, sub = b & 1, rest = b >> 1, l = rest / TTWG;
            const uint32_t tile = min(tt0 + rest % TTWG, TT - 1);
            src[i] = a.planes + l * lstride + ((size_t)tile * KB + sub) * FRAG + lane * 16;
            step[i] = 2 * FRAG;
        }
    }
    const uint32_t ring = lds_offset(smem);
    auto issue = [&](uint32_t ks) {
        const uint32_t base = ring + (ks % STAGES) * STAGE;
#pragma unroll
        for (uint32_t i = 0; i < PER_WAVE; i++)
            copy_to_lds16(src[i] + (size_t)ks * step[i], base + (wave + G::WAVES * i) * FRAG);
    };
#pragma unroll
    for (uint32_t s = 0; s < STAGES - 1; s++)
        if (s < KS) issue(s);
    for (uint32_t ks = 0; ks < KS; ks++) {
        if (STAGES >= 3 && ks + 2 < KS) wait_vmem<(STAGES >= 3 ? 1 : 0) * PER_WAVE>();
        else wait_vmem<0>();
        lds_barrier();
        if (ks + STAGES - 1 < KS) issue(ks + STAGES - 1);
        const int8_t* st = smem + (ks % STAGES) * STAGE + lane * 16;
#pragma unroll
        for (uint32_t sub = 0; sub < 2; sub++) {
            v4i fa[G::RI][WP];
#pragma unroll
            for (int i = 0; i < G::RI; i++)
#pragma unroll
                for (int p = 0; p < WP; p++)
                    fa[i][p] = *(const v4i*)(st + (p * 2 * RT + 2 * (wr * G::RI + i) + sub) * FRAG);
#pragma unroll
            for (int l = 0; l < LG; l++) {
                const v4i fb = *(const v4i*)(st + (2 * RT * WP + 2 * (l * TTWG + wt) + sub) * FRAG);
#pragma unroll
                for (int i = 0; i < G::RI; i++)
#pragma unroll
                    for (int p = 0; p < WP; p++)
                        acc[i][p + l] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i][p], fb, acc[i][p + l], 0, 0, 0);
            }
        }
    }
    lds_barrier();
}

template <int WP, int LG>
__device__ __forceinline__ void fold_pass(const GemvArgs& a, int8_t* smem, uint32_t rt0, uint32_t tt0) {
    using G = FoldShape<WP, LG>;
    v16i acc[G::RI][G::NS];
#pragma unroll
    for (int i = 0; i < G::RI; i++)
#pragma unroll
        for (int s = 0; s < G::NS; s++) acc[i][s] = v16i{};
    fold_mainloop<G, WP, LG>(a, smem, rt0, tt0, acc);
    const uint32_t lane = threadIdx.x & 63, wr = (threadIdx.x >> 6) % 2;
    const Q8View& w = a.w;
    park_and_store<G, 1>(a, smem, rt0, tt0, [&](int i, int, int32_t (&v)[16]) __attribute__((always_inline)) {
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const uint32_t row = rt0 * 32 + (wr * G::RI + i) * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
            dn::i128 tot = 0;
#pragma unroll
            for (int s = 0; s < G::NS; s++) tot += (dn::i128)((dn::u128)(dn::i128)acc[i][s][e] << (8 * s));
            v[e] = row < w.rows ? dn::round_to_i32((dn::i128)((dn::u128)tot << w.fold_shift[row]), 24) : 0;
        }
    });
}

// 128 folded weight rows (64 for four to six planes) x 64 tokens per workgroup, blocks ordered as in
// q8_gemm_row_kernel (contiguous ranges per XCD, bands of 8 row groups).
template <int WP>
__global__ __launch_bounds__(256, 1) void q8_gemm_fold_kernel(const GemvArgs a) {
    __shared__ __attribute__((aligned(1024))) int8_t smem[FoldShape<WP, 5>::SMEM > FoldShape<WP, 3>::SMEM
                                                                ? FoldShape<WP, 5>::SMEM
                                                                : FoldShape<WP, 3>::SMEM];
    int& s_limbs = *(int*)smem;
    const uint32_t tid = threadIdx.x;
    const uint32_t TT = (a.tokens + 31) / 32;
    constexpr uint32_t RT = FoldShape<WP, 3>::RT, TG = 2;  // 32-row tiles, 32-token tiles per workgroup
    const uint32_t n_rg = (a.w.tiles + 2 * RT - 1) / (2 * RT), n_tg = (TT + TG - 1) / TG;
    const uint32_t total = n_rg * n_tg;
    uint32_t b = blockIdx.x;
    if (total % 8 == 0) b = (b % 8) * (total / 8) + b / 8;
    const uint32_t band = b / (GM_BAND * n_tg), first = band * GM_BAND, rows_in_band = min(GM_BAND, n_rg - first);
    const uint32_t r = b - band * GM_BAND * n_tg;
    const uint32_t rt0 = (first + r % rows_in_band) * RT, tt0 = (r / rows_in_band) * TG;
    const int limbs = tiles_limbs(a, tt0, TG, s_limbs);
    switch (limbs) {
        case 1: fold_pass<WP, 1>(a, smem, rt0, tt0); break;
        case 2: fold_pass<WP, 2>(a, smem, rt0, tt0); break;
        case 3: fold_pass<WP, 3>(a, smem, rt0, tt0); break;
        case 4: fold_pass<WP, 4>(a, smem, rt0, tt0); break;
        default: fold_pass<WP, 5>(a, smem, rt0, tt0); break;
    }
}

}  // namespace

bool iris_gemm_applies(const GemvArgs& a) {
    if (!a.planes || !a.token_limbs || a.tokens < 2 || a.w.cols % 64 || a.epilogue == EPI_HEAD_SELECT ||
        a.prologue == PRO_NORM_RES_NORM)
        return false;
    if (a.w.scale_mode == Q8_SCALE_ROW) return a.w.cols < (1u << 17);
    // Folded per-block scales: shared-shift sums stay below 2^31.
    return a.w.scale_mode == Q8_SCALE_F16 && a.w.fold_planes && a.w.fold_nplanes >= 1 &&
           a.w.fold_nplanes <= Q8_FOLD_MAX_PLANES && a.w.cols <= 16384;
}

int iris_gemm_launch(const GemvArgs& a, hipStream_t stream) {
    if (!iris_gemm_applies(a) || a.x_stride % 4 || ((uintptr_t)a.x & 15) || ((uintptr_t)a.planes & 255))
        return IRIS_E_INVALID;
    if (a.prologue == PRO_RMSNORM && ((uintptr_t)a.norm_w & 15)) return IRIS_E_INVALID;
    if (a.planes_ready && a.prologue != PRO_NONE) return IRIS_E_INVALID;
    const bool gated = a.epilogue == EPI_SWIGLU || a.epilogue == EPI_GEGLU;
    if (a.out_gemm_planes && (!gated || !a.out_gemm_limbs || (a.w.rows / 2) % 32 || ((uintptr_t)a.out_gemm_planes & 255) ||
                              a.out_gemm_planes == a.planes || a.out_gemm_limbs == a.token_limbs))
        return IRIS_E_INVALID;
    if (!a.out && !a.out_gemm_planes) return IRIS_E_INVALID;
    const uint32_t TT = (a.tokens + 31) / 32, KB = a.w.cols / 32;
    if (!a.planes_ready) {
        if (a.prologue == PRO_RMSNORM)
            hipLaunchKernelGGL(token_prep_kernel, dim3((a.tokens + 3) / 4), dim3(256), 0, stream, a);
        hipLaunchKernelGGL(digit_planes_kernel, dim3(TT, (KB + PLANE_KB - 1) / PLANE_KB), dim3(256), 0, stream, a);
    }
    if (a.out_gemm_planes) {
        // The gated rows' counts start at 1 (every workgroup raises its own).
        const uint32_t n = (uint32_t)(gemm_limb_ints(a.w.rows / 2, a.tokens) - a.tokens);
        hipLaunchKernelGGL(fill_ints_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, a.out_gemm_limbs + a.tokens, n, 1);
    }
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return (int)st;
    if (a.w.scale_mode == Q8_SCALE_F16) {
        // 32-row tiles per workgroup: 4, or 2 for four to six planes (FoldShape::RT).
        const uint32_t rt = a.w.fold_nplanes <= 3 ? 4 : 2;
        const uint32_t n = (a.w.tiles + 2 * rt - 1) / (2 * rt) * ((TT + 1) / 2);
        switch (a.w.fold_nplanes) {
            case 1: hipLaunchKernelGGL(q8_gemm_fold_kernel<1>, dim3(n), dim3(256), 0, stream, a); break;
            case 2: hipLaunchKernelGGL(q8_gemm_fold_kernel<2>, dim3(n), dim3(256), 0, stream, a); break;
            case 3: hipLaunchKernelGGL(q8_gemm_fold_kernel<3>, dim3(n), dim3(256), 0, stream, a); break;
            case 4: hipLaunchKernelGGL(q8_gemm_fold_kernel<4>, dim3(n), dim3(256), 0, stream, a); break;
            case 5: hipLaunchKernelGGL(q8_gemm_fold_kernel<5>, dim3(n), dim3(256), 0, stream, a); break;
            default: hipLaunchKernelGGL(q8_gemm_fold_kernel<6>, dim3(n), dim3(256), 0, stream, a); break;
        }
        return (int)hipGetLastError();
    }
    // Two waves per SIMD and 256 rows x 128 tokens when that still gives
    // every CU a workgroup in at most half the rounds of the 128-row shape
    // (whose workgroups do half the work: q/k/v at 2048 tokens, 384 of the
    // larger against 768 of the smaller, 2048-row pass 69.35 -> 69.17 ms),
    // else one wave per SIMD and 128 rows, with 64
    // tokens when the rounds of workgroups that gives cost less: a 64-token
    // workgroup takes about 2/3 of a 128-token one's time (M=512, K=N=4096:
    // 256 of them 60.6 us, 128 of the larger 92.1 us).
    const uint32_t n_tg = (TT + GM_TT - 1) / GM_TT, n_tg2 = (TT + 1) / 2;
    const uint32_t cus = (uint32_t)iris_device_cus();
    const uint32_t n8 = (a.w.tiles + 15) / 16 * n_tg, n4 = (a.w.tiles + 7) / 8 * n_tg;
    const uint32_t n42 = (a.w.tiles + 7) / 8 * n_tg2;
    const uint32_t rounds8 = (n8 + cus - 1) / cus, rounds4 = (n4 + cus - 1) / cus, rounds2 = (n42 + cus - 1) / cus;
    // The four-wave shapes split the k steps between two wave groups when
    // there is an even number of them (both groups' barriers pair up).
    const bool split = (a.w.cols / 64) % 2 == 0;
    // Deeper rings for long rows (at least 64 k steps per wave group).
    const bool deep = a.w.cols >= 8192;
    if (n8 >= cus && (2 * rounds8 <= rounds4 || !split))
        hipLaunchKernelGGL((q8_gemm_row_kernel<8, 4>), dim3(n8), dim3(512), 0, stream, a);
    else if (n42 != n4 && 2 * rounds2 <= 3 * rounds4) {
        if (split && deep) hipLaunchKernelGGL((q8_gemm_row_kernel<4, 2, 2, true>), dim3(n42), dim3(512), 0, stream, a);
        else if (split) hipLaunchKernelGGL((q8_gemm_row_kernel<4, 2, 2>), dim3(n42), dim3(512), 0, stream, a);
        else hipLaunchKernelGGL((q8_gemm_row_kernel<4, 2>), dim3(n42), dim3(256), 0, stream, a);
    } else {
        if (split && deep) hipLaunchKernelGGL((q8_gemm_row_kernel<4, 4, 2, true>), dim3(n4), dim3(512), 0, stream, a);
        else if (split) hipLaunchKernelGGL((q8_gemm_row_kernel<4, 4, 2>), dim3(n4), dim3(512), 0, stream, a);
        else hipLaunchKernelGGL((q8_gemm_row_kernel<4, 4>), dim3(n4), dim3(256), 0, stream, a);
    }
    return (int)hipGetLastError();
}

int iris_q8_prepare_fold(Q8GpuMatrix* m, hipStream_t stream) {
    static std::mutex lock;  // a matrix is folded once, whichever thread gets there first
    std::lock_guard<std::mutex> guard(lock);
    if (!m || m->fold_tried || m->scale_mode != Q8_SCALE_F16 || !m->sc16 || m->cols % 64) return 0;
    m->fold_tried = true;
    const size_t plane_bytes = (size_t)m->tiles * m->nb * Q8_TILE_BLOCK_BYTES;
    int* d_need = nullptr;
    int need = 0;
    hipError_t st = hipMalloc((void**)&m->fold.shift, (size_t)m->tiles * Q8_TILE_ROWS * sizeof(int32_t));
    if (st == hipSuccess) st = hipMalloc((void**)&d_need, sizeof(int));
    if (st == hipSuccess) st = hipMemsetAsync(m->fold.shift, 0, (size_t)m->tiles * Q8_TILE_ROWS * sizeof(int32_t), stream);
    if (st == hipSuccess) st = hipMemsetAsync(d_need, 0, sizeof(int), stream);
    if (st == hipSuccess) {
        hipLaunchKernelGGL(fold_rows_kernel, dim3((m->rows + 255) / 256), dim3(256), 0, stream, m->qs, m->sc16, m->rows,
                           m->nb, m->fold.shift, d_need);
        st = hipGetLastError();
    }
    if (st == hipSuccess) st = hipMemcpyAsync(&need, d_need, sizeof(int), hipMemcpyDeviceToHost, stream);
    if (st == hipSuccess) st = hipStreamSynchronize(stream);
    hipFree(d_need);
    if (st == hipSuccess && need >= 1 && need <= (int)Q8_FOLD_MAX_PLANES) {
        // Rows past the matrix in its last tile keep zero weights in every plane.
        st = hipMalloc((void**)&m->fold.planes, plane_bytes * need);
        if (st == hipSuccess) st = hipMemsetAsync(m->fold.planes, 0, plane_bytes * need, stream);
        const size_t n = (size_t)m->rows * m->nb;
        if (st == hipSuccess && n) {
            hipLaunchKernelGGL(fold_planes_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, m->qs,
                               m->sc16, m->rows, m->nb, m->fold.shift, (uint32_t)need, plane_bytes, m->fold.planes);
            st = hipGetLastError();
        }
        if (st == hipSuccess) st = hipStreamSynchronize(stream);
        if (st == hipSuccess) {
            m->fold.nplanes = (uint32_t)need;
            m->device_bytes += plane_bytes * need + (size_t)m->tiles * Q8_TILE_ROWS * sizeof(int32_t);
            return 0;
        }
    }
    hipFree(m->fold.planes);
    hipFree(m->fold.shift);
    m->fold = Q8Folded{};
    return (int)st;
}
