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
// (|sum| <= K * 2^14 < 2^31 for K < 2^17) on v_mfma_i32_16x16x64_i8.
//
// Operand layout. One 16x16x64 MFMA takes, in lane l, 16 bytes of row (or
// token) l % 16 at k-offset 16 * (l / 16). Two consecutive 512-byte
// tile-blocks of a 16-row weight tile ([half][16 rows][16 bytes] each) are
// exactly that 1 KB A operand, so the weights need no second layout; the
// digit planes are written in the same shape: plane l, 16-token tile tt and
// 64-wide k-step ks form one 1 KB block at ((l * TT + tt) * KS + ks) * 1024.
// Every operand the kernel stages is then one contiguous kilobyte, copied
// from global memory straight into LDS (global_load_lds_dwordx4, no
// registers in between) through a four-deep ring, and read back by each lane
// as one conflict-free 16-byte LDS load.
#include "detnum_dev.h"
#include "q8_epilogue.h"
#include "q8_internal.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int PL_MAX = 5;                   // digit planes of an i32
constexpr uint32_t GM_RT = 8;               // 16-row weight tiles per workgroup (128 rows)
constexpr uint32_t GM_TT = 8;               // 16-token tiles per workgroup (128 tokens)
constexpr uint32_t GM_THREADS = 256;        // 4 waves: 2 (row halves) x 2 (token halves)
constexpr uint32_t GM_STAGES = 4;           // ring depth: three k-steps in flight
constexpr uint32_t FRAG = 1024;             // bytes of one 16 x 64 operand
constexpr uint32_t GM_STAGE = 32 * FRAG;    // 8 weight + up to 24 digit-plane operands
constexpr uint32_t GM_BAND = 8;             // row groups per band of the launch order

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

// The digit planes of one 16-token tile per workgroup, after the optional
// rms_norm (ops.rs:98-114: mul_sat(mul_sat(v, scale), w)), in the operand
// layout above, and the digits each token needs. Tokens past the end of the
// last tile get zero digits.
__global__ __launch_bounds__(256) void digit_planes_kernel(const GemvArgs a) {
    __shared__ int32_t s_scale[16];
    __shared__ int s_need[16];
    const uint32_t tt = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t K = a.w.cols, M = a.tokens, TT = (M + 15) / 16, KS = K / 64;
    const bool norm = a.prologue == PRO_RMSNORM;
    if (tid < 16) s_need[tid] = 1;
    if (norm) {
        // Wave w sums the squares of tokens 4w..4w+3 of the tile (the sum of
        // non-negative terms saturates the same way in any order).
        for (uint32_t i = 0; i < 4; i++) {
            const uint32_t t = tt * 16 + wave * 4 + i;
            int64_t s = 0;
            if (t < M) {
                const int32_t* x = a.x + (size_t)t * a.x_stride;
                for (uint32_t k = lane * 4; k < K; k += 256) {
                    const int4 v = *(const int4*)(x + k);
                    s = dn::acc_add_sat(s, (int64_t)v.x * v.x);
                    s = dn::acc_add_sat(s, (int64_t)v.y * v.y);
                    s = dn::acc_add_sat(s, (int64_t)v.z * v.z);
                    s = dn::acc_add_sat(s, (int64_t)v.w * v.w);
                }
            }
            for (int off = 32; off >= 1; off >>= 1) s = dn::acc_add_sat(s, __shfl_xor(s, off));
            if (lane == 0) s_scale[wave * 4 + i] = t < M ? dn::rms_scale_from_sum(s, K, a.norm_eps) : 0;
        }
    }
    __syncthreads();
    // Lane l writes the 16 bytes of token l % 16 at k-offset 16 * (l / 16)
    // of each k-step the wave takes.
    const uint32_t tl = lane & 15, q = lane >> 4, t = tt * 16 + tl;
    const bool valid = t < M;
    const int32_t scale = norm ? s_scale[tl] : 0;
    const int32_t* x = a.x + (size_t)(valid ? t : 0) * a.x_stride;
    const size_t lstride = (size_t)TT * KS * FRAG;
    int need = 1;
    for (uint32_t ks = wave; ks < KS; ks += 4) {
        const uint32_t k0 = ks * 64 + q * 16;
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
        int8_t* dst = a.planes + ((size_t)tt * KS + ks) * FRAG + lane * 16;
#pragma unroll
        for (int l = 0; l < PL_MAX; l++)
            *(uint4*)(dst + l * lstride) = make_uint4(out[l][0], out[l][1], out[l][2], out[l][3]);
    }
    need = max(need, __shfl_xor(need, 16));
    need = max(need, __shfl_xor(need, 32));
    if (lane < 16) atomicMax(&s_need[lane], need);
    __syncthreads();
    if (tid < 16 && tt * 16 + tid < M) a.token_limbs[tt * 16 + tid] = s_need[tid];
}

template <int N>
__device__ __forceinline__ void wait_vmem() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// All of this wave's LDS reads have returned, then every wave meets.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// One pass of the workgroup over the whole k range: 8 weight tiles (rows
// rt0*16 ..) times 2*TTW token tiles (from tt0) times LG digit planes. Wave
// (wr, wt) accumulates weight tiles wr*4..wr*4+3 against token tiles
// wt*TTW..: acc[i][j][l] is the int32 sum of plane l for its 16 x 16 block.
// Operands past the last tile are clamped onto it (read, never stored).
template <int LG, int TTW>
__device__ __forceinline__ void gemm_mainloop(const GemvArgs& a, int8_t* smem, uint32_t rt0, uint32_t tt0,
                                              v4i (&acc)[4][TTW][LG]) {
    constexpr uint32_t TTWG = 2 * TTW;             // token tiles per pass
    constexpr uint32_t CHUNKS = GM_RT + LG * TTWG; // 1 KB operands per stage
    constexpr uint32_t PER_WAVE = CHUNKS / 4;
    static_assert(CHUNKS % 4 == 0 && CHUNKS * FRAG <= GM_STAGE, "stage layout");
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wr = wave & 1, wt = wave >> 1;
    const Q8View& w = a.w;
    const uint32_t KS = w.cols / 64, TT = (a.tokens + 15) / 16;
    const size_t lstride = (size_t)TT * KS * FRAG;

    // Operand c of a stage: c < 8 is weight tile rt0 + c, then plane l, token
    // tile j at 8 + l * TTWG + j. Wave w copies operands w, w + 4, ...
    const int8_t* src[PER_WAVE];
#pragma unroll
    for (uint32_t i = 0; i < PER_WAVE; i++) {
        const uint32_t c = wave + 4 * i;
        if (c < GM_RT) {
            const uint32_t tile = min(rt0 + c, w.tiles - 1);
            src[i] = (const int8_t*)w.qs + (size_t)tile * w.nb * Q8_TILE_BLOCK_BYTES + lane * 16;
        } else {
            const uint32_t b = c - GM_RT, l = b / TTWG, tile = min(tt0 + b % TTWG, TT - 1);
            src[i] = a.planes + l * lstride + (size_t)tile * KS * FRAG + lane * 16;
        }
    }
    auto issue = [&](uint32_t ks) {
        int8_t* base = smem + (ks % GM_STAGES) * GM_STAGE;
#pragma unroll
        for (uint32_t i = 0; i < PER_WAVE; i++)
            __builtin_amdgcn_global_load_lds(src[i] + (size_t)ks * FRAG,
                                             (__attribute__((address_space(3))) void*)(base + (wave + 4 * i) * FRAG),
                                             16, 0, 0);
    };

#pragma unroll
    for (uint32_t s = 0; s < GM_STAGES - 1; s++)
        if (s < KS) issue(s);
    for (uint32_t ks = 0; ks < KS; ks++) {
        // This wave's copies for step ks are in LDS once at most the later
        // steps' copies are outstanding; the barrier makes every wave's
        // visible and frees the slot the next copy overwrites (read at ks-1).
        if (ks + 2 < KS) wait_vmem<2 * PER_WAVE>();
        else if (ks + 1 < KS) wait_vmem<PER_WAVE>();
        else wait_vmem<0>();
        lds_barrier();
        if (ks + GM_STAGES - 1 < KS) issue(ks + GM_STAGES - 1);
        const int8_t* sA = smem + (ks % GM_STAGES) * GM_STAGE;
        const int8_t* sB = sA + GM_RT * FRAG;
        v4i fa[4];
#pragma unroll
        for (int i = 0; i < 4; i++) fa[i] = *(const v4i*)(sA + (wr * 4 + i) * FRAG + lane * 16);
#pragma unroll
        for (int l = 0; l < LG; l++) {
            v4i fb[TTW];
#pragma unroll
            for (int j = 0; j < TTW; j++) fb[j] = *(const v4i*)(sB + (l * TTWG + wt * TTW + j) * FRAG + lane * 16);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < TTW; j++)
                    acc[i][j][l] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j][l], 0, 0, 0);
        }
    }
    lds_barrier();  // every wave is done with the ring before it is reused
}

// Lane l holds rows 4 * (l / 16) + e of each weight tile for token l % 16 of
// each token tile: recombine the planes, scale, round once, park the block
// in LDS as [row][token], then run the epilogue row-fastest.
template <int LG, int TTW>
__device__ __forceinline__ void gemm_epilogue(const GemvArgs& a, int8_t* smem, uint32_t rt0, uint32_t tt0,
                                              const v4i (&acc)[4][TTW][LG]) {
    constexpr uint32_t NTOK = 32 * TTW, ROWS = GM_RT * 16, STRIDE = NTOK + 1;
    static_assert(ROWS * STRIDE * 4 <= GM_STAGES * GM_STAGE, "output block must fit the ring");
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wr = wave & 1, wt = wave >> 1;
    const Q8View& w = a.w;
    int32_t* sC = (int32_t*)smem;
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int j = 0; j < TTW; j++) {
            const uint32_t tl = (wt * TTW + j) * 16 + (lane % 16);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t rl = (wr * 4 + i) * 16 + (lane / 16) * 4 + e, row = rt0 * 16 + rl;
                int64_t tot = 0;  // the row's integer dot product, |tot| < K * 2^38
#pragma unroll
                for (int l = 0; l < LG; l++) tot += (int64_t)acc[i][j][l][e] * ((int64_t)1 << (8 * l));
                sC[rl * STRIDE + tl] =
                    row < w.rows ? dn::round_to_i32((dn::i128)tot * (dn::i128)w.row_scale[row], 24) : 0;
            }
        }
    }
    __syncthreads();
    for (uint32_t c = tid; c < ROWS * NTOK; c += GM_THREADS) {
        const uint32_t rl = c % ROWS, tl = c / ROWS;
        const uint32_t row = rt0 * 16 + rl, token = tt0 * 16 + tl;
        if (row < w.rows && token < a.tokens)
            store_output(a, row, token, sC[rl * STRIDE + tl], sC[(rl ^ 1) * STRIDE + tl]);
    }
    __syncthreads();
}

template <int LG, int TTW>
__device__ __forceinline__ void gemm_pass(const GemvArgs& a, int8_t* smem, uint32_t rt0, uint32_t tt0) {
    v4i acc[4][TTW][LG];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < TTW; j++)
#pragma unroll
            for (int l = 0; l < LG; l++) acc[i][j][l] = v4i{0, 0, 0, 0};
    gemm_mainloop<LG, TTW>(a, smem, rt0, tt0, acc);
    gemm_epilogue<LG, TTW>(a, smem, rt0, tt0, acc);
}

// 128 weight rows x 128 tokens per workgroup, one wave per SIMD. Up to three
// digit planes (the usual case) are accumulated side by side in one pass;
// a block whose tokens need four or five takes two passes of 64 tokens.
// Workgroups are ordered so that each XCD (blocks are dealt to the 8 XCDs
// in turn) takes a contiguous range, walked in bands of 8 row groups with
// the token groups inside a band, so blocks in flight together share
// operands in their XCD's L2.
__global__ __launch_bounds__(GM_THREADS, 1) void q8_gemm_row_kernel(const GemvArgs a) {
    __shared__ __attribute__((aligned(1024))) int8_t smem[GM_STAGES * GM_STAGE];
    __shared__ int s_limbs;
    const uint32_t tid = threadIdx.x;
    const uint32_t TT = (a.tokens + 15) / 16;
    const uint32_t n_rg = (a.w.tiles + GM_RT - 1) / GM_RT, n_tg = (TT + GM_TT - 1) / GM_TT, total = n_rg * n_tg;
    uint32_t b = blockIdx.x;
    if (total % 8 == 0) b = (b % 8) * (total / 8) + b / 8;
    const uint32_t band = b / (GM_BAND * n_tg), first = band * GM_BAND, rows_in_band = min(GM_BAND, n_rg - first);
    const uint32_t r = b - band * GM_BAND * n_tg;
    const uint32_t rt0 = (first + r % rows_in_band) * GM_RT, tt0 = (r / rows_in_band) * GM_TT;

    if (tid == 0) s_limbs = 1;
    __syncthreads();
    if (tid < GM_TT * 16 && tt0 * 16 + tid < a.tokens) atomicMax(&s_limbs, a.token_limbs[tt0 * 16 + tid]);
    __syncthreads();
    switch (s_limbs) {
        case 1: gemm_pass<1, 4>(a, smem, rt0, tt0); break;
        case 2: gemm_pass<2, 4>(a, smem, rt0, tt0); break;
        case 3: gemm_pass<3, 4>(a, smem, rt0, tt0); break;
        case 4:
            gemm_pass<4, 2>(a, smem, rt0, tt0);
            gemm_pass<4, 2>(a, smem, rt0, tt0 + 4);
            break;
        default:
            gemm_pass<5, 2>(a, smem, rt0, tt0);
            gemm_pass<5, 2>(a, smem, rt0, tt0 + 4);
            break;
    }
}

}  // namespace

bool iris_gemm_applies(const GemvArgs& a) {
    return a.planes && a.token_limbs && a.tokens >= 2 && a.w.scale_mode == Q8_SCALE_ROW && a.w.cols % 64 == 0 &&
           a.w.cols < (1u << 17) && a.epilogue != EPI_HEAD_SELECT;
}

int iris_gemm_launch(const GemvArgs& a, hipStream_t stream) {
    if (!iris_gemm_applies(a) || a.x_stride % 4 || ((uintptr_t)a.x & 15) || ((uintptr_t)a.planes & 255))
        return IRIS_E_INVALID;
    if (a.prologue == PRO_RMSNORM && ((uintptr_t)a.norm_w & 15)) return IRIS_E_INVALID;
    const uint32_t TT = (a.tokens + 15) / 16;
    hipLaunchKernelGGL(digit_planes_kernel, dim3(TT), dim3(256), 0, stream, a);
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return (int)st;
    const uint32_t n_rg = (a.w.tiles + GM_RT - 1) / GM_RT, n_tg = (TT + GM_TT - 1) / GM_TT;
    hipLaunchKernelGGL(q8_gemm_row_kernel, dim3(n_rg * n_tg), dim3(GM_THREADS), 0, stream, a);
    return (int)hipGetLastError();
}
