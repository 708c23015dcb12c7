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
// The weights need no second layout: two consecutive 512-byte tile-blocks
// of a 16-row tile ([half][16 rows][16 bytes] each) are, byte for byte, the
// 64-lane A operand of one 16x16x64 MFMA (lane l: row l % 16, 16 bytes of
// the k-group l / 16). The B operand takes the same k-group's 16 digits of
// token l % 16 from the planes.
#include "detnum_dev.h"
#include "q8_epilogue.h"
#include "q8_internal.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int PL_MAX = 5;                 // digit planes of an i32
constexpr uint32_t GM_TILES = 8;          // 16-row weight tiles per workgroup (128 rows)
constexpr uint32_t GM_TOK = 64;           // tokens per workgroup
constexpr uint32_t GM_K = 64;             // k per step: two Q8_0 blocks
constexpr uint32_t GM_THREADS = 256;      // 4 waves: 2 (rows) x 2 (tokens)
constexpr uint32_t B_ROW = GM_K + 16;     // LDS bytes per token row of a plane (padded: no bank conflicts)

__device__ __forceinline__ uint64_t digits5(int32_t v) {
    return (uint64_t)((int64_t)v + 0x8080808080LL) ^ 0x8080808080ULL;
}

__device__ __forceinline__ int limbs_needed(uint64_t d) {
    return (d >> 32) ? 5 : (d >> 24) ? 4 : (d >> 16) ? 3 : (d >> 8) ? 2 : 1;
}

// The digit planes of one token per workgroup (after the optional rms_norm,
// ops.rs:98-114: mul_sat(mul_sat(v, scale), w)), planes[l][t][k], and the
// digits the token needs.
__global__ __launch_bounds__(256) void digit_planes_kernel(const GemvArgs a) {
    __shared__ int64_t s_red[4];
    __shared__ int32_t s_scale;
    __shared__ int s_need;
    const uint32_t t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t K = a.w.cols;
    const int32_t* x = a.x + (size_t)t * a.x_stride;
    const bool norm = a.prologue == PRO_RMSNORM;
    if (tid == 0) s_need = 1;
    int32_t scale = 0;
    if (norm) {
        int64_t s = 0;
        for (uint32_t k = tid * 4; k < K; k += 1024) {
            const int4 v = *(const int4*)(x + k);
            s = dn::acc_add_sat(s, (int64_t)v.x * v.x);
            s = dn::acc_add_sat(s, (int64_t)v.y * v.y);
            s = dn::acc_add_sat(s, (int64_t)v.z * v.z);
            s = dn::acc_add_sat(s, (int64_t)v.w * v.w);
        }
        for (int off = 32; off >= 1; off >>= 1) s = dn::acc_add_sat(s, __shfl_xor(s, off));
        if (lane == 0) s_red[wave] = s;
        __syncthreads();
        if (tid == 0) {
            int64_t tot = 0;
            for (int i = 0; i < 4; i++) tot = dn::acc_add_sat(tot, s_red[i]);
            s_scale = dn::rms_scale_from_sum(tot, K, a.norm_eps);
        }
    }
    __syncthreads();
    if (norm) scale = s_scale;
    const size_t ps = (size_t)a.tokens * K;
    int8_t* p0 = a.planes + (size_t)t * K;
    int need = 1;
    for (uint32_t k = tid * 4; k < K; k += 1024) {
        int4 v = *(const int4*)(x + k);
        if (norm) {
            const int4 nw = *(const int4*)(a.norm_w + k);
            v.x = dn::mul_sat(dn::mul_sat(v.x, scale), nw.x);
            v.y = dn::mul_sat(dn::mul_sat(v.y, scale), nw.y);
            v.z = dn::mul_sat(dn::mul_sat(v.z, scale), nw.z);
            v.w = dn::mul_sat(dn::mul_sat(v.w, scale), nw.w);
        }
        const uint64_t d0 = digits5(v.x), d1 = digits5(v.y), d2 = digits5(v.z), d3 = digits5(v.w);
        need = max(need, max(max(limbs_needed(d0), limbs_needed(d1)), max(limbs_needed(d2), limbs_needed(d3))));
#pragma unroll
        for (int l = 0; l < PL_MAX; l++) {
            const int sh = 8 * l;
            *(uint32_t*)(p0 + (size_t)l * ps + k) = (uint32_t)((d0 >> sh) & 0xff) | ((uint32_t)((d1 >> sh) & 0xff) << 8) |
                                                    ((uint32_t)((d2 >> sh) & 0xff) << 16) |
                                                    ((uint32_t)((d3 >> sh) & 0xff) << 24);
        }
    }
    for (int off = 32; off >= 1; off >>= 1) need = max(need, __shfl_xor(need, off));
    if (lane == 0) atomicMax(&s_need, need);
    __syncthreads();
    if (tid == 0) a.token_limbs[t] = s_need;
}

// 128 weight rows x 64 tokens per workgroup; wave (wr, wt) owns 4 tiles x 32
// tokens, one int32 accumulator set per digit plane. Planes past the most
// any of the workgroup's tokens needs are zero and skipped.
__global__ __launch_bounds__(GM_THREADS) void q8_gemm_row_kernel(const GemvArgs a) {
    // Staging for the k loop (weights, then digit planes); afterwards the
    // finished tile of 128 x 64 outputs.
    constexpr uint32_t SMEM = GM_TILES * 1024 + PL_MAX * GM_TOK * B_ROW;
    static_assert(SMEM >= GM_TILES * Q8_TILE_ROWS * GM_TOK * 4, "output tile must fit the staging space");
    __shared__ __attribute__((aligned(16))) int8_t smem[SMEM];
    int8_t* sA = smem;
    int8_t* sB = smem + GM_TILES * 1024;
    __shared__ int s_limbs;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t tok0 = blockIdx.x * GM_TOK, tile0 = blockIdx.y * GM_TILES;
    const Q8View& w = a.w;
    const uint32_t K = w.cols, M = a.tokens;
    if (tid == 0) s_limbs = 1;
    __syncthreads();
    if (tid < GM_TOK && tok0 + tid < M) atomicMax(&s_limbs, a.token_limbs[tok0 + tid]);
    __syncthreads();
    const int L = s_limbs;
    const size_t ps = (size_t)M * K;
    const uint32_t wr = wave & 1, wt = wave >> 1;

    v4i acc[4][2][PL_MAX];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int l = 0; l < PL_MAX; l++) acc[i][j][l] = v4i{0, 0, 0, 0};

    for (uint32_t k0 = 0; k0 < K; k0 += GM_K) {
        // Stage the step's weights (8 tiles x 1 KB, copied as they lie) and
        // the digit planes it needs (64 tokens x 64 bytes each).
        for (uint32_t c = tid; c < GM_TILES * 64; c += GM_THREADS) {
            const uint32_t rt = c / 64, off = (c % 64) * 16, tile = tile0 + rt;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (tile < w.tiles) v = *(const uint4*)(w.qs + ((size_t)tile * w.nb + k0 / 32) * Q8_TILE_BLOCK_BYTES + off);
            *(uint4*)(sA + rt * 1024 + off) = v;
        }
        for (uint32_t c = tid; c < (uint32_t)L * GM_TOK * 4; c += GM_THREADS) {
            const uint32_t l = c / (GM_TOK * 4), rem = c % (GM_TOK * 4), tk = rem / 4, q = rem % 4;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (tok0 + tk < M) v = *(const uint4*)(a.planes + l * ps + (size_t)(tok0 + tk) * K + k0 + q * 16);
            *(uint4*)(sB + (l * GM_TOK + tk) * B_ROW + q * 16) = v;
        }
        __syncthreads();
        v4i fa[4];
#pragma unroll
        for (int i = 0; i < 4; i++) fa[i] = *(const v4i*)(sA + (wr * 4 + i) * 1024 + lane * 16);
#pragma unroll
        for (int l = 0; l < PL_MAX; l++) {
            if (l < L) {
                v4i fb[2];
#pragma unroll
                for (int j = 0; j < 2; j++)
                    fb[j] = *(const v4i*)(sB + (l * GM_TOK + wt * 32 + j * 16 + (lane % 16)) * B_ROW + (lane / 16) * 16);
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        acc[i][j][l] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j][l], 0, 0, 0);
            }
        }
        __syncthreads();
    }

    // Lane l holds rows 4 * (l / 16) + e of each tile for token l % 16 of
    // each token group: recombine the planes, scale, round once, and park
    // the tile in LDS as [row][token]; then the epilogue runs row-fastest.
    int32_t* sC = (int32_t*)smem;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t rt = wr * 4 + i, tile = tile0 + rt;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t tl = wt * 32 + j * 16 + (lane % 16);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t rl = rt * Q8_TILE_ROWS + (lane / 16) * 4 + e, row = tile0 * Q8_TILE_ROWS + rl;
                int64_t tot = 0;  // the row's integer dot product, |tot| < K * 2^38
#pragma unroll
                for (int l = 0; l < PL_MAX; l++)
                    if (l < L) tot += (int64_t)acc[i][j][l][e] * ((int64_t)1 << (8 * l));
                sC[rl * GM_TOK + tl] =
                    (tile < w.tiles && row < w.rows) ? dn::round_to_i32((dn::i128)tot * (dn::i128)w.row_scale[row], 24) : 0;
            }
        }
    }
    __syncthreads();
    for (uint32_t c = tid; c < GM_TILES * Q8_TILE_ROWS * GM_TOK; c += GM_THREADS) {
        const uint32_t rl = c % (GM_TILES * Q8_TILE_ROWS), tl = c / (GM_TILES * Q8_TILE_ROWS);
        const uint32_t row = tile0 * Q8_TILE_ROWS + rl, token = tok0 + tl;
        if (row < w.rows && token < M) store_output(a, row, token, sC[rl * GM_TOK + tl], sC[(rl ^ 1) * GM_TOK + tl]);
    }
}

}  // namespace

bool iris_gemm_applies(const GemvArgs& a) {
    return a.planes && a.token_limbs && a.tokens >= 2 && a.w.scale_mode == Q8_SCALE_ROW && a.w.cols % GM_K == 0 &&
           a.w.cols < (1u << 17) && a.epilogue != EPI_HEAD_SELECT;
}

int iris_gemm_launch(const GemvArgs& a, hipStream_t stream) {
    if (!iris_gemm_applies(a) || a.x_stride % 4 || ((uintptr_t)a.x & 15)) return IRIS_E_INVALID;
    if (a.prologue == PRO_RMSNORM && ((uintptr_t)a.norm_w & 15)) return IRIS_E_INVALID;
    hipLaunchKernelGGL(digit_planes_kernel, dim3(a.tokens), dim3(256), 0, stream, a);
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return (int)st;
    const dim3 grid((a.tokens + GM_TOK - 1) / GM_TOK, (a.w.tiles + GM_TILES - 1) / GM_TILES);
    hipLaunchKernelGGL(q8_gemm_row_kernel, grid, dim3(GM_THREADS), 0, stream, a);
    return (int)hipGetLastError();
}
