// One-token Q8_0 products whose activation row arrives as digit planes
// written by its producer (act_planes.h): the decode O product (the
// attention's values launch writes the planes of its context row) and the
// down product (the gate/up product's SwiGLU epilogue writes those of the
// gated row).
//
// Every lane of a wave takes one row of four 16-row tiles, and the whole
// wave walks the same blocks, so the activation digits a block needs are
// the same for every lane: they come through scalar loads straight into
// scalar registers, the dot products' shared operand. No row is staged
// through LDS, and no row load queues behind the weight stream: a vector
// load issued behind ~100 KB of weight loads on a CU returns 2-3 us later,
// a scalar load in under 0.1 us (measured on MI355X).
//
// A workgroup of BC_W waves takes one group of four tiles and one of
// `parts` slices of the row (each wave 1/BC_W of the slice). The slices'
// exact partial sums meet through the k split's scratch: each workgroup
// stores its 64 sums with agent-scope atomic stores, waits for them, and
// adds one to the group's counter; the workgroup that arrives last adds
// the others' sums, finishes the rows and clears the counter. Integer sums
// are the same in any order, so the result does not depend on which
// workgroup arrives last. No wait spins: every workgroup runs to its end.
//
// Exactness: as the staged GEMV (q8_gemv.hip), each block's 32 weights
// times the value digits plane by plane in int32 (|sum| < 32 * 127 * 128),
// shifted into an int64 block sum, summed in int64 (|block sum| < 2^44,
// blocks < 2^17), times the row scale in 128 bits and rounded (ops.rs
// dot_row; q8_product.cu:50-101 forms the same exact sum).
#include "act_planes.h"
#include "q8_epilogue.h"
#include "q8_internal.h"
#include "wave_ops.h"

namespace {

constexpr int BC_W = 8;       // waves per workgroup
constexpr int BC_AHEAD = 4;   // blocks of weights in flight per lane

// Plane l's dot products of one block (32 weights q0|q1 against the 8
// dwords of its digits at p), added to the plane's two int32 chains.
__device__ __forceinline__ void bcast_plane_dots(const uint4 q0, const uint4 q1, const uint32_t* __restrict__ p,
                                                 int& s0, int& s1) {
    s0 = __builtin_amdgcn_sdot4((int)q0.x, (int)p[0], s0, false);
    s1 = __builtin_amdgcn_sdot4((int)q1.x, (int)p[4], s1, false);
    s0 = __builtin_amdgcn_sdot4((int)q0.y, (int)p[1], s0, false);
    s1 = __builtin_amdgcn_sdot4((int)q1.y, (int)p[5], s1, false);
    s0 = __builtin_amdgcn_sdot4((int)q0.z, (int)p[2], s0, false);
    s1 = __builtin_amdgcn_sdot4((int)q1.z, (int)p[6], s1, false);
    s0 = __builtin_amdgcn_sdot4((int)q0.w, (int)p[3], s0, false);
    s1 = __builtin_amdgcn_sdot4((int)q1.w, (int)p[7], s1, false);
}

// Blocks [b0, b1) of the lane's row (qrow: the row's first block), the
// first BC_AHEAD already loaded into q (clamped to b1 - 1). Whole groups of
// BC_AHEAD blocks sum each plane over the group in int32 (at most 4 * 16
// products of |127 * 128|: no overflow) before the shifted int64 add; the
// last partial group's blocks are taken one by one under a branch that is
// the same for the whole wave. Loads past b1 re-read block b1 - 1.
template <int L>
__device__ __forceinline__ int64_t bcast_blocks(const uint8_t* qrow, const uint32_t* __restrict__ planes, uint32_t pw,
                                                uint32_t b0, uint32_t b1, uint4 (&q)[BC_AHEAD][2]) {
    int64_t acc = 0;
    uint32_t b = b0;
    for (; b + BC_AHEAD <= b1; b += BC_AHEAD) {
        int s0[L], s1[L];
#pragma unroll
        for (int l = 0; l < L; l++) s0[l] = s1[l] = 0;
#pragma unroll
        for (int u = 0; u < BC_AHEAD; u++) {
#pragma unroll
            for (int l = 0; l < L; l++) bcast_plane_dots(q[u][0], q[u][1], planes + (b + u) * 8 + l * pw, s0[l], s1[l]);
            const uint32_t nb = min(b + BC_AHEAD + u, b1 - 1);
            q[u][0] = *(const uint4*)(qrow + (size_t)nb * Q8_TILE_BLOCK_BYTES);
            q[u][1] = *(const uint4*)(qrow + (size_t)nb * Q8_TILE_BLOCK_BYTES + 256);
        }
#pragma unroll
        for (int l = 0; l < L; l++) acc += (int64_t)(s0[l] + s1[l]) << (8 * l);
    }
#pragma unroll
    for (int u = 0; u < BC_AHEAD - 1; u++) {
        if (b + u < b1) {
#pragma unroll
            for (int l = 0; l < L; l++) {
                int s0 = 0, s1 = 0;
                bcast_plane_dots(q[u][0], q[u][1], planes + (b + u) * 8 + l * pw, s0, s1);
                acc += (int64_t)(s0 + s1) << (8 * l);
            }
        }
    }
    return acc;
}

// The same sums for L (4 or 5) planes, one block and one plane at a time.
__device__ __forceinline__ int64_t bcast_blocks_wide(const uint8_t* qrow, const uint32_t* __restrict__ planes,
                                                     uint32_t pw, uint32_t b0, uint32_t b1, uint32_t L,
                                                     uint4 (&q)[BC_AHEAD][2]) {
    int64_t acc = 0;
#pragma unroll 1
    for (uint32_t b = b0; b < b1; b += BC_AHEAD) {
#pragma unroll
        for (int u = 0; u < BC_AHEAD; u++) {
            if (b + u < b1) {
#pragma unroll 1
                for (uint32_t l = 0; l < L; l++) {
                    int s0 = 0, s1 = 0;
                    bcast_plane_dots(q[u][0], q[u][1], planes + (b + u) * 8 + l * pw, s0, s1);
                    acc += (int64_t)(s0 + s1) << (8 * l);
                }
            }
            const uint32_t nb = min(b + BC_AHEAD + u, b1 - 1);
            q[u][0] = *(const uint4*)(qrow + (size_t)nb * Q8_TILE_BLOCK_BYTES);
            q[u][1] = *(const uint4*)(qrow + (size_t)nb * Q8_TILE_BLOCK_BYTES + 256);
        }
    }
    return acc;
}

__global__ __launch_bounds__(BC_W * 64) void q8_gemv_bcast_kernel(const GemvArgs a, const uint32_t* __restrict__ planes,
                                                                  const uint32_t* __restrict__ counts, uint32_t parts) {
    __shared__ int64_t red[BC_W][64];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const Q8View& w = a.w;
    const uint32_t nb = w.nb, pw = w.cols / 4;
    const uint32_t grp = blockIdx.x / parts, part = blockIdx.x % parts;
    const uint32_t tile = min(grp * 4 + (lane >> 4), w.tiles - 1);
    const uint32_t slices = parts * BC_W;
    const uint32_t b0 = __builtin_amdgcn_readfirstlane((part * BC_W + wave) * nb / slices);
    const uint32_t b1 = __builtin_amdgcn_readfirstlane((part * BC_W + wave + 1) * nb / slices);
    const uint8_t* qrow = w.qs + (size_t)tile * nb * Q8_TILE_BLOCK_BYTES + (lane & 15) * 16;
    uint4 q[BC_AHEAD][2];
#pragma unroll
    for (int u = 0; u < BC_AHEAD; u++) {
        const uint32_t b = min(b0 + u, b1 - 1);
        q[u][0] = *(const uint4*)(qrow + (size_t)b * Q8_TILE_BLOCK_BYTES);
        q[u][1] = *(const uint4*)(qrow + (size_t)b * Q8_TILE_BLOCK_BYTES + 256);
    }
    // The digits this wave's blocks need: the most of their counts (four
    // bytes per block, read as one dword).
    // Sixteen at a time (clamped repeats), all issued before one wait.
    uint32_t need = 1;
    for (uint32_t c0 = b0; c0 < b1; c0 += 16) {
        uint32_t c[16];
#pragma unroll
        for (int i = 0; i < 16; i++) c[i] = counts[min(c0 + i, b1 - 1)];
#pragma unroll
        for (int i = 0; i < 16; i++)
            need = max(need, max(max(c[i] & 0xff, (c[i] >> 8) & 0xff), max((c[i] >> 16) & 0xff, c[i] >> 24)));
    }
    // Rows whose values all fit three digits (the planes above are zero,
    // so fewer digits take the same path) run the unrolled sums; wider
    // values take the compact loop, so its registers do not set the
    // kernel's occupancy.
    const int64_t acc = need <= 3 ? bcast_blocks<3>(qrow, planes, pw, b0, b1, q)
                                  : bcast_blocks_wide(qrow, planes, pw, b0, b1, need, q);
    // The epilogue's inputs of the row this lane finishes (wave 0), loaded
    // while the workgroup's sums meet.
    const uint32_t row = grp * 64 + lane, rowc = min(row, w.rows - 1);
    int64_t rs = 0;
    EpiIn in{};
    if (wave == 0) {
        rs = w.row_scale[rowc];
        in = epilogue_inputs(a, rowc, 0);
    }
    red[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    int64_t t = 0;
#pragma unroll
    for (int i = 0; i < BC_W; i++) t += red[i][lane];
    if (parts > 1) {
        const uint32_t rows = w.tiles * Q8_TILE_ROWS;
        __hip_atomic_store(&a.kpart[(size_t)part * rows + min(row, rows - 1)], t, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        // Every partial stored (performed at agent scope) before the count.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        uint32_t old = 0;
        if (lane == 0) old = __hip_atomic_fetch_add(&a.kcount[grp], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = __builtin_amdgcn_readfirstlane(old);
        if (old != parts - 1) return;
        for (uint32_t k = 0; k < parts; k++)
            if (k != part)
                t += __hip_atomic_load(&a.kpart[(size_t)k * rows + min(row, rows - 1)], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        if (lane == 0) __hip_atomic_store(&a.kcount[grp], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const int32_t v = dn::round_to_i32((dn::i128)t * (dn::i128)rs, 24);
    const int32_t o = a.epilogue == EPI_RESIDUAL ? dn::add_sat(v, in.res) : v;
    const bool own = row < w.rows;
    if (a.ssq_out) {
        // Each tile's rows as stored, squared and summed with saturation
        // over its 16 lanes (the staged GEMV's slots).
        const int64_t sq = row16_sum_sat_nonneg(own ? (int64_t)o * o : 0);
        if ((lane & 15) == 0 && grp * 4 + (lane >> 4) < w.tiles) a.ssq_out[grp * 4 + (lane >> 4)] = sq;
    }
    if (own) a.out[row] = o;
}

// Row slices per group: four where each wave still gets at least four
// blocks (measured: N=4096 K=14336 13.6 us at four, 14.8 at two; N=14336
// K=4096 13.3 us at four, 14.6 at two), else two, else one.
uint32_t bcast_parts(uint32_t nb) {
    for (uint32_t p = BCAST_MAX_PARTS; p > 1; p /= 2)
        if (nb / (p * BC_W) >= 4) return p;
    return 1;
}

// A row's digit planes from its int32 values, one 32-value block per
// 64-lane workgroup (the producer of an isolated product's row).
__global__ __launch_bounds__(64) void act_planes_kernel(const int32_t* x, uint32_t cols, uint32_t* planes,
                                                        uint8_t* counts) {
    const uint32_t lane = threadIdx.x, first = blockIdx.x * 32;
    act_planes_store32(x[first + (lane & 31)], lane, first, cols, planes, counts);
}

}  // namespace

bool iris_gemv_bcast_applies(const GemvArgs& a) {
    return a.x && a.x_planes && a.x_counts && a.tokens == 1 && a.w.scale_mode == Q8_SCALE_ROW && a.prologue == PRO_NONE &&
           (a.epilogue == EPI_RESIDUAL || a.epilogue == EPI_STORE) && a.w.nb >= (uint32_t)BC_W && a.kpart &&
           a.kcount && ((uintptr_t)a.x_counts & 3) == 0;
}

int iris_gemv_bcast_launch(const GemvArgs& a, hipStream_t stream) {
    if (!iris_gemv_bcast_applies(a)) return IRIS_E_INVALID;
    const uint32_t parts = bcast_parts(a.w.nb);
    const uint32_t groups = bcast_groups(a.w.rows);
    hipLaunchKernelGGL(q8_gemv_bcast_kernel, dim3(groups * parts), dim3(BC_W * 64), 0, stream, a, a.x_planes,
                       (const uint32_t*)a.x_counts, parts);
    return (int)hipGetLastError();
}

extern "C" int iris_time_bcast_product(const Q8GpuMatrix* const* ms, uint32_t count, const int32_t* d_x, int32_t* d_out,
                                       uint32_t iterations, double* ms_per_product) {
    if (!ms || count == 0 || !ms[0] || !d_x || !d_out || !ms_per_product || iterations == 0) return IRIS_E_INVALID;
    const Q8GpuMatrix& m0 = *ms[0];
    for (uint32_t i = 0; i < count; i++)
        if (!ms[i] || ms[i]->rows != m0.rows || ms[i]->cols != m0.cols || ms[i]->scale_mode != Q8_SCALE_ROW)
            return IRIS_E_INVALID;
    if (m0.cols % 32 || m0.nb < (uint32_t)BC_W || ((uintptr_t)d_x & 15)) return IRIS_E_INVALID;
    const uint64_t plane_bytes = act_planes_dwords(m0.cols) * 4, count_bytes = (act_counts_bytes(m0.cols) + 15) / 16 * 16;
    const uint64_t part_bytes = (uint64_t)BCAST_MAX_PARTS * m0.tiles * Q8_TILE_ROWS * 8;
    const uint64_t cnt_bytes = (uint64_t)bcast_groups(m0.rows) * 4;
    char* buf = nullptr;
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = (int)hipMalloc(&buf, plane_bytes + count_bytes + part_bytes + cnt_bytes);
    if (rc == 0) rc = (int)hipStreamCreate(&s);
    if (rc == 0) rc = (int)hipEventCreate(&e0);
    if (rc == 0) rc = (int)hipEventCreate(&e1);
    GemvArgs a{};
    if (rc == 0) {
        a.x_planes = (const uint32_t*)buf;
        a.x_counts = (const uint8_t*)(buf + plane_bytes);
        a.kpart = (int64_t*)(buf + plane_bytes + count_bytes);
        a.kcount = (uint32_t*)(buf + plane_bytes + count_bytes + part_bytes);
        rc = (int)hipMemsetAsync(a.kcount, 0, cnt_bytes, s);
    }
    if (rc == 0) {
        hipLaunchKernelGGL(act_planes_kernel, dim3(m0.cols / 32), dim3(64), 0, s, d_x, m0.cols, (uint32_t*)a.x_planes,
                           (uint8_t*)a.x_counts);
        rc = (int)hipGetLastError();
    }
    a.x = d_x;
    a.x_stride = m0.cols;
    a.tokens = 1;
    a.epilogue = EPI_STORE;
    a.out = d_out;
    a.out_stride = m0.rows;
    auto launch = [&](const Q8GpuMatrix* m) {
        a.w = q8_view(m);
        return iris_gemv_bcast_launch(a, s);
    };
    for (uint32_t i = 0; rc == 0 && i < count; i++) rc = launch(ms[i]);
    if (rc == 0) rc = (int)hipEventRecord(e0, s);
    for (uint32_t i = 0; rc == 0 && i < iterations; i++) rc = launch(ms[i % count]);
    if (rc == 0) rc = (int)hipEventRecord(e1, s);
    if (rc == 0) rc = (int)hipEventSynchronize(e1);
    float elapsed = 0.f;
    if (rc == 0) rc = (int)hipEventElapsedTime(&elapsed, e0, e1);
    if (rc == 0) *ms_per_product = (double)elapsed / iterations;
    if (s) (void)hipStreamSynchronize(s);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (s) (void)hipStreamDestroy(s);
    if (buf) (void)hipFree(buf);
    return rc;
}
