// The gemma-dense layer's kernels that are not Q8_0 products:
//  - the per-head q/k rms_norm + RoPE and v value-norm after the q|k|v
//    product, with the K/V cache store (prefill_range.rs:607-647);
//  - rms_norm of a product's rows followed by the residual add (the post
//    norms, prefill_range.rs:879-958);
//  - products with Q16.16 matrices, dot_bits rows (tensor.rs:522-528), for
//    the per-layer-input (PLE) gate and projection;
//  - the PLE prepare step of every layer (view_kernels.rs:59-99);
//  - the RoPE frequency ladder (ops.rs:154-199, 558-620), built once.
#include "detnum_dev.h"
#include "layer_kernels.h"

namespace {

constexpr uint32_t NT = 256;  // threads per workgroup in this file
constexpr uint32_t NW = NT / 64;

__device__ __forceinline__ int64_t wave_sum_sat(int64_t v) {
    for (int off = 32; off >= 1; off >>= 1) v = dn::acc_add_sat(v, __shfl_xor(v, off));
    return v;
}

// Saturating sum of non-negative terms over the workgroup (order-free:
// the result is min(true sum, i64::MAX) whatever the order).
__device__ __forceinline__ int64_t block_sum_sat(int64_t v, int64_t* s_red) {
    const uint32_t tid = threadIdx.x;
    v = wave_sum_sat(v);
    if ((tid & 63) == 0) s_red[tid >> 6] = v;
    __syncthreads();
    int64_t t = 0;
    for (uint32_t i = 0; i < NW; i++) t = dn::acc_add_sat(t, s_red[i]);
    __syncthreads();  // s_red may be reused by the caller
    return t;
}

// One head of one row per workgroup. Heads [0, heads) are queries,
// [heads, heads+kv_heads) keys, then values, as the q|k|v product stacks
// them. q, k: rms_norm with their weights, then RoPE on pairs
// (i, i + rotary/2); v: the weightless value norm (ops.rs:124-134).
__global__ __launch_bounds__(NT) void gemma_qkv_finish_kernel(const GemmaQkvArgs a) {
    __shared__ int32_t s_v[GEMMA_MAX_HEAD_DIM];
    __shared__ int64_t s_red[NW];
    const uint32_t h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    const uint32_t hd = a.head_dim;
    const int32_t* src = a.qkv + (size_t)t * a.qkv_stride + (size_t)h * hd;
    int64_t ss = 0;
    for (uint32_t i = tid; i < hd; i += NT) {
        const int32_t v = src[i];
        s_v[i] = v;
        ss = dn::acc_add_sat(ss, (int64_t)v * v);
    }
    const int32_t scale = dn::rms_scale_from_sum(block_sum_sat(ss, s_red), hd, a.eps);
    const bool is_q = h < a.heads, is_k = !is_q && h < a.heads + a.kv_heads;
    const int32_t* nw = is_q ? a.q_norm : a.k_norm;
    for (uint32_t i = tid; i < hd; i += NT)
        s_v[i] = (is_q || is_k) ? dn::mul_sat(dn::mul_sat(s_v[i], scale), nw[i]) : dn::mul_sat(s_v[i], scale);
    __syncthreads();
    const uint32_t pos = (uint32_t)(*a.d_pos) + t;
    if ((is_q || is_k) && pos != 0 && a.rotary_dim != 0) {
        const uint32_t half = a.rotary_dim / 2;
        for (uint32_t i = tid; i < half; i += NT) {
            // mul_usize_by_acc (ops.rs:616-620): position * inv_f, clamped.
            const int64_t angle = dn::clamp_i128_to_i64((dn::i128)pos * (dn::i128)a.inv_freq[i]);
            int32_t c, s;
            dn::sin_cos_acc(angle, c, s);
            const int32_t lhs = s_v[i], rhs = s_v[i + half];
            s_v[i] = dn::sub_sat(dn::mul_sat(lhs, c), dn::mul_sat(rhs, s));
            s_v[i + half] = dn::add_sat(dn::mul_sat(rhs, c), dn::mul_sat(lhs, s));
        }
        __syncthreads();
    }
    if (is_q) {
        int32_t* dst = a.q_out + (size_t)t * a.q_stride + (size_t)h * hd;
        for (uint32_t i = tid; i < hd; i += NT) dst[i] = s_v[i];
    } else if (is_k) {
        const size_t kbase = (size_t)(h - a.heads) * hd;
        for (uint32_t i = tid; i < hd; i += NT) a.k_cache[(kbase + i) * a.k_pos_stride + pos] = s_v[i];
    } else {
        const size_t vbase = (size_t)(h - a.heads - a.kv_heads) * hd;
        int32_t* dst = a.v_cache + (size_t)pos * ((size_t)a.kv_heads * hd) + vbase;
        for (uint32_t i = tid; i < hd; i += NT) dst[i] = s_v[i];
    }
}

// out = add_sat(rms_norm(a, w), res), then mul_sat(., scalar) when scalar is
// set (the layer scalar, prefill_range.rs:946-958). One row per workgroup;
// out may be res (each element is read and written by one thread).
__global__ __launch_bounds__(NT) void norm_residual_kernel(const int32_t* a, uint32_t a_stride, const int32_t* w,
                                                           int64_t eps, const int32_t* res, uint32_t res_stride,
                                                           int32_t scalar, int32_t* out, uint32_t out_stride,
                                                           uint32_t n) {
    __shared__ int64_t s_red[NW];
    const uint32_t t = blockIdx.x, tid = threadIdx.x;
    const int32_t* ar = a + (size_t)t * a_stride;
    int64_t ss = 0;
    for (uint32_t i = tid; i < n; i += NT) ss = dn::acc_add_sat(ss, (int64_t)ar[i] * ar[i]);
    const int32_t scale = dn::rms_scale_from_sum(block_sum_sat(ss, s_red), n, eps);
    const int32_t* rr = res + (size_t)t * res_stride;
    int32_t* orow = out + (size_t)t * out_stride;
    for (uint32_t i = tid; i < n; i += NT) {
        int32_t v = dn::add_sat(dn::mul_sat(dn::mul_sat(ar[i], scale), w[i]), rr[i]);
        if (scalar != 0) v = dn::mul_sat(v, scalar);
        orow[i] = v;
    }
}

// out[t][r] = requantize(wrapping sum_k x[t][k] * W[r][k]) for a Q16.16
// matrix W [rows][cols] (dot_bits, tensor.rs:522-528; mac_bits ops.rs:17-19),
// optionally followed by mul_sat(gelu(.), aux[t][r]) (the PLE gate,
// prefill_range.rs:931-944). Four waves per workgroup, rows_per_wave rows
// each (row = base + j * NW + wave).
//
// One-row extras (I32GemvArgs): the input formed in LDS as the post-norm
// and residual of the previous product (norm_residual_kernel's arithmetic),
// and per-workgroup sums of squares of the outputs.
constexpr uint32_t I32_ROUND = 8;  // 16-byte loads a lane has in flight per row chunk

__global__ __launch_bounds__(NT) void i32_gemv_kernel(const I32GemvArgs a, uint32_t rows_per_wave) {
    extern __shared__ __align__(16) int32_t s_x[];  // the staged input row (res_in set)
    __shared__ int64_t s_red[NW];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t t = blockIdx.y;
    const int32_t* xr = a.x + (size_t)t * a.x_stride;
    const uint32_t c4 = a.cols / 4;
    if (a.res_in) {
        // Every load of the thread's share first (clamped indices, at most
        // I32_GEMV_MAX_STAGED / 4 / NT 16-byte loads per array), then the
        // slots' sum, then the row.
        constexpr uint32_t PER = I32_GEMV_MAX_STAGED / 4 / NT;
        int4 xv[PER], wv[PER], rv[PER];
#pragma unroll
        for (uint32_t u = 0; u < PER; u++) xv[u] = ((const int4*)xr)[min(u * NT + tid, c4 - 1)];
#pragma unroll
        for (uint32_t u = 0; u < PER; u++) wv[u] = ((const int4*)a.res_norm_w)[min(u * NT + tid, c4 - 1)];
#pragma unroll
        for (uint32_t u = 0; u < PER; u++) rv[u] = ((const int4*)a.res_in)[min(u * NT + tid, c4 - 1)];
        int64_t sl[I32_GEMV_MAX_SLOTS / 64];
#pragma unroll
        for (uint32_t u = 0; u < I32_GEMV_MAX_SLOTS / 64; u++) sl[u] = a.ssq_in[min(lane + 64 * u, a.ssq_n - 1)];
        int64_t ss = 0;
#pragma unroll
        for (uint32_t u = 0; u < I32_GEMV_MAX_SLOTS / 64; u++)
            if (lane + 64 * u < a.ssq_n) ss = dn::acc_add_sat(ss, sl[u]);
        const int32_t scale = dn::rms_scale_from_sum(wave_sum_sat(ss), a.cols, a.eps);
        const bool store = a.res_out != nullptr && blockIdx.x == 0;
#pragma unroll
        for (uint32_t u = 0; u < PER; u++) {
            const uint32_t i = u * NT + tid;
            if (i < c4) {
                int4 y;
                y.x = dn::add_sat(dn::mul_sat(dn::mul_sat(xv[u].x, scale), wv[u].x), rv[u].x);
                y.y = dn::add_sat(dn::mul_sat(dn::mul_sat(xv[u].y, scale), wv[u].y), rv[u].y);
                y.z = dn::add_sat(dn::mul_sat(dn::mul_sat(xv[u].z, scale), wv[u].z), rv[u].z);
                y.w = dn::add_sat(dn::mul_sat(dn::mul_sat(xv[u].w, scale), wv[u].w), rv[u].w);
                ((int4*)s_x)[i] = y;
                if (store) ((int4*)a.res_out)[i] = y;
            }
        }
        __syncthreads();
        xr = s_x;
    }
    int64_t sq = 0;
    const uint32_t base = blockIdx.x * NW * rows_per_wave;
    for (uint32_t j = 0; j < rows_per_wave; j++) {
        const uint32_t row = base + j * NW + wave;
        if (row >= a.rows) break;
        const int4* wr = (const int4*)(a.w + (size_t)row * a.cols);
        uint64_t acc = 0;
        // I32_ROUND loads of the row in flight at once (clamped, dropped
        // past the row's end).
        for (uint32_t k0 = 0; k0 < c4; k0 += 64 * I32_ROUND) {
            int4 wv[I32_ROUND], xv[I32_ROUND];
#pragma unroll
            for (uint32_t u = 0; u < I32_ROUND; u++) wv[u] = wr[min(k0 + u * 64 + lane, c4 - 1)];
#pragma unroll
            for (uint32_t u = 0; u < I32_ROUND; u++) xv[u] = ((const int4*)xr)[min(k0 + u * 64 + lane, c4 - 1)];
#pragma unroll
            for (uint32_t u = 0; u < I32_ROUND; u++) {
                if (k0 + u * 64 + lane < c4) {
                    acc += (uint64_t)((int64_t)xv[u].x * wv[u].x);
                    acc += (uint64_t)((int64_t)xv[u].y * wv[u].y);
                    acc += (uint64_t)((int64_t)xv[u].z * wv[u].z);
                    acc += (uint64_t)((int64_t)xv[u].w * wv[u].w);
                }
            }
        }
        for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
        int32_t v = dn::requantize((int64_t)acc);
        if (a.aux) v = dn::mul_sat(dn::gelu(v), a.aux[(size_t)t * a.aux_stride + row]);
        if (lane == 0) a.out[(size_t)t * a.out_stride + row] = v;
        sq = dn::acc_add_sat(sq, (int64_t)v * v);
    }
    if (a.ssq_out) {
        // Every lane holds its wave's sum (the values are wave-uniform).
        if (lane == 0) s_red[wave] = sq;
        __syncthreads();
        if (tid == 0) {
            int64_t total = 0;
            for (uint32_t i = 0; i < NW; i++) total = dn::acc_add_sat(total, s_red[i]);
            a.ssq_out[blockIdx.x] = total;
        }
    }
}

// The PLE input of one layer segment for one row (view_kernels.rs:74-88):
// p = rms_norm(mul_sat(proj, projection_scalar), norm); e = the token's
// dequantized embed_tokens_per_layer columns of the segment, times the
// embedding scale; out = mul_sat(add_sat(e, p), input_scale).
__global__ __launch_bounds__(NT) void ple_prepare_kernel(const PleArgs a) {
    __shared__ int32_t s_p[GEMMA_MAX_PLE];
    __shared__ int64_t s_red[NW];
    const uint32_t seg = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    const uint32_t P = a.ple_width;
    const int32_t* pr = a.proj + (size_t)t * a.row_stride + (size_t)seg * P;
    int64_t ss = 0;
    for (uint32_t c = tid; c < P; c += NT) {
        const int32_t p = dn::mul_sat(pr[c], a.projection_scalar);
        s_p[c] = p;
        ss = dn::acc_add_sat(ss, (int64_t)p * p);
    }
    const int32_t scale = dn::rms_scale_from_sum(block_sum_sat(ss, s_red), P, a.eps);
    const uint8_t* er = a.emb + (size_t)a.ids[t] * a.emb_row_bytes;
    int32_t* orow = a.out + (size_t)t * a.row_stride + (size_t)seg * P;
    for (uint32_t c = tid; c < P; c += NT) {
        const int32_t p = dn::mul_sat(dn::mul_sat(s_p[c], scale), a.norm_w[c]);
        const uint32_t col = seg * P + c;
        const uint8_t* blk = er + (size_t)(col / 32) * 34;
        const int64_t sc = dn::scale_q24((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        int32_t e = dn::round_to_i32((dn::i128)((int64_t)(int8_t)blk[2 + col % 32] * sc), 8);
        e = dn::add_sat(dn::mul_sat(e, a.embedding_scale), p);
        orow[c] = dn::mul_sat(e, a.input_scale);
    }
}

// inv_f[i] for i < half: ONE, then repeated acc_mul by
// step = div_acc(ONE, nth_root(base, freq_base_dim / 2)) (ops.rs:154-199,
// 558-562). Sequential by definition; one thread, once per model.
__global__ void rope_ladder_kernel(int64_t base, uint32_t freq_base_dim, uint32_t half, int64_t* out) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    const int64_t step = dn::div_acc(dn::ONE_ACC, dn::nth_root_acc(base, freq_base_dim / 2));
    int64_t f = dn::ONE_ACC;
    for (uint32_t i = 0; i < half; i++) {
        out[i] = f;
        f = dn::acc_mul(f, step);
    }
}

}  // namespace

int iris_gemma_qkv_finish_launch(const GemmaQkvArgs& a, uint32_t rows, hipStream_t stream) {
    if (a.head_dim == 0 || a.head_dim > GEMMA_MAX_HEAD_DIM || a.rotary_dim > a.head_dim || a.rotary_dim % 2)
        return IRIS_E_INVALID;
    if (rows == 0) return 0;
    hipLaunchKernelGGL(gemma_qkv_finish_kernel, dim3(a.heads + 2 * a.kv_heads, rows), dim3(NT), 0, stream, a);
    return (int)hipGetLastError();
}

int iris_norm_residual_launch(const int32_t* a, uint32_t a_stride, const int32_t* w, int64_t eps, const int32_t* res,
                              uint32_t res_stride, int32_t scalar, int32_t* out, uint32_t out_stride, uint32_t n,
                              uint32_t rows, hipStream_t stream) {
    if (n == 0) return IRIS_E_INVALID;
    if (rows == 0) return 0;
    hipLaunchKernelGGL(norm_residual_kernel, dim3(rows), dim3(NT), 0, stream, a, a_stride, w, eps, res, res_stride,
                       scalar, out, out_stride, n);
    return (int)hipGetLastError();
}

uint32_t i32_gemv_slots(uint32_t rows) {
    const uint32_t per_wave = (rows + NW * I32_GEMV_MAX_SLOTS - 1) / (NW * I32_GEMV_MAX_SLOTS);
    return (rows + NW * per_wave - 1) / (NW * per_wave);
}

int iris_i32_gemv_launch(const I32GemvArgs& a, uint32_t tokens, hipStream_t stream) {
    if (a.rows == 0 || a.cols == 0 || a.cols % 4 || a.x_stride % 4) return IRIS_E_INVALID;
    if (((uintptr_t)a.x | (uintptr_t)a.w) & 15) return IRIS_E_INVALID;
    if (tokens == 0) return 0;
    if ((a.res_in || a.ssq_out) && tokens != 1) return IRIS_E_INVALID;
    size_t shmem = 0;
    if (a.res_in) {
        if (!a.res_norm_w || !a.ssq_in || a.ssq_n == 0 || a.ssq_n > I32_GEMV_MAX_SLOTS || a.cols > I32_GEMV_MAX_STAGED)
            return IRIS_E_INVALID;
        if (((uintptr_t)a.x | (uintptr_t)a.res_in | (uintptr_t)a.res_norm_w | (uintptr_t)a.res_out) & 15)
            return IRIS_E_INVALID;
        if (a.res_out && (a.res_out == a.res_in || a.res_out == a.x)) return IRIS_E_INVALID;
        shmem = (size_t)a.cols * 4;
    }
    uint32_t per_wave = 1, wgs = (a.rows + NW - 1) / NW;
    if (a.ssq_out) {
        wgs = i32_gemv_slots(a.rows);
        per_wave = (a.rows + NW * I32_GEMV_MAX_SLOTS - 1) / (NW * I32_GEMV_MAX_SLOTS);
    }
    hipLaunchKernelGGL(i32_gemv_kernel, dim3(wgs, tokens), dim3(NT), shmem, stream, a, per_wave);
    return (int)hipGetLastError();
}

int iris_ple_prepare_launch(const PleArgs& a, uint32_t segments, uint32_t rows, hipStream_t stream) {
    if (a.ple_width == 0 || a.ple_width > GEMMA_MAX_PLE) return IRIS_E_INVALID;
    if (rows == 0 || segments == 0) return 0;
    hipLaunchKernelGGL(ple_prepare_kernel, dim3(segments, rows), dim3(NT), 0, stream, a);
    return (int)hipGetLastError();
}

int iris_rope_ladder_launch(int64_t base, uint32_t freq_base_dim, uint32_t half, int64_t* out, hipStream_t stream) {
    if (half == 0) return 0;
    hipLaunchKernelGGL(rope_ladder_kernel, dim3(1), dim3(64), 0, stream, base, freq_base_dim, half, out);
    return (int)hipGetLastError();
}
