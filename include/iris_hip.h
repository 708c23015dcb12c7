/*
 * libiris_hip: exact Q8_0 products and the deterministic token loop on an
 * AMD Instinct MI355X (gfx950).
 *
 * Every value these entry points produce is bit-identical to the reference's
 * CPU kernels (casettek/iris, crates/det-num and crates/inference/kernels):
 * the arithmetic is integer-only, with the reference's rounding and
 * saturation at every step, and no result depends on launch shape, thread
 * count or reduction order.
 *
 * Return codes: 0 is success; a positive value is a hipError_t; a negative
 * value is a library code (see q8gpu_error for its text).
 */
#ifndef IRIS_HIP_H
#define IRIS_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------
 * Drop-in for the reference's NVIDIA product library: the same five symbols
 * with the same layouts and semantics.
 *   replaces crates/inference/kernels/cuda/q8_product.cu:122-197,
 *   bound by crates/inference/kernels/src/gpu.rs:40-62.
 * ---------------------------------------------------------------------- */

/* Opaque device matrix (gpu.rs:40-43). */
typedef struct Q8GpuMatrix Q8GpuMatrix;

/* Static text for any return code of this library (q8_product.cu:131). */
const char* q8gpu_error(int code);

/* Creates the device context; fails when there is no usable device
 * (q8_product.cu:134-139). */
int q8gpu_init(void);

/* Copies a matrix to the device (q8_product.cu:150-172): `weights` is
 * rows*cols signed bytes row by row, `scales` one Q.24 scale per 32-weight
 * block, rows*(cols/32) values. *out is NULL on failure. */
int q8gpu_upload(const int8_t* weights, const int64_t* scales, uint32_t rows, uint32_t cols,
                 Q8GpuMatrix** out);

/* Releases a matrix; NULL is ignored (q8_product.cu:141-146). */
void q8gpu_free(Q8GpuMatrix* matrix);

/* out[token*rows + row] = det_num::q8::dot_row(activations[token], row);
 * activations is tokens*cols Q16.16 values, token by token, in host memory;
 * synchronous (q8_product.cu:176-195). */
int q8gpu_product(const Q8GpuMatrix* matrix, const int32_t* activations, uint32_t tokens, int32_t* out);

/* ------------------------------------------------------------------------
 * Device-resident extensions (no reference counterpart in C; they replace
 * the Rust side's de-interleaving upload, gpu.rs:154-219, and its per-product
 * host round trip, gpu.rs:249-309).
 * ---------------------------------------------------------------------- */

/* Uploads a Q8_0 matrix from its committed bytes: rows of cols/32 blocks of
 * 34 bytes (f16 scale little-endian, then 32 signed bytes), as
 * MatrixSource::q8_source hands them over (crates/inference/kernels/src/tensor.rs:110-115).
 * Fails with a library code for a non-finite scale, as dot_row does. */
int q8gpu_upload_q8_0(const uint8_t* blocks, uint32_t rows, uint32_t cols, Q8GpuMatrix** out);

/* The same product as q8gpu_product, on device pointers, enqueued on
 * `stream` (a hipStream_t; NULL = the null stream). Does not synchronise. */
int q8gpu_product_device(const Q8GpuMatrix* matrix, const int32_t* d_activations, uint32_t tokens,
                         int32_t* d_out, void* stream);

/* rows, cols and the device layout the upload chose: 0 = one scale per row
 * (every block of each row shares it), 1 = one f16 per block, 2 = one i64 per
 * block; bytes = device memory held. */
int q8gpu_matrix_info(const Q8GpuMatrix* matrix, uint32_t* rows, uint32_t* cols, int* scale_mode,
                      uint64_t* bytes);

/* Waits for all work on the device. */
int q8gpu_synchronize(void);

/* ------------------------------------------------------------------------
 * Plumbing for callers with no HIP binding of their own (tests, benchmarks).
 * ---------------------------------------------------------------------- */

int iris_device_malloc(uint64_t bytes, void** out);
int iris_device_free(void* ptr);
int iris_memcpy_h2d(void* dst, const void* src, uint64_t bytes);
int iris_memcpy_d2h(void* dst, const void* src, uint64_t bytes);

/* Runs q8gpu_product_device `iterations` times back to back on one stream
 * after one warm-up call and reports the mean time per product from HIP
 * events recorded on that stream. */
int iris_time_product(const Q8GpuMatrix* matrix, const int32_t* d_activations, uint32_t tokens, int32_t* d_out,
                      uint32_t iterations, double* ms_per_product);

#ifdef __cplusplus
}
#endif

#endif /* IRIS_HIP_H */
