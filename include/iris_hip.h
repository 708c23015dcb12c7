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
 * value is a library code (see q8gpu_error for its text): -1 invalid
 * argument or shape, -2 non-finite Q8_0 scale, -3 host allocation failed,
 * -4 wrong state, -5 past the object's capacity, -6 past the no-allocation
 * scratch, -7 graph replays asked for under a kernel tracer.
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

/* Device bytes of work space a `tokens`-token product may use (0 for a
 * single token). */
uint64_t q8gpu_workspace_bytes(const Q8GpuMatrix* matrix, uint32_t tokens);

/* q8gpu_product_device with caller-provided device work space of at least
 * q8gpu_workspace_bytes: a multi-token product of a matrix whose blocks share
 * one scale per row, or of a per-block scale matrix that
 * q8gpu_prepare_matrix_cores has folded, then runs on the int8 matrix cores
 * (same bits). NULL work space = q8gpu_product_device. Returns IRIS_E_RANGE
 * (-5) when it is too small. Asynchronous: it allocates nothing and never
 * changes the matrix. The synchronous q8gpu_product uses its own work
 * space. */
int q8gpu_product_device_ws(const Q8GpuMatrix* matrix, const int32_t* d_activations, uint32_t tokens,
                            int32_t* d_out, void* d_workspace, uint64_t workspace_bytes, void* stream);

/* Folds a per-block scale matrix's scales into weight digit planes so that
 * its multi-token products (q8gpu_product_device_ws, _noalloc and
 * q8gpu_product) run on the int8 matrix cores. Every matrix of finite
 * scales folds: 1 to Q8_FOLD_MAX_PLANES (6) planes, by how far a row's
 * scales spread (3 for the reference bundles' layout, 6 for a subnormal
 * block beside exponent 30). Allocates that many x rows x cols bytes more
 * device memory, plus 4 bytes per row (reported by q8gpu_matrix_info's
 * bytes), and synchronises `stream`. Does nothing, and returns 0, for a
 * row-scale matrix or one already prepared. Not to be called while other
 * calls use the matrix. No counterpart in the reference (whose device cache budgets
 * rows*cols + blocks*8 bytes per matrix, gpu.rs:171-173: a prepared matrix
 * holds more). */
int q8gpu_prepare_matrix_cores(Q8GpuMatrix* matrix, void* stream);

/* Bytes of each device's scratch array (below): 32 MiB. */
#define IRIS_NOALLOC_SCRATCH_BYTES (32ull << 20)

/* q8gpu_product_device_ws without any allocation: the work space is a
 * file-scope device array of IRIS_NOALLOC_SCRATCH_BYTES per device, held
 * until the process ends. No counterpart in the reference: it is for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Returns IRIS_E_SCRATCH (-6), and runs
 * nothing, when q8gpu_workspace_bytes(matrix, tokens) exceeds the array.
 * Every call on one device shares that device's array: calls that overlap on
 * one device (other streams, other threads) race and must be serialised by
 * the caller; calls in order on one stream are safe. */
int q8gpu_product_device_noalloc(const Q8GpuMatrix* matrix, const int32_t* d_activations, uint32_t tokens,
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
/* Device-to-device copy (a plain copy kernel of known size, which is what
 * hardware byte counters are calibrated against). */
int iris_memcpy_d2d(void* dst, const void* src, uint64_t bytes);

/* Runs q8gpu_product_device `iterations` times back to back on one stream,
 * cycling through `count` matrices of one shape (so that, with enough of
 * them, every product reads its weights from HBM rather than from the
 * last-level cache), after one warm-up pass over all of them, and reports
 * the mean time per product from HIP events recorded on that stream. */
int iris_time_product(const Q8GpuMatrix* const* matrices, uint32_t count, const int32_t* d_activations,
                      uint32_t tokens, int32_t* d_out, uint32_t iterations, double* ms_per_product);

/* The one-token product as the decode loop runs it when the row's producer
 * leaves the row as digit planes (no counterpart in the reference; a
 * measurement and parity entry): forms the planes of d_activations (one row
 * of cols int32 values) once, then runs the product from them `iterations`
 * times back to back cycling through `count` row-scale matrices of one shape
 * (cols >= 256), as iris_time_product does, and reports the mean time per
 * product. d_out holds the last product's rows (the same as
 * q8gpu_product_device's for that matrix). */
int iris_time_bcast_product(const Q8GpuMatrix* const* matrices, uint32_t count, const int32_t* d_activations,
                            int32_t* d_out, uint32_t iterations, double* ms_per_product);

/* As iris_time_product for one matrix through q8gpu_product_device_ws: with
 * the work space, multi-token products of row-scale matrices run on the int8
 * matrix cores (digit planes plus the MFMA GEMM), and this times them. */
int iris_time_product_ws(const Q8GpuMatrix* matrix, const int32_t* d_activations, uint32_t tokens, int32_t* d_out,
                         void* d_workspace, uint64_t workspace_bytes, uint32_t iterations, double* ms_per_product);

/* Measured peaks of the device (no counterpart in the reference; reported
 * beside the vendor figures). iris_probe_hbm_read: the read rate of a plain
 * streaming kernel (16-byte loads at a grid stride, the best of a few grid
 * sizes) over `bytes` of device memory at d_buf (16-byte aligned; larger
 * than the last-level cache for an HBM figure), averaged over `repeats`
 * passes, in GB/s. iris_probe_mfma_i8: the rate of v_mfma_i32_32x32x32_i8 in
 * a loop of independent accumulators on every SIMD (four waves per SIMD),
 * `iterations` (at least 4) instructions per accumulator, in TOP/s, with
 * constant operands (random_operands = 0) or with random operands that
 * change every instruction (1). */
int iris_probe_hbm_read(const void* d_buf, uint64_t bytes, uint32_t repeats, double* gb_per_s);
int iris_probe_mfma_i8(uint32_t random_operands, uint32_t iterations, double* tops);
/* Handoffs between workgroups inside one launch (no counterpart in the
 * reference; what a kernel that waits on other workgroups pays, against a
 * launch boundary): the round trip of a flag between two workgroups on
 * different XCDs through agent-scope atomic stores and loads, in
 * microseconds; one of a chain of dependent agent-scope atomic adds, in
 * microseconds; and an arrival barrier of `workgroups` (2..1024) workgroups
 * on one counter, from the last arrival to the last release, in
 * microseconds. Every wait is bounded: -4 when one gave up. */
int iris_probe_handoff(uint32_t workgroups, double* round_trip_us, double* atomic_us, double* barrier_us);

/* The latency of one load a product's activation row needs, issued while
 * `flood_waves` (0-15) other waves of each CU's workgroup stream a cold
 * buffer with 16 loads per lane in flight (no counterpart in the reference;
 * a measurement): the median over one workgroup per CU of a vector load of
 * a line other workgroups read and of a scalar load, in microseconds. */
int iris_probe_row_latency(uint32_t flood_waves, double* vector_us, double* scalar_us);

/* ------------------------------------------------------------------------
 * The deterministic token loop, device-resident.
 *
 * A model holds one family's weights on the device; a session holds a KV
 * cache and runs passes over it. Together they replace the reference's
 * direct-infer executor (crates/inference/direct/src/executor.rs:41-290,
 * run_layers_and_logits :293-360, run_mistral_layers_and_logits :364-401)
 * and its per-layer kernels (crates/inference/kernels/src/mistral/layer.rs:107-318,
 * crates/inference/kernels/src/prefill_range.rs:307-958), with every layer
 * product going through the same exact Q8_0 arithmetic as
 * linear_slab_from_source (tensor.rs:437-520).
 * ---------------------------------------------------------------------- */

typedef struct IrisModel IrisModel;
typedef struct IrisSession IrisSession;

enum { IRIS_FAMILY_MISTRAL_DENSE = 0, IRIS_FAMILY_GEMMA_DENSE = 1 };

/* Shape scalars, as inference_artifacts::{MistralShape, DirectInferShape}
 * carry them (crates/inference/artifacts/src/direct.rs:241-290). Fields a
 * family does not use are ignored. */
typedef struct IrisModelDesc {
    int32_t family;
    uint32_t hidden, layers, heads, kv_heads, head_dim, ffn, vocab;
    int64_t norm_eps;               /* Q32.32 */
    uint32_t attention_scale_q32;   /* mistral-dense */
    uint32_t max_positions;         /* mistral-dense: positions from here on are refused */
    int32_t tied_head;              /* head reads the embedding table */
    /* gemma-dense */
    uint32_t global_head_dim, ple_width, sliding_window, num_kv_shared_layers;
    int64_t rope_base_sliding, rope_base_full;   /* Q32.32 */
    int32_t partial_rotary_q16;
    int32_t embedding_scale, ple_embedding_scale, ple_projection_scalar, ple_input_scale;
    int32_t final_logit_softcap;
    const uint8_t* layer_is_sliding;  /* layers entries, 1 = sliding_attention */
} IrisModelDesc;

int iris_model_create(const IrisModelDesc* desc, IrisModel** out);

/* Hands one tensor to the model under its DETWGT name
 * (crates/inference/direct/src/model.rs:489-588 naming): width 8 = Q8_0 rows
 * (rows x cols/32*34 bytes), 32 = int32 Q16.16 values (rows x cols), 64 =
 * int64 values (the mistral rotation table "rope_inverse_frequencies").
 * Matrices go to the device as soon as the set they belong to is complete. */
int iris_model_set_tensor(IrisModel* model, const char* name, int32_t width, const void* data, uint64_t rows,
                          uint64_t cols);

/* Checks every tensor arrived and finishes the upload. */
int iris_model_finalize(IrisModel* model);
void iris_model_free(IrisModel* model);
/* Device bytes held by the model's weights. */
uint64_t iris_model_device_bytes(const IrisModel* model);

/* A KV cache for positions 0..max_positions and work space for passes of up
 * to max_rows rows. max_positions is at most 65535 (-5 beyond: the
 * matrix-core attention's exact value sums stay in int32 below 2^16 keys);
 * the reference bounds a view only by the model's max_positions
 * (crates/inference/kernels/src/mistral/layer.rs:121-127). */
int iris_session_create(IrisModel* model, uint32_t max_positions, uint32_t max_rows, IrisSession** out);
void iris_session_free(IrisSession* session);

/* Greedy generation (executor.rs:143-185): one pass over the prompt rows at
 * position 0, then per token: select the first maximum, stop at an EOS id or
 * the budget, else one pass over the selected token's row. out_tokens gets up
 * to `tokens` ids and *out_count how many were produced; out_logits (nullable,
 * tokens x vocab) the logits each selection was made from. use_graph = 1
 * replays each decode pass as a captured HIP graph; it returns -7, and runs
 * nothing, while a kernel tracer is loaded in the process (see
 * iris_kernel_tracer_loaded). A model of no layers is accepted (embedding,
 * final norm, head, selection). */
int iris_session_generate(IrisSession* session, const int32_t* prompt, uint32_t prompt_len, uint32_t tokens,
                          const int32_t* eos_ids, uint32_t n_eos, int32_t* out_tokens, uint32_t* out_count,
                          int32_t* out_logits, int32_t use_graph);

/* The teacher-forced per-layer pass (the chain's layer stages,
 * crates/inference/staged/src/routines/layer_mistral.rs:80-99 ->
 * crates/inference/kernels/src/mistral/stage.rs:172-226): every layer over
 * all `count` rows at position 0, each layer's output rows written to
 * out_rows (nullable; layers x count x hidden) and hashed into out_hashes
 * (nullable; layers x 32 bytes, SHA-256 of the layer's output rows as
 * little-endian int32). */
int iris_session_layer_pass(IrisSession* session, const int32_t* ids, uint32_t count, int32_t* out_rows,
                            uint8_t* out_hashes);

/* The same chain pass over one range of a longer text: `count` rows at
 * positions start_position.. attending over the keys the session's caches
 * already hold for the positions before it (an earlier range's pass on this
 * session, or keys carried in by iris_session_write_kv), as the range stages
 * do (crates/inference/kernels/src/mistral/stage.rs:172-226,
 * crates/inference/kernels/src/prefill_range.rs:82-172). Each layer's own
 * keys stay in its cache for the next range (iris_session_read_kv returns
 * them). Returns IRIS_E_STATE when a cache lacks a position the range needs
 * (every one before start_position; for a sliding layer those in the first
 * row's window), the reference's cache-coverage refusal
 * (raster-stages/layer-mistral/src/lib.rs:889-940,
 * raster-stages/prefill-range/src/lib.rs:1237-1290). A range at position 0
 * starts the caches afresh. */
int iris_session_layer_range(IrisSession* session, const int32_t* ids, uint32_t count, uint32_t start_position,
                             int32_t* out_rows, uint8_t* out_hashes);

/* One layer's stage over one range (run_layer_stage,
 * crates/inference/kernels/src/mistral/stage.rs:172-226; gemma-dense
 * run_prefill_range_direct, crates/inference/kernels/src/prefill_range.rs:82-172):
 * in_rows (count x hidden, the layer below's output rows) at positions
 * start_position.. over the layer's cached keys; out_rows gets the layer's
 * rows and the rows' own keys join the layer's cache. gemma-dense also takes
 * the layer's PLE rows (count x ple_width, the reference's PleRow values);
 * mistral-dense passes null. Same coverage refusal as
 * iris_session_layer_range, for this layer only. Synchronous. */
int iris_session_layer_stage(IrisSession* session, uint32_t layer, const int32_t* in_rows, uint32_t count,
                             uint32_t start_position, const int32_t* ple_rows, int32_t* out_rows);

/* Writes carried keys into a layer's cache: positions pos0..pos0+count, one
 * row of kv_heads*head_dim int32 of k and of v per position (the k and v of
 * the reference's KeyRow, raster-stages/prefill-range/src/input.rs:185-189,
 * that a range inherits as prior_kv). Waits for the session's work first. */
int iris_session_write_kv(IrisSession* session, uint32_t layer, uint32_t pos0, uint32_t count, const int32_t* k,
                          const int32_t* v);

/* Copies a layer's cached keys and values of positions pos0..pos0+count to
 * host memory: k_out and v_out get one row of kv_heads*head_dim int32 per
 * position, the k and v of the reference's KeyRow
 * (raster-stages/prefill-range/src/input.rs:185-189; emitted per layer by
 * crates/inference/kernels/src/mistral/stage.rs:172-226). Waits for the
 * session's work first. */
int iris_session_read_kv(IrisSession* session, uint32_t layer, uint32_t pos0, uint32_t count, int32_t* k_out,
                         int32_t* v_out);

/* Times `steps` decode passes (graph replays) after the prompt pass and
 * reports milliseconds per decode token from HIP events on the session's
 * stream; the generated ids are written to out_tokens (nullable). */
int iris_session_time_decode(IrisSession* session, const int32_t* prompt, uint32_t prompt_len, uint32_t steps,
                             double* ms_per_token, double* prefill_ms, int32_t* out_tokens);

/* iris_session_time_decode with the decode passes issued as graph replays
 * (use_graph != 0, the same as iris_session_time_decode) or launch by launch
 * from the host (use_graph == 0: the same kernels and arguments; what a
 * kernel tracer sees without graph interception). Graph replays return -7
 * while a kernel tracer is loaded. */
int iris_session_time_decode_launches(IrisSession* session, const int32_t* prompt, uint32_t prompt_len,
                                      uint32_t steps, int use_graph, double* ms_per_token, double* prefill_ms,
                                      int32_t* out_tokens);

/* 1 when a kernel tracer (the ROCm profiler SDK, as rocprofv3 loads it, or
 * the older rocprofiler) is loaded in this process, else 0. Graph replays of
 * the decode pass are refused then: under rocprofv3 --kernel-trace they
 * ended in a segfault inside the HIP runtime with no cause shown in this
 * library. No counterpart in the reference. */
int iris_kernel_tracer_loaded(void);

/* Times one pass of every layer over `count` rows at position 0 (the
 * teacher-forced pass without downloading rows or hashing) with HIP events
 * on the session's stream. */
int iris_session_time_pass(IrisSession* session, const int32_t* ids, uint32_t count, double* ms);

/* Numerics check of the attention kernels' narrow routines, run on the
 * device over n inputs (device pointers; synchronous): exp_out[i] is the
 * softmax exp term of a logit diff[i] below its row maximum, weight_out[i]
 * the raw weight requantize(div_acc(e[i], sum[i])) for e[i] <= 2^32 <=
 * sum[i], score_out[i] the scaled score of the wrapping dot product dot[i].
 * No counterpart in the reference: it compares these routines with the
 * reference's attention_softmax_exp_term and attention_softmax_raw_weight
 * (crates/det-num/src/ops.rs:264-271) and scaled_score
 * (crates/det-num/src/mistral.rs:130-145). */
int iris_attention_numerics(const uint32_t* diff, const uint64_t* e, const uint64_t* sum, const int64_t* dot,
                            uint32_t scale_q32, uint32_t n, uint64_t* exp_out, int32_t* weight_out,
                            int32_t* score_out);

/* Numerics check: silu (crates/det-num/src/mistral.rs:59-77, the SwiGLU
 * gate) of n Q16.16 values on the device, as the product epilogues compute
 * it (device pointers; synchronous). No counterpart in the reference. */
int iris_silu_device(const int32_t* x, uint32_t n, int32_t* out);

/* Numerics check: the same silu through the device's silu table, as the
 * matrix-core SwiGLU epilogues look it up (device pointers; synchronous; the
 * table is made on the first call on a device). No counterpart in the
 * reference. */
int iris_silu_table_device(const int32_t* x, uint32_t n, int32_t* out);

/* SHA-256 (FIPS 180-4) of `len` bytes into out[32]; the hash
 * iris_session_layer_pass uses. Host code only. */
int iris_sha256_bytes(const uint8_t* data, uint64_t len, uint8_t* out);

#ifdef __cplusplus
}
#endif

#endif /* IRIS_HIP_H */
