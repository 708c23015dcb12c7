// Internal declarations shared by the HIP sources of libiris_hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/iris_hip.h"

// Library-defined error codes (negative, distinct from hipError_t values).
enum {
    IRIS_E_INVALID = -1,      // a shape or argument the call does not accept
    IRIS_E_SCALE = -2,        // a Q8_0 block scale that is not finite
    IRIS_E_NOMEM = -3,        // host allocation failed
    IRIS_E_STATE = -4,        // call made in the wrong state (e.g. before finalize)
    IRIS_E_RANGE = -5,        // position or size past what the object was built for
    IRIS_E_SCRATCH = -6,      // work space needed exceeds the no-allocation scratch
    IRIS_E_TRACED = -7,       // graph replays asked for while a kernel tracer is loaded
};

// Scale layouts of a device Q8_0 matrix.
enum Q8ScaleMode : int {
    Q8_SCALE_ROW = 0,  // every block of a row shares one scale: one i64 Q.24 per row
    Q8_SCALE_F16 = 1,  // one f16 per block (the reference's encoding)
    Q8_SCALE_I64 = 2,  // one arbitrary i64 Q.24 per block (q8gpu_upload's input)
};

// Rows per tile and the tiled byte layout:
//   qs : [tiles][nb][2 halves][16 rows][16 bytes]   (512 B per tile-block)
//   sc16 / sc64 : [tiles][nb][16 rows]
//   row_scale : [tiles * 16]
constexpr int Q8_TILE_ROWS = 16;
constexpr int Q8_TILE_BLOCK_BYTES = 512;

// Per-block f16 scales folded into the weights for the matrix cores: with
// s_b = sign_b * m_b * 2^sh_b the Q.24 value of block b's scale (m_b < 2^11)
// and R the least sh_b of the row, the integers w' = q * sign_b * (m_b <<
// (sh_b - R)) give dot_row's total as 2^R * sum_k w'_k x_k. Each w' is kept
// as `planes` signed byte digits (the activations' digit scheme), each
// plane in the qs tile layout; `shift` holds R per row.
struct Q8Folded {
    int8_t* planes;    // [planes][tiles][nb][512]
    int32_t* shift;    // [tiles * 16]
    uint32_t nplanes;  // 0 = not prepared
};

// Weight digit planes of a folded matrix, at most: the widest spread of a
// row's f16 scales (a subnormal block beside exponent 30, 29 binary orders)
// makes |w'| <= 127 * 2047 * 2^29 < 2^47, six signed byte digits, so every
// matrix with finite scales folds.
constexpr uint32_t Q8_FOLD_MAX_PLANES = 6;

struct Q8GpuMatrix {
    uint32_t rows, cols, nb, tiles;
    int scale_mode;
    uint8_t* qs;
    uint16_t* sc16;
    int64_t* sc64;
    int64_t* row_scale;
    uint64_t device_bytes;
    Q8Folded fold;
    bool fold_tried;  // the folding was attempted (prepared or refused)
};

// Kernel-side view of a matrix.
struct Q8View {
    const uint8_t* qs;
    const uint16_t* sc16;
    const int64_t* sc64;
    const int64_t* row_scale;
    uint32_t rows, cols, nb, tiles;
    int scale_mode;
    const int8_t* fold_planes;
    const int32_t* fold_shift;
    uint32_t fold_nplanes;
};

inline Q8View q8_view(const Q8GpuMatrix* m) {
    return Q8View{m->qs,   m->sc16,       m->sc64,       m->row_scale,      m->rows,        m->cols,
                  m->nb,   m->tiles,      m->scale_mode, m->fold.planes,    m->fold.shift,  m->fold.nplanes};
}

// Builds m's folded planes (once; per-block scale matrices only) so that
// multi-token products of it run on the matrix cores. Allocates device
// memory (one byte per weight per digit plane, 1 to Q8_FOLD_MAX_PLANES).
int iris_q8_prepare_fold(Q8GpuMatrix* m, hipStream_t stream);

// Prologue applied to the activations while they are staged.
enum GemvPrologue : int {
    PRO_NONE = 0,
    PRO_RMSNORM = 1,  // rms_norm(x, norm_w, eps) (ops.rs:98-114), computed per workgroup
    // One row (gemma-dense's post-norm, residual and layer scalar, then the
    // next norm, prefill_range.rs:879-958): y = add_sat(rms_norm(x,
    // res_norm_w), res_in), times res_scalar when set; the product takes
    // rms_norm(y, norm_w). The first norm's sum of squares comes from the
    // producer's tile slots (ssq_in); workgroup 0 writes y to res_out
    // (nullable).
    PRO_NORM_RES_NORM = 2,
};

// Epilogue applied to each finished output.
enum GemvEpilogue : int {
    EPI_STORE = 0,     // out = value
    EPI_RESIDUAL = 1,  // out = add_sat(value, residual)
    EPI_SOFTCAP = 2,   // out = softcap(value, cap) (cap <= 0 passes through)
    EPI_SWIGLU = 3,    // rows interleave gate/up: out[row/2] = mul(silu(gate), up)
    EPI_GEGLU = 4,     // rows interleave gate/up: out[row/2] = mul(gelu(gate), up)
    EPI_ROPE_KV = 5,   // rows q|k|v: rotate q and k pairs at the token's position
                       // (mistral consecutive pairs), q -> out, k/v -> caches
    EPI_HEAD_SELECT = 6,  // logits = softcap(value) and each tile's first maximum
                          // to sel_partial, for iris_select_launch
};

struct GemvArgs {
    Q8View w;
    const int32_t* x;
    uint32_t x_stride;
    uint32_t tokens;
    int prologue;
    const int32_t* norm_w;
    int64_t norm_eps;
    int epilogue;
    int32_t* out;
    uint32_t out_stride;
    const int32_t* residual;
    uint32_t residual_stride;
    int32_t softcap;
    // EPI_ROPE_KV
    const int32_t* d_pos;       // absolute position of token 0 of this launch
    const int64_t* inv_freq;    // head_dim/2 Q32.32 angles per position
    const int64_t* rope_sc;     // nullable: [tokens][head_dim/2][sin, cos] Q30 for these positions
    uint32_t head_dim, q_rows, kv_rows;
    int32_t* k_cache;           // transposed: [kv_rows][k_pos_stride]
    uint32_t k_pos_stride;
    int32_t* v_cache;           // [position][kv_rows]
    // EPI_HEAD_SELECT
    int32_t* logits_keep;       // [steps][rows] or null
    int32_t* d_step;
    int32_t* d_pos_rw;
    uint32_t rows_in_pass;
    int32_t* tokens_out;        // [steps]
    const uint8_t* embed_raw;   // Q8_0 rows, reference layout
    uint32_t embed_row_bytes, hidden;
    int32_t embed_scale;        // Q16.16 multiplier of the embedded row (1.0 for mistral-dense)
    int32_t* x_next;            // [hidden]
    int32_t* ids_next;          // nullable: the selected id is also stored here
    uint64_t* sel_partial;      // [tiles]: (index << 32) | (uint32)value of each tile's first maximum
    int64_t* rope_next;         // nullable: the next one-row pass's RoPE (sin, cos) pairs, [rope_half][2]
    uint32_t rope_half;         // pairs per position (head_dim / 2)
    // Multi-token products of row-scale matrices go through the int8 MFMA
    // GEMM when this work space is given (null: the GEMV path).
    int8_t* planes;             // gemm_planes_bytes(cols, tokens): 5 digit planes, MFMA-operand tiled
    int32_t* token_limbs;       // gemm_limb_ints(cols, tokens): each token's rms_norm scale, then the digits
                                // each (k chunk, 32-token tile) of the activations needs, [chunk][tile]
    // One-token launches only. ssq_out (EPI_RESIDUAL or EPI_STORE): each
    // tile's saturating sum of the squares of its outputs, slot [tile].
    // ssq_in (PRO_RMSNORM, PRO_NORM_RES_NORM: the first norm):
    // such slots of the row being normed, ssq_n of them (at most
    // GEMV_SSQ_SLOTS): the norm's sum of squares is their saturating sum
    // (non-negative terms: the same in any grouping), so the workgroups skip
    // their own reduction. Null: not used.
    int64_t* ssq_out;
    const int64_t* ssq_in;
    uint32_t ssq_n;
    // PRO_NORM_RES_NORM
    const int32_t* res_norm_w;
    const int32_t* res_in;
    int32_t res_scalar;         // 0 = none
    int32_t* res_out;
    // EPI_SWIGLU of the matrix-core products: the device's silu table
    // (iris_silu_table); null computes each silu.
    const int32_t* silu_tab;
    // One-token products whose input row comes as digit planes written by
    // its producer (ActPlanes layout; PRO_NONE, row scales, EPI_RESIDUAL or
    // EPI_STORE): the row's planes and digit counts, and the k split's
    // scratch, partial sums [BCAST_MAX_PARTS][rows] and arrival counters
    // [bcast_groups(rows)] (zero at allocation; each launch leaves them
    // zero). Null x_planes: the row is staged from x.
    const uint32_t* x_planes;
    const uint8_t* x_counts;
    int64_t* kpart;
    uint32_t* kcount;
    // One-token EPI_SWIGLU / EPI_GEGLU launches: the outputs' digit planes
    // too (ActPlanes layout over out's row; null: not written).
    uint32_t* out_planes;
    uint8_t* out_counts;
    // Multi-token EPI_SWIGLU / EPI_GEGLU products on the matrix cores: the
    // gated rows also as the next product's digit planes (the `planes`
    // layout over rows / 2 columns, gemm_planes_bytes) and the digits each
    // (k chunk, 32-token tile) needs (the `token_limbs` layout after the
    // first `tokens` ints; the launcher sets them to 1 first). Null: not
    // written. With them, `out` may be null: the gated rows are then kept
    // only as planes.
    int8_t* out_gemm_planes;
    int32_t* out_gemm_limbs;
    // Multi-token PRO_NONE products whose planes and counts are already in
    // planes / token_limbs (their producer wrote them): no preparation.
    int planes_ready;
};

// A row of int32 values as the broadcast products read it: plane l (of
// ACT_PLANES) holds dword i = the signed byte digits l of values 4i..4i+3
// (balanced base 256, digits5), at planes[l * cols/4 + i]; counts[j] holds
// the digits values 8j..8j+7 need (1-5), so a 32-value block's four counts
// are one dword. cols % 32 == 0.
constexpr uint32_t ACT_PLANES = 5;  // signed byte digits of an int32
inline uint64_t act_planes_dwords(uint32_t cols) { return (uint64_t)ACT_PLANES * cols / 4; }
inline uint64_t act_counts_bytes(uint32_t cols) { return cols / 8; }
// The broadcast products' workgroups: four 16-row tiles (64 rows) times up
// to BCAST_MAX_PARTS slices of the row.
constexpr uint32_t BCAST_MAX_PARTS = 4;
inline uint32_t bcast_groups(uint32_t rows) { return (rows + 63) / 64; }
int iris_gemv_bcast_launch(const GemvArgs& a, hipStream_t stream);
bool iris_gemv_bcast_applies(const GemvArgs& a);

constexpr uint32_t GEMV_SSQ_SLOTS = 256;

// Barrier for LDS traffic only: global loads still in flight (a prefetch)
// stay in flight, where __syncthreads would wait for every one of them.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Bytes of the MFMA product's digit planes: 5 planes of the tokens rounded
// up to whole 32-token tiles, times cols, 256-byte aligned.
inline uint64_t gemm_planes_bytes(uint32_t cols, uint32_t tokens) {
    return (5ull * ((tokens + 31ull) & ~31ull) * cols + 255) & ~255ull;
}

constexpr uint32_t GEMM_PLANE_KB = 8;  // 32-wide k blocks per digit-plane workgroup (one k chunk)

// The ints of token_limbs a multi-token product uses: one rms_norm scale per
// token, then one digit count per (k chunk, 32-token tile).
inline uint64_t gemm_limb_ints(uint32_t cols, uint32_t tokens) {
    const uint64_t chunks = ((uint64_t)cols / 32 + GEMM_PLANE_KB - 1) / GEMM_PLANE_KB;
    return tokens + chunks * ((tokens + 31ull) / 32);
}

// The MFMA GEMM for a multi-token product (row-scale matrix, planes set);
// returns IRIS_E_INVALID when the launch does not qualify.
int iris_gemm_launch(const GemvArgs& a, hipStream_t stream);
bool iris_gemm_applies(const GemvArgs& a);

// After an EPI_HEAD_SELECT product with the same arguments: selects the first
// maximum over the tile partials, writes the token, embeds it as the next
// row and advances step and position.
int iris_select_launch(const GemvArgs& a, hipStream_t stream);

// Launches the exact Q8_0 product out[t][r] = dot_row(x[t], W[r]) (with the
// prologue/epilogue) on `stream`. Returns a hipError_t value.
int iris_gemv_launch(const GemvArgs& a, hipStream_t stream);
// Reads the device's CU count and raises the product kernels' LDS limit;
// called before any launch can be captured into a graph.
void iris_gemv_prepare();
// Compute units of the current device (queried once).
int iris_device_cus();

// Packs raw Q8_0 rows (device memory, reference layout) into m's tiled layout
// and fills its scales; `m` must have its buffers allocated for `mode`.
int iris_q8_pack_device(const uint8_t* d_raw, Q8GpuMatrix* m, hipStream_t stream, uint32_t interleave_half = 0);

// Allocates a matrix from raw Q8_0 bytes in host memory (34-byte blocks).
int iris_q8_upload_raw(const uint8_t* host_raw, uint32_t rows, uint32_t cols, Q8GpuMatrix** out,
                       hipStream_t stream);

// Allocates one matrix from several row-blocks of raw Q8_0 bytes, stacked in
// order; with `interleave` (two parts of equal rows) device row 2i is part
// 0's row i and row 2i+1 part 1's row i.
int iris_q8_upload_parts(const uint8_t* const* parts, const uint32_t* part_rows, int nparts, uint32_t cols,
                         int interleave, Q8GpuMatrix** out, hipStream_t stream);

// Thread-local last-error text for library-defined codes.
void iris_set_error_text(const char* text);
