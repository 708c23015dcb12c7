// Host side of the Q8_0 product ABI: matrix upload (raw Q8_0 rows, or the
// reference's de-interleaved weights + i64 scales), the synchronous drop-in
// product and the device-pointer product.
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "q8_internal.h"

namespace {

thread_local const char* g_error_text = nullptr;

// q8gpu_product's host round trip runs in one device arena, carved per call
// into the activations, the outputs and the MFMA work space (each region
// 256-byte aligned). The arena only grows, to the next power of two of what
// a call needs, so a run of similar products allocates once. Calls are
// serialised by the arena's lock, as the reference's global device lock
// serialises its products (gpu.rs:113-116).
struct RoundTripArena {
    std::mutex lock;
    uint8_t* base = nullptr;
    uint64_t capacity = 0;

    static uint64_t aligned(uint64_t bytes) { return (bytes + 255) & ~uint64_t(255); }

    // Points act/out/ws at regions of the asked sizes (ws null when 0).
    hipError_t carve(uint64_t act, uint64_t out, uint64_t ws, int32_t** a, int32_t** o, void** w) {
        const uint64_t need = aligned(act) + aligned(out) + aligned(ws);
        if (need > capacity) {
            uint64_t grown = 1ull << 20;
            while (grown < need) grown <<= 1;
            if (base) hipFree(base);
            base = nullptr;
            capacity = 0;
            const hipError_t st = hipMalloc((void**)&base, grown);
            if (st != hipSuccess) return st;
            capacity = grown;
        }
        *a = (int32_t*)base;
        *o = (int32_t*)(base + aligned(act));
        *w = ws ? (void*)(base + aligned(act) + aligned(out)) : nullptr;
        return hipSuccess;
    }
};
RoundTripArena g_round_trip;

// Work space of a multi-token product: 5 digit planes of the activations
// (256-byte aligned), then one digit count and one norm scale per token.
uint64_t planes_bytes(uint32_t cols, uint32_t tokens) { return gemm_planes_bytes(cols, tokens); }

Q8GpuMatrix* alloc_matrix(uint32_t rows, uint32_t cols) {
    Q8GpuMatrix* m = (Q8GpuMatrix*)std::calloc(1, sizeof(Q8GpuMatrix));
    if (!m) return nullptr;
    m->rows = rows;
    m->cols = cols;
    m->nb = cols / 32;
    m->tiles = (rows + Q8_TILE_ROWS - 1) / Q8_TILE_ROWS;
    return m;
}

// f16 bits whose exact Q.24 value is s, or -1 when no finite f16 has it.
int f16_bits_of_q24(int64_t s) {
    uint64_t mag = s < 0 ? (uint64_t)0 - (uint64_t)s : (uint64_t)s;
    uint32_t sign = s < 0 ? 0x8000u : 0;
    if (mag < 1024) return (int)(sign | (uint32_t)mag);  // subnormal (and zero)
    int top = 63 - __builtin_clzll(mag);                 // 2^top <= mag
    int e = top - 10;                                    // mag = M << e, M in [1024, 2047]
    if (e > 29) return -1;
    if (mag & ((1ull << e) - 1)) return -1;
    uint32_t mant = (uint32_t)(mag >> e) - 1024;
    return (int)(sign | ((uint32_t)(e + 1) << 10) | mant);
}

// The no-allocation product's work space: one array per device, holding the
// digit planes and per-token digit counts of one multi-token product. In host
// code `scratch` only names the symbol; its device address on each device
// comes from hipGetSymbolAddress, resolved once per device (q8gpu_init for
// the current device, else the entry point's first call there) and kept in
// g_scratch_dev, which is all host code ever passes on.
__device__ __align__(256) uint8_t scratch[IRIS_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_lock;
uint8_t* g_scratch_dev[MAX_DEVICES] = {};

int scratch_for_current_device(uint8_t** out) {
    int dev = 0;
    hipError_t st = hipGetDevice(&dev);
    if (st != hipSuccess) return (int)st;
    if (dev < 0 || dev >= MAX_DEVICES) return IRIS_E_INVALID;
    std::lock_guard<std::mutex> guard(g_scratch_lock);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        st = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (st != hipSuccess) return (int)st;
        if (!p) return IRIS_E_STATE;
        g_scratch_dev[dev] = (uint8_t*)p;
    }
    *out = g_scratch_dev[dev];
    return 0;
}

}  // namespace

void iris_set_error_text(const char* text) { g_error_text = text; }

int iris_q8_upload_parts(const uint8_t* const* parts, const uint32_t* part_rows, int nparts, uint32_t cols,
                         int interleave, Q8GpuMatrix** out, hipStream_t stream) {
    *out = nullptr;
    if (nparts <= 0 || cols == 0 || cols % 32) return IRIS_E_INVALID;
    uint32_t rows = 0;
    for (int i = 0; i < nparts; i++) rows += part_rows[i];
    if (rows == 0) return IRIS_E_INVALID;
    if (interleave && (nparts != 2 || part_rows[0] != part_rows[1])) return IRIS_E_INVALID;
    Q8GpuMatrix* m = alloc_matrix(rows, cols);
    if (!m) return IRIS_E_NOMEM;
    const size_t row_bytes = (size_t)m->nb * 34;
    const size_t raw_bytes = (size_t)rows * row_bytes;
    const size_t qs_bytes = (size_t)m->tiles * m->nb * Q8_TILE_BLOCK_BYTES;
    const size_t sc_bytes = (size_t)m->tiles * m->nb * Q8_TILE_ROWS * sizeof(uint16_t);
    const size_t rs_bytes = (size_t)m->tiles * Q8_TILE_ROWS * sizeof(int64_t);
    uint8_t* d_raw = nullptr;
    hipError_t st = hipMalloc((void**)&m->qs, qs_bytes);
    if (st == hipSuccess) st = hipMalloc((void**)&m->sc16, sc_bytes);
    if (st == hipSuccess) st = hipMalloc((void**)&m->row_scale, rs_bytes);
    if (st == hipSuccess) st = hipMalloc((void**)&d_raw, raw_bytes);
    // Padding rows of the last tile hold zero weights and zero scales.
    if (st == hipSuccess) st = hipMemsetAsync(m->qs, 0, qs_bytes, stream);
    if (st == hipSuccess) st = hipMemsetAsync(m->sc16, 0, sc_bytes, stream);
    if (st == hipSuccess) st = hipMemsetAsync(m->row_scale, 0, rs_bytes, stream);
    size_t off = 0;
    for (int i = 0; i < nparts && st == hipSuccess; i++) {
        st = hipMemcpyAsync(d_raw + off, parts[i], (size_t)part_rows[i] * row_bytes, hipMemcpyHostToDevice, stream);
        off += (size_t)part_rows[i] * row_bytes;
    }
    int rc = (int)st;
    if (rc == 0) rc = iris_q8_pack_device(d_raw, m, stream, interleave ? part_rows[0] : 0);
    hipFree(d_raw);
    if (rc != 0) {
        if (rc == IRIS_E_SCALE) iris_set_error_text("Q8_0 block scale is not finite");
        q8gpu_free(m);
        return rc;
    }
    if (m->scale_mode == Q8_SCALE_ROW) {
        hipFree(m->sc16);
        m->sc16 = nullptr;
        m->device_bytes = qs_bytes + rs_bytes;
    } else {
        hipFree(m->row_scale);
        m->row_scale = nullptr;
        m->device_bytes = qs_bytes + sc_bytes;
    }
    *out = m;
    return 0;
}

int iris_q8_upload_raw(const uint8_t* host_raw, uint32_t rows, uint32_t cols, Q8GpuMatrix** out,
                       hipStream_t stream) {
    return iris_q8_upload_parts(&host_raw, &rows, 1, cols, 0, out, stream);
}

extern "C" {

const char* q8gpu_error(int code) {
    switch (code) {
        case IRIS_E_INVALID: return "invalid argument or shape";
        case IRIS_E_SCALE: return "Q8_0 block scale is not finite";
        case IRIS_E_NOMEM: return "host allocation failed";
        case IRIS_E_STATE: return "call made in the wrong state";
        case IRIS_E_RANGE: return "position or size past what the object was built for";
        case IRIS_E_SCRATCH: return "work space needed exceeds the no-allocation scratch (IRIS_NOALLOC_SCRATCH_BYTES)";
        case IRIS_E_TRACED:
            return "graph replays are not run while a kernel tracer is loaded; decode launch by launch (use_graph = 0)";
        default: break;
    }
    if (code < 0) return g_error_text ? g_error_text : "unknown library error";
    return hipGetErrorString((hipError_t)code);
}

int q8gpu_init(void) {
    void* probe = nullptr;
    hipError_t st = hipMalloc(&probe, 1 << 20);
    if (st != hipSuccess) return (int)st;
    iris_gemv_prepare();
    st = hipFree(probe);
    if (st != hipSuccess) return (int)st;
    uint8_t* ws = nullptr;
    return scratch_for_current_device(&ws);
}

void q8gpu_free(Q8GpuMatrix* m) {
    if (!m) return;
    hipFree(m->qs);
    hipFree(m->sc16);
    hipFree(m->sc64);
    hipFree(m->row_scale);
    hipFree(m->fold.planes);
    hipFree(m->fold.shift);
    std::free(m);
}

int q8gpu_upload_q8_0(const uint8_t* blocks, uint32_t rows, uint32_t cols, Q8GpuMatrix** out) {
    if (!out) return IRIS_E_INVALID;
    int rc = iris_q8_upload_raw(blocks, rows, cols, out, nullptr);
    if (rc == 0) rc = (int)hipStreamSynchronize(nullptr);
    return rc;
}

int q8gpu_upload(const int8_t* weights, const int64_t* scales, uint32_t rows, uint32_t cols,
                 Q8GpuMatrix** out_matrix) {
    if (!out_matrix) return IRIS_E_INVALID;
    *out_matrix = nullptr;
    if (rows == 0 || cols == 0 || cols % 32) return IRIS_E_INVALID;
    const uint32_t nb = cols / 32;
    const size_t blocks = (size_t)rows * nb;
    // Scales that are exact f16 values travel as Q8_0 rows; anything else
    // keeps one i64 per block.
    bool f16_ok = true;
    for (size_t i = 0; i < blocks && f16_ok; i++) f16_ok = f16_bits_of_q24(scales[i]) >= 0;
    if (f16_ok) {
        std::vector<uint8_t> raw;
        try {
            raw.resize(blocks * 34);
        } catch (...) {
            return IRIS_E_NOMEM;
        }
        for (size_t i = 0; i < blocks; i++) {
            const int bits = f16_bits_of_q24(scales[i]);
            raw[i * 34] = (uint8_t)(bits & 0xff);
            raw[i * 34 + 1] = (uint8_t)(bits >> 8);
            std::memcpy(&raw[i * 34 + 2], weights + i * 32, 32);
        }
        return q8gpu_upload_q8_0(raw.data(), rows, cols, out_matrix);
    }
    Q8GpuMatrix* m = alloc_matrix(rows, cols);
    if (!m) return IRIS_E_NOMEM;
    m->scale_mode = Q8_SCALE_I64;
    const size_t qs_bytes = (size_t)m->tiles * nb * Q8_TILE_BLOCK_BYTES;
    const size_t sc_bytes = (size_t)m->tiles * nb * Q8_TILE_ROWS * sizeof(int64_t);
    std::vector<uint8_t> qs;
    std::vector<int64_t> sc;
    try {
        qs.assign(qs_bytes, 0);
        sc.assign(sc_bytes / sizeof(int64_t), 0);
    } catch (...) {
        std::free(m);
        return IRIS_E_NOMEM;
    }
    for (uint32_t row = 0; row < rows; row++) {
        const uint32_t tile = row / Q8_TILE_ROWS, r = row % Q8_TILE_ROWS;
        for (uint32_t b = 0; b < nb; b++) {
            uint8_t* dst = &qs[((size_t)tile * nb + b) * Q8_TILE_BLOCK_BYTES + r * 16];
            const int8_t* src = weights + (size_t)row * cols + (size_t)b * 32;
            std::memcpy(dst, src, 16);
            std::memcpy(dst + 256, src + 16, 16);
            sc[((size_t)tile * nb + b) * Q8_TILE_ROWS + r] = scales[(size_t)row * nb + b];
        }
    }
    hipError_t st = hipMalloc((void**)&m->qs, qs_bytes);
    if (st == hipSuccess) st = hipMalloc((void**)&m->sc64, sc_bytes);
    if (st == hipSuccess) st = hipMemcpy(m->qs, qs.data(), qs_bytes, hipMemcpyHostToDevice);
    if (st == hipSuccess) st = hipMemcpy(m->sc64, sc.data(), sc_bytes, hipMemcpyHostToDevice);
    if (st != hipSuccess) {
        q8gpu_free(m);
        return (int)st;
    }
    m->device_bytes = qs_bytes + sc_bytes;
    *out_matrix = m;
    return 0;
}

int q8gpu_product_device(const Q8GpuMatrix* m, const int32_t* d_act, uint32_t tokens, int32_t* d_out,
                         void* stream) {
    return q8gpu_product_device_ws(m, d_act, tokens, d_out, nullptr, 0, stream);
}

uint64_t q8gpu_workspace_bytes(const Q8GpuMatrix* m, uint32_t tokens) {
    if (!m || tokens < 2) return 0;
    return planes_bytes(m->cols, tokens) + 4ull * gemm_limb_ints(m->cols, tokens);
}

}  // extern "C"

// The product with optional work space. A per-block scale matrix takes the
// matrix cores only once q8gpu_prepare_matrix_cores has folded it; nothing
// here allocates, synchronises or changes the matrix.
static int product_with_space(const Q8GpuMatrix* m, const int32_t* d_act, uint32_t tokens, int32_t* d_out,
                              void* d_workspace, uint64_t workspace_bytes, void* stream) {
    if (!m || (tokens && (!d_act || !d_out))) return IRIS_E_INVALID;
    GemvArgs a{};
    a.w = q8_view(m);
    a.x = d_act;
    a.x_stride = m->cols;
    a.tokens = tokens;
    a.prologue = PRO_NONE;
    a.epilogue = EPI_STORE;
    a.out = d_out;
    a.out_stride = m->rows;
    if (d_workspace && tokens >= 2) {
        if (workspace_bytes < q8gpu_workspace_bytes(m, tokens)) return IRIS_E_RANGE;
        a.planes = (int8_t*)d_workspace;
        a.token_limbs = (int32_t*)((char*)d_workspace + planes_bytes(m->cols, tokens));
    }
    return iris_gemv_launch(a, (hipStream_t)stream);
}

extern "C" {

int q8gpu_product_device_ws(const Q8GpuMatrix* m, const int32_t* d_act, uint32_t tokens, int32_t* d_out,
                            void* d_workspace, uint64_t workspace_bytes, void* stream) {
    return product_with_space(m, d_act, tokens, d_out, d_workspace, workspace_bytes, stream);
}

int q8gpu_prepare_matrix_cores(Q8GpuMatrix* m, void* stream) {
    if (!m) return IRIS_E_INVALID;
    return iris_q8_prepare_fold(m, (hipStream_t)stream);
}

// q8gpu_product_device_ws with the device's scratch array as the work space:
// no allocation of any kind. The digit counts are reset per token and every
// plane of the used region is written by the call itself before it is read,
// so nothing carried over from an earlier call is used.
int q8gpu_product_device_noalloc(const Q8GpuMatrix* m, const int32_t* d_act, uint32_t tokens, int32_t* d_out,
                                 void* stream) {
    if (!m || (tokens && (!d_act || !d_out))) return IRIS_E_INVALID;
    const uint64_t need = q8gpu_workspace_bytes(m, tokens);
    if (need == 0) return q8gpu_product_device_ws(m, d_act, tokens, d_out, nullptr, 0, stream);
    if (need > IRIS_NOALLOC_SCRATCH_BYTES) return IRIS_E_SCRATCH;
    uint8_t* ws = nullptr;
    const int rc = scratch_for_current_device(&ws);
    if (rc != 0) return rc;
    return product_with_space(m, d_act, tokens, d_out, ws, IRIS_NOALLOC_SCRATCH_BYTES, stream);
}

int q8gpu_product(const Q8GpuMatrix* m, const int32_t* activations, uint32_t tokens, int32_t* out) {
    if (!m || (tokens && (!activations || !out))) return IRIS_E_INVALID;
    if (tokens == 0) return 0;
    std::lock_guard<std::mutex> guard(g_round_trip.lock);
    const size_t act_bytes = (size_t)tokens * m->cols * sizeof(int32_t);
    const size_t out_bytes = (size_t)tokens * m->rows * sizeof(int32_t);
    const size_t ws_bytes = q8gpu_workspace_bytes(m, tokens);
    int32_t *d_act = nullptr, *d_out = nullptr;
    void* d_ws = nullptr;
    hipError_t st = g_round_trip.carve(act_bytes, out_bytes, ws_bytes, &d_act, &d_out, &d_ws);
    if (st == hipSuccess) st = hipMemcpy(d_act, activations, act_bytes, hipMemcpyHostToDevice);
    if (st != hipSuccess) return (int)st;
    int rc = q8gpu_product_device_ws(m, d_act, tokens, d_out, d_ws, ws_bytes, nullptr);
    if (rc != 0) return rc;
    st = hipMemcpy(out, d_out, out_bytes, hipMemcpyDeviceToHost);
    return (int)st;
}

int q8gpu_matrix_info(const Q8GpuMatrix* m, uint32_t* rows, uint32_t* cols, int* scale_mode, uint64_t* bytes) {
    if (!m) return IRIS_E_INVALID;
    if (rows) *rows = m->rows;
    if (cols) *cols = m->cols;
    if (scale_mode) *scale_mode = m->scale_mode;
    if (bytes) *bytes = m->device_bytes;
    return 0;
}

int q8gpu_synchronize(void) { return (int)hipDeviceSynchronize(); }

int iris_device_malloc(uint64_t bytes, void** out) {
    if (!out) return IRIS_E_INVALID;
    return (int)hipMalloc(out, bytes ? bytes : 1);
}

int iris_device_free(void* ptr) { return (int)hipFree(ptr); }

int iris_memcpy_h2d(void* dst, const void* src, uint64_t bytes) {
    return (int)hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
}

int iris_memcpy_d2h(void* dst, const void* src, uint64_t bytes) {
    return (int)hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
}

int iris_memcpy_d2d(void* dst, const void* src, uint64_t bytes) {
    return (int)hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice);
}

int iris_time_product(const Q8GpuMatrix* const* ms, uint32_t count, const int32_t* d_act, uint32_t tokens,
                      int32_t* d_out, uint32_t iterations, double* ms_per_product) {
    if (!ms || count == 0 || !ms_per_product || iterations == 0) return IRIS_E_INVALID;
    for (uint32_t i = 0; i < count; i++)
        if (!ms[i] || ms[i]->rows != ms[0]->rows || ms[i]->cols != ms[0]->cols) return IRIS_E_INVALID;
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t st = hipStreamCreate(&s);
    if (st == hipSuccess) st = hipEventCreate(&e0);
    if (st == hipSuccess) st = hipEventCreate(&e1);
    int rc = (int)st;
    for (uint32_t i = 0; rc == 0 && i < count; i++) rc = q8gpu_product_device(ms[i], d_act, tokens, d_out, s);
    if (rc == 0) rc = (int)hipEventRecord(e0, s);
    for (uint32_t i = 0; rc == 0 && i < iterations; i++)
        rc = q8gpu_product_device(ms[i % count], d_act, tokens, d_out, s);
    if (rc == 0) rc = (int)hipEventRecord(e1, s);
    if (rc == 0) rc = (int)hipEventSynchronize(e1);
    float elapsed = 0.f;
    if (rc == 0) rc = (int)hipEventElapsedTime(&elapsed, e0, e1);
    if (rc == 0) *ms_per_product = (double)elapsed / iterations;
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    if (s) hipStreamDestroy(s);
    return rc;
}

int iris_time_product_ws(const Q8GpuMatrix* m, const int32_t* d_act, uint32_t tokens, int32_t* d_out,
                         void* d_workspace, uint64_t workspace_bytes, uint32_t iterations, double* ms_per_product) {
    if (!m || !ms_per_product || iterations == 0) return IRIS_E_INVALID;
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t st = hipStreamCreate(&s);
    if (st == hipSuccess) st = hipEventCreate(&e0);
    if (st == hipSuccess) st = hipEventCreate(&e1);
    int rc = (int)st;
    if (rc == 0) rc = q8gpu_product_device_ws(m, d_act, tokens, d_out, d_workspace, workspace_bytes, s);
    if (rc == 0) rc = (int)hipEventRecord(e0, s);
    for (uint32_t i = 0; rc == 0 && i < iterations; i++)
        rc = q8gpu_product_device_ws(m, d_act, tokens, d_out, d_workspace, workspace_bytes, s);
    if (rc == 0) rc = (int)hipEventRecord(e1, s);
    if (rc == 0) rc = (int)hipEventSynchronize(e1);
    float elapsed = 0.f;
    if (rc == 0) rc = (int)hipEventElapsedTime(&elapsed, e0, e1);
    if (rc == 0) *ms_per_product = (double)elapsed / iterations;
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    if (s) hipStreamDestroy(s);
    return rc;
}

}  // extern "C"
