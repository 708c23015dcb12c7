// Measured peaks of the part, reported beside the vendor figures: the HBM
// read rate of a plain streaming kernel, and the int8 matrix-core rate of a
// loop of independent v_mfma_i32_32x32x32_i8 on constant or on changing
// random operands (the matrix cores' clock falls under switching
// operands, so the second is the ceiling the exact products can meet).
#include <algorithm>
#include <vector>

#include "q8_internal.h"

namespace {

constexpr uint32_t STREAM_THREADS = 256;
constexpr uint32_t STREAM_UNROLL = 4;  // 16-byte loads in flight per thread

// Every thread reads 16-byte words at a grid stride, STREAM_UNROLL at a
// time, and folds them with xor; one word per workgroup is written only if
// the fold hits a value no real buffer gives, so the loads are not dead.
__global__ __launch_bounds__(STREAM_THREADS) void stream_read_kernel(const uint4* buf, uint64_t words, uint32_t* out) {
    const uint64_t stride = (uint64_t)gridDim.x * STREAM_THREADS;
    uint32_t acc = 0;
    uint64_t i = (uint64_t)blockIdx.x * STREAM_THREADS + threadIdx.x;
    for (; i + (STREAM_UNROLL - 1) * stride < words; i += STREAM_UNROLL * stride) {
        uint4 v[STREAM_UNROLL];
#pragma unroll
        for (uint32_t u = 0; u < STREAM_UNROLL; u++) v[u] = buf[i + u * stride];
#pragma unroll
        for (uint32_t u = 0; u < STREAM_UNROLL; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < words; i += stride) {
        const uint4 v = buf[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u) out[blockIdx.x] = acc;
}

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr uint32_t MFMA_CHAINS = 4;  // independent accumulators per wave
constexpr uint32_t MFMA_ROT = 4;     // operand pairs cycled (random operands)
constexpr uint32_t MFMA_OPS = 2 * 32 * 32 * 32;

__device__ __forceinline__ uint32_t mix32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    return x ^ (x >> 16);
}

// `rounds` x MFMA_ROT rounds of MFMA_CHAINS independent 32x32x32 int8
// MFMAs per wave. RANDOM: MFMA_ROT operand pairs of random bytes, cycled
// (the unrolled rotation keeps the indexing static), so the operands change
// every instruction; else one constant pair.
template <bool RANDOM>
__global__ __launch_bounds__(256) void mfma_i8_kernel(uint32_t rounds, uint32_t* out) {
    const uint32_t seed = (blockIdx.x * 256 + threadIdx.x) * 0x9E3779B9u;
    v4i a[MFMA_ROT], b[MFMA_ROT];
#pragma unroll
    for (uint32_t k = 0; k < MFMA_ROT; k++)
#pragma unroll
        for (int c = 0; c < 4; c++) {
            a[k][c] = RANDOM ? (int)mix32(seed + 8 * k + c) : 0x01020304;
            b[k][c] = RANDOM ? (int)mix32(seed + 8 * k + 4 + c + 0x5bd1e995u) : 0x05060708;
        }
    v16i acc[MFMA_CHAINS];
#pragma unroll
    for (uint32_t c = 0; c < MFMA_CHAINS; c++) acc[c] = v16i{};
    for (uint32_t it = 0; it < rounds; it++) {
#pragma unroll
        for (uint32_t r = 0; r < MFMA_ROT; r++)
#pragma unroll
            for (uint32_t c = 0; c < MFMA_CHAINS; c++)
                acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[(r + c) % MFMA_ROT], b[(r + 2 * c + 1) % MFMA_ROT],
                                                               acc[c], 0, 0, 0);
    }
    int s = 0;
#pragma unroll
    for (uint32_t c = 0; c < MFMA_CHAINS; c++)
#pragma unroll
        for (int e = 0; e < 16; e++) s ^= acc[c][e];
    if ((uint32_t)s == 0x9E3779B9u) out[blockIdx.x] = (uint32_t)s;
}

// ---- Handoffs between workgroups ----
// Every wait polls at most HANDOFF_SPIN times (each poll a memory round
// trip) and then gives up, setting err, so every workgroup ends. Times come
// from s_memrealtime, a device-wide 100 MHz counter (10 ns per tick).
constexpr uint32_t HANDOFF_SPIN = 1u << 20;

__device__ __forceinline__ uint32_t poll(uint32_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void post(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroups 0 and 1 (dealt to different XCDs) pass a flag back and forth
// `rounds` times through agent-scope atomic stores and loads: flags[0] from
// workgroup 0, flags[32] (another cache line) from workgroup 1. out[0..1]:
// workgroup 0's first and last tick.
__global__ void handoff_pingpong_kernel(uint32_t* flags, uint64_t* out, uint32_t rounds, uint32_t* err) {
    if (threadIdx.x != 0) return;
    const bool first = blockIdx.x == 0;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (uint32_t r = 1; r <= rounds; r++) {
        if (first) post(&flags[0], r);
        uint32_t n = 0;
        while (poll(&flags[first ? 32 : 0]) != r)
            if (++n == HANDOFF_SPIN) break;
        if (n == HANDOFF_SPIN) {
            post(err, 1);
            break;
        }
        if (!first) post(&flags[32], r);
    }
    if (first) {
        out[0] = t0;
        out[1] = __builtin_amdgcn_s_memrealtime();
    }
}

// `count` dependent agent-scope atomic adds on one word; out[0]: the ticks.
__global__ void handoff_atomic_chain_kernel(uint32_t* word, uint64_t* out, uint32_t count) {
    if (threadIdx.x != 0) return;
    uint32_t v = 0;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (uint32_t i = 0; i < count; i++)
        v = __hip_atomic_fetch_add(word + (v >> 31), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    out[0] = __builtin_amdgcn_s_memrealtime() - t0;
    out[1] = v;
}

// Every workgroup adds one to *count and polls it until all have: out[2g]
// its arrival tick, out[2g + 1] its release tick.
__global__ void handoff_barrier_kernel(uint32_t* count, uint64_t* out, uint32_t* err) {
    if (threadIdx.x != 0) return;
    const uint64_t ta = __builtin_amdgcn_s_memrealtime();
    __hip_atomic_fetch_add(count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t n = 0;
    while (poll(count) < gridDim.x)
        if (++n == HANDOFF_SPIN) {
            post(err, 1);
            break;
        }
    out[2 * blockIdx.x] = ta;
    out[2 * blockIdx.x + 1] = __builtin_amdgcn_s_memrealtime();
}

// ---- A row load behind the weight stream ----
// Every workgroup: `flood` waves each keep ROW_FLOOD_LOADS 16-byte loads per
// lane in flight from their own slice of a cold buffer (a product's weight
// stream), and one more wave, after ROW_DELAY ticks (the stream under way),
// times one vector load of a line other workgroups have read (a product's
// activation row) and one scalar load, each waited for on its own.
// out[3g]: the vector load's ticks, out[3g + 1]: the scalar load's.
constexpr uint32_t ROW_FLOOD_LOADS = 16;
constexpr uint32_t ROW_DELAY = 100;  // ticks of 10 ns

__global__ __launch_bounds__(1024) void row_latency_kernel(const uint4* cold, uint64_t words_per_wave,
                                                           const uint32_t* hot, uint32_t hot_words, uint64_t* out) {
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63, flood = blockDim.x / 64 - 1;
    if (wave < flood) {
        const uint4* b = cold + ((uint64_t)blockIdx.x * flood + wave) * words_per_wave;
        uint32_t acc = 0;
        for (uint64_t i = lane; i + (ROW_FLOOD_LOADS - 1) * 64 < words_per_wave; i += ROW_FLOOD_LOADS * 64) {
            uint4 v[ROW_FLOOD_LOADS];
#pragma unroll
            for (uint32_t u = 0; u < ROW_FLOOD_LOADS; u++) v[u] = b[i + u * 64];
#pragma unroll
            for (uint32_t u = 0; u < ROW_FLOOD_LOADS; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
        }
        if (acc == 0x9E3779B9u) out[3 * blockIdx.x + 2] = acc;
        return;
    }
    const uint64_t t = __builtin_amdgcn_s_memrealtime();
    while (__builtin_amdgcn_s_memrealtime() - t < ROW_DELAY) {}
    const uint32_t off = (blockIdx.x * 64) % (hot_words - 64);
    const uint32_t* vp = hot + off + lane;
    const uint32_t* sp = hot + (off + hot_words / 2) % (hot_words - 64);
    uint32_t v, sv;
    const uint64_t ta = __builtin_amdgcn_s_memrealtime();
    asm volatile("global_load_dword %0, %1, off\n\ts_waitcnt vmcnt(0)" : "=v"(v) : "v"(vp) : "memory");
    const uint64_t tb = __builtin_amdgcn_s_memrealtime();
    asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(sv) : "s"(sp) : "memory");
    const uint64_t tc = __builtin_amdgcn_s_memrealtime();
    if (lane == 0) {
        out[3 * blockIdx.x] = tb - ta;
        out[3 * blockIdx.x + 1] = tc - tb;
        if (v + sv == 0x9E3779B9u) out[3 * blockIdx.x + 2] = v;
    }
}

template <class Launch>
int time_launches(Launch&& launch, uint32_t repeats, double* ms_per_launch) {
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t st = hipEventCreate(&e0);
    if (st == hipSuccess) st = hipEventCreate(&e1);
    if (st == hipSuccess) {
        launch();  // warm-up
        st = hipGetLastError();
    }
    if (st == hipSuccess) st = hipEventRecord(e0, nullptr);
    for (uint32_t r = 0; st == hipSuccess && r < repeats; r++) {
        launch();
        st = hipGetLastError();
    }
    if (st == hipSuccess) st = hipEventRecord(e1, nullptr);
    if (st == hipSuccess) st = hipEventSynchronize(e1);
    float ms = 0.f;
    if (st == hipSuccess) st = hipEventElapsedTime(&ms, e0, e1);
    if (st == hipSuccess) *ms_per_launch = (double)ms / repeats;
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    return (int)st;
}

}  // namespace

extern "C" int iris_probe_hbm_read(const void* d_buf, uint64_t bytes, uint32_t repeats, double* gb_per_s) {
    if (!d_buf || !gb_per_s || repeats == 0 || bytes < 16 || ((uintptr_t)d_buf & 15)) return IRIS_E_INVALID;
    const int cus = iris_device_cus();
    // The best of a few grid sizes (2, 4 and 32 workgroups of 256 threads
    // per CU; two has been the fastest on this part).
    const uint32_t per_cu[] = {2, 4, 32};
    uint32_t* out = nullptr;
    hipError_t st = hipMalloc((void**)&out, (size_t)cus * 32 * 4);
    if (st != hipSuccess) return (int)st;
    const uint64_t words = bytes / 16;
    double best = 0;
    int rc = 0;
    for (uint32_t k : per_cu) {
        const uint32_t wgs = (uint32_t)cus * k;
        double ms = 0;
        rc = time_launches(
            [&] {
                hipLaunchKernelGGL(stream_read_kernel, dim3(wgs), dim3(STREAM_THREADS), 0, nullptr,
                                   (const uint4*)d_buf, words, out);
            },
            repeats, &ms);
        if (rc != 0) break;
        best = std::max(best, (double)(words * 16) / (ms * 1e-3) / 1e9);
    }
    hipFree(out);
    if (rc == 0) *gb_per_s = best;
    return rc;
}

extern "C" int iris_probe_mfma_i8(uint32_t random_operands, uint32_t iterations, double* tops) {
    if (!tops || iterations < MFMA_ROT) return IRIS_E_INVALID;
    const int cus = iris_device_cus();
    const uint32_t wgs = (uint32_t)cus * 4;  // four 4-wave workgroups per CU: four waves per SIMD
    const uint32_t rounds = iterations / MFMA_ROT;
    uint32_t* out = nullptr;
    hipError_t st = hipMalloc((void**)&out, (size_t)wgs * 4);
    if (st != hipSuccess) return (int)st;
    double ms = 0;
    int rc = time_launches(
        [&] {
            if (random_operands)
                hipLaunchKernelGGL(mfma_i8_kernel<true>, dim3(wgs), dim3(256), 0, nullptr, rounds, out);
            else
                hipLaunchKernelGGL(mfma_i8_kernel<false>, dim3(wgs), dim3(256), 0, nullptr, rounds, out);
        },
        3, &ms);
    hipFree(out);
    if (rc == 0) {
        const double ops = (double)wgs * 4 * rounds * MFMA_ROT * MFMA_CHAINS * MFMA_OPS;
        *tops = ops / (ms * 1e-3) / 1e12;
    }
    return rc;
}

extern "C" int iris_probe_handoff(uint32_t workgroups, double* round_trip_us, double* atomic_us, double* barrier_us) {
    if (!round_trip_us || !atomic_us || !barrier_us || workgroups < 2 || workgroups > 1024) return IRIS_E_INVALID;
    constexpr uint32_t ROUNDS = 2000, CHAIN = 1000;
    // [0, 256): flags and counters; then err; then the barrier's ticks.
    uint32_t* mem = nullptr;
    hipError_t st = hipMalloc((void**)&mem, 4096 + 16ull * workgroups);
    if (st != hipSuccess) return (int)st;
    uint32_t* err = mem + 256;
    uint64_t* ticks = (uint64_t*)(mem + 512);
    std::vector<uint64_t> h(2 * (size_t)workgroups);
    uint32_t herr = 0;
    auto run = [&](auto launch, size_t n_ticks) -> hipError_t {
        hipError_t e = hipMemset(mem, 0, 4096);
        if (e == hipSuccess) {
            launch();
            e = hipGetLastError();
        }
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e == hipSuccess) e = hipMemcpy(h.data(), ticks, n_ticks * 8, hipMemcpyDeviceToHost);
        if (e == hipSuccess) e = hipMemcpy(&herr, err, 4, hipMemcpyDeviceToHost);
        return e;
    };
    st = run([&] { hipLaunchKernelGGL(handoff_pingpong_kernel, dim3(2), dim3(64), 0, nullptr, mem, ticks, ROUNDS, err); }, 2);
    if (st == hipSuccess && !herr) *round_trip_us = (double)(h[1] - h[0]) * 0.01 / ROUNDS;
    if (st == hipSuccess && !herr)
        st = run([&] { hipLaunchKernelGGL(handoff_atomic_chain_kernel, dim3(1), dim3(64), 0, nullptr, mem, ticks, CHAIN); }, 2);
    if (st == hipSuccess && !herr) *atomic_us = (double)h[0] * 0.01 / CHAIN;
    if (st == hipSuccess && !herr)
        st = run([&] { hipLaunchKernelGGL(handoff_barrier_kernel, dim3(workgroups), dim3(64), 0, nullptr, mem, ticks, err); },
                 2 * (size_t)workgroups);
    if (st == hipSuccess && !herr) {
        uint64_t last_arrival = 0, last_release = 0;
        for (uint32_t g = 0; g < workgroups; g++) {
            last_arrival = std::max(last_arrival, h[2 * g]);
            last_release = std::max(last_release, h[2 * g + 1]);
        }
        *barrier_us = (double)(last_release - last_arrival) * 0.01;
    }
    hipFree(mem);
    if (st != hipSuccess) return (int)st;
    return herr ? IRIS_E_STATE : 0;
}

extern "C" int iris_probe_row_latency(uint32_t flood_waves, double* vector_us, double* scalar_us) {
    if (!vector_us || !scalar_us || flood_waves > 15) return IRIS_E_INVALID;
    const uint32_t wgs = (uint32_t)iris_device_cus();
    const uint32_t waves = flood_waves + 1;
    // 1 MB of cold stream per flooding wave, at least 256 MB in all.
    const uint64_t words_per_wave = flood_waves ? std::max<uint64_t>((256ull << 20) / 16 / ((uint64_t)wgs * flood_waves),
                                                                   (1ull << 20) / 16)
                                                : 0;
    const uint64_t cold_bytes = std::max<uint64_t>(16, words_per_wave * 16 * wgs * flood_waves);
    constexpr uint32_t HOT_WORDS = 8192;
    char* mem = nullptr;
    hipError_t st = hipMalloc((void**)&mem, cold_bytes + HOT_WORDS * 4 + 24ull * wgs);
    if (st != hipSuccess) return (int)st;
    const uint4* cold = (const uint4*)mem;
    uint32_t* hot = (uint32_t*)(mem + cold_bytes);
    uint64_t* out = (uint64_t*)(mem + cold_bytes + HOT_WORDS * 4);
    st = hipMemset(mem, 1, cold_bytes + HOT_WORDS * 4);
    std::vector<uint64_t> h(3 * (size_t)wgs);
    for (int rep = 0; st == hipSuccess && rep < 3; rep++) {
        hipLaunchKernelGGL(row_latency_kernel, dim3(wgs), dim3(64 * waves), 0, nullptr, cold, words_per_wave, hot,
                           HOT_WORDS, out);
        st = hipGetLastError();
        if (st == hipSuccess) st = hipDeviceSynchronize();
    }
    if (st == hipSuccess) st = hipMemcpy(h.data(), out, h.size() * 8, hipMemcpyDeviceToHost);
    hipFree(mem);
    if (st != hipSuccess) return (int)st;
    std::vector<uint64_t> vt(wgs), sc(wgs);
    for (uint32_t g = 0; g < wgs; g++) {
        vt[g] = h[3 * g];
        sc[g] = h[3 * g + 1];
    }
    std::sort(vt.begin(), vt.end());
    std::sort(sc.begin(), sc.end());
    *vector_us = (double)vt[wgs / 2] * 0.01;
    *scalar_us = (double)sc[wgs / 2] * 0.01;
    return 0;
}
