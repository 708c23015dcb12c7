// Wave-wide reductions through DPP lane moves (register to register within
// each 16-lane row) and readlane across the four rows: no LDS round trip per
// step, as a __shfl_xor ladder would take. Every lane of the wave must be
// active where these are called.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "detnum_dev.h"

// A 64-bit value from another lane of the same 16-lane row (DPP control CTRL).
template <int CTRL>
__device__ __forceinline__ int64_t dpp64(int64_t v) {
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)((uint64_t)v >> 32), CTRL, 0xF, 0xF, false);
    return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

__device__ __forceinline__ uint64_t readlane64(uint64_t v, int lane) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
    return ((uint64_t)hi << 32) | lo;
}

// Saturating sum of non-negative terms over each 16-lane row, in every lane
// of the row: min(true sum, i64::MAX), the same in any order. Lanes swap
// within quads (1, then 2 apart), then mirror within half rows and rows.
__device__ __forceinline__ int64_t row16_sum_sat_nonneg(int64_t v) {
    v = dn::acc_add_sat(v, dpp64<0xB1>(v));   // quad_perm [1,0,3,2]
    v = dn::acc_add_sat(v, dpp64<0x4E>(v));   // quad_perm [2,3,0,1]
    v = dn::acc_add_sat(v, dpp64<0x141>(v));  // row_half_mirror
    v = dn::acc_add_sat(v, dpp64<0x140>(v));  // row_mirror
    return v;
}

// The same over the whole wave: the four row sums through scalar registers.
__device__ __forceinline__ int64_t wave_sum_sat_nonneg(int64_t v) {
    v = row16_sum_sat_nonneg(v);
    int64_t t = 0;
#pragma unroll
    for (int r = 0; r < 4; r++) t = dn::acc_add_sat(t, (int64_t)readlane64((uint64_t)v, 16 * r));
    return t;
}

// Wrapping 64-bit sum over the wave (the same in any order).
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
    v += (uint64_t)dpp64<0xB1>((int64_t)v);
    v += (uint64_t)dpp64<0x4E>((int64_t)v);
    v += (uint64_t)dpp64<0x141>((int64_t)v);
    v += (uint64_t)dpp64<0x140>((int64_t)v);
    uint64_t t = 0;
#pragma unroll
    for (int r = 0; r < 4; r++) t += readlane64(v, 16 * r);
    return t;
}

// Maximum of unsigned 64-bit keys over the wave.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    uint64_t o;
    o = (uint64_t)dpp64<0xB1>((int64_t)v);
    v = o > v ? o : v;
    o = (uint64_t)dpp64<0x4E>((int64_t)v);
    v = o > v ? o : v;
    o = (uint64_t)dpp64<0x141>((int64_t)v);
    v = o > v ? o : v;
    o = (uint64_t)dpp64<0x140>((int64_t)v);
    v = o > v ? o : v;
    uint64_t t = 0;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        o = readlane64(v, 16 * r);
        t = o > t ? o : t;
    }
    return t;
}
