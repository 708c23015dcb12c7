// A row's digit planes written by the kernel that produces the row (the
// layout act_planes_dwords / act_counts_bytes describe in q8_internal.h),
// so that the one-token product reading it takes its digits through scalar
// loads instead of staging the row itself.
#pragma once

#include "q8_internal.h"

// Balanced signed base-256 digits of v, low byte first: each byte read as
// int8, sum byte_l * 256^l == v.
__device__ __forceinline__ uint64_t act_digits(int32_t v) {
    return (uint64_t)((int64_t)v + 0x8080808080LL) ^ 0x8080808080ULL;
}

// Digits v needs (1-5): the highest non-zero byte of act_digits(v).
__device__ __forceinline__ uint32_t act_digit_count(uint64_t d) {
    return (d >> 32) ? 5 : (d >> 24) ? 4 : (d >> 16) ? 3 : (d >> 8) ? 2 : 1;
}

// Byte l of four digit words, packed low to high.
__device__ __forceinline__ uint32_t act_plane_dword(uint64_t d0, uint64_t d1, uint64_t d2, uint64_t d3, int l) {
    const int sh = 8 * l;
    return (uint32_t)((d0 >> sh) & 0xff) | ((uint32_t)((d1 >> sh) & 0xff) << 8) |
           ((uint32_t)((d2 >> sh) & 0xff) << 16) | ((uint32_t)((d3 >> sh) & 0xff) << 24);
}

// Values first + i (i < 32, a multiple-of-32 first) held by lanes i = 0..31
// of a wave, one each: their planes and digit counts. Every lane of the
// wave calls it (cross-lane shuffles); lanes 32..63 only take part.
__device__ __forceinline__ void act_planes_store32(int32_t v, uint32_t lane, uint32_t first, uint32_t cols,
                                                   uint32_t* planes, uint8_t* counts) {
    const uint64_t d = act_digits(lane < 32 ? v : 0);
    const uint32_t q = lane & ~3u;
    const uint64_t d1 = __shfl(d, q + 1), d2 = __shfl(d, q + 2), d3 = __shfl(d, q + 3);
    uint32_t need = act_digit_count(d);
    need = max(need, (uint32_t)__shfl_xor((int)need, 1));
    need = max(need, (uint32_t)__shfl_xor((int)need, 2));
    need = max(need, (uint32_t)__shfl_xor((int)need, 4));
    if (lane < 32 && (lane & 3) == 0) {
        const uint32_t pw = cols / 4, i = (first + lane) / 4;
#pragma unroll
        for (int l = 0; l < (int)ACT_PLANES; l++) planes[l * pw + i] = act_plane_dword(d, d1, d2, d3, l);
    }
    if (lane < 32 && (lane & 7) == 0) counts[(first + lane) / 8] = (uint8_t)need;
}

// The eight outputs of a gated tile (rows interleaving gate and up): output
// j = first + j (first a multiple of 8) held by lane 2j of the tile's 16
// lanes (the even rows; the odd lanes and lanes 16..63 hold anything). Every
// lane calls it.
__device__ __forceinline__ void act_planes_store8_even(int32_t o, uint32_t lane, uint32_t first, uint32_t cols,
                                                       uint32_t* planes, uint8_t* counts) {
    const bool own = lane < 16 && (lane & 1) == 0;
    const uint64_t d = act_digits(own ? o : 0);
    const uint32_t b = lane & ~7u;
    const uint64_t d1 = __shfl(d, b + 2), d2 = __shfl(d, b + 4), d3 = __shfl(d, b + 6);
    uint32_t need = own ? act_digit_count(d) : 1;
    need = max(need, (uint32_t)__shfl_xor((int)need, 2));
    need = max(need, (uint32_t)__shfl_xor((int)need, 4));
    need = max(need, (uint32_t)__shfl_xor((int)need, 8));
    if (lane < 16 && (lane & 7) == 0) {
        const uint32_t pw = cols / 4, i = first / 4 + lane / 8;
#pragma unroll
        for (int l = 0; l < (int)ACT_PLANES; l++) planes[l * pw + i] = act_plane_dword(d, d1, d2, d3, l);
    }
    if (lane == 0) counts[first / 8] = (uint8_t)need;
}
