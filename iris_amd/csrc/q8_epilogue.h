// The per-value epilogue of a Q8_0 product, shared by the GEMV and the GEMM:
// one finished output (row, token) with the value of its pair partner
// (row ^ 1), written as the launch's epilogue asks.
#pragma once

#include "detnum_dev.h"
#include "q8_internal.h"

// What an output's epilogue reads besides the product: the residual, or
// the position and its pair's rotation (sin and cos from the table, or the
// angle step). Loading these apart from the store lets a kernel issue them
// early, so their latency is not on the output's path: the loads are
// unconditional (an epilogue that does not use one reads x instead) and
// nothing is computed from them here, so no wait follows them. row must be
// a valid row of the launch (callers clamp).
struct EpiIn {
    int32_t res;   // EPI_RESIDUAL
    int32_t pos;   // EPI_ROPE_KV: the position of token 0
    int64_t s, c;  // EPI_ROPE_KV: sin and cos of the pair (table), or s = the pair's angle step
};

__device__ __forceinline__ EpiIn epilogue_inputs(const GemvArgs& a, uint32_t row, uint32_t token) {
    const bool res = a.epilogue == EPI_RESIDUAL, rope = a.epilogue == EPI_ROPE_KV;
    const int32_t* rp = res ? a.residual + (size_t)token * a.residual_stride + row : a.x;
    const int32_t* pp = rope ? a.d_pos : a.x;
    const uint32_t j = rope ? (row % a.head_dim) >> 1 : 0;
    const int64_t* sp = !rope ? (const int64_t*)a.x
                        : a.rope_sc ? a.rope_sc + ((size_t)token * (a.head_dim >> 1) + j) * 2
                                    : a.inv_freq + j;
    EpiIn in;
    in.res = *rp;
    in.pos = *pp;
    in.s = sp[0];
    in.c = rope && a.rope_sc ? sp[1] : 0;
    return in;
}

__device__ __forceinline__ void store_output_in(const GemvArgs& a, uint32_t row, uint32_t token, int32_t v,
                                                int32_t partner, const EpiIn& in) {
    switch (a.epilogue) {
        case EPI_RESIDUAL:
            a.out[(size_t)token * a.out_stride + row] = dn::add_sat(v, in.res);
            break;
        case EPI_SOFTCAP:
            a.out[(size_t)token * a.out_stride + row] = dn::softcap(v, a.softcap);
            break;
        case EPI_SWIGLU:
        case EPI_GEGLU:
            if ((row & 1) == 0) {
                const int32_t act = a.epilogue == EPI_SWIGLU ? dn::silu(v) : dn::gelu(v);
                a.out[(size_t)token * a.out_stride + (row >> 1)] = dn::mul_sat(act, partner);
            }
            break;
        case EPI_ROPE_KV: {
            const uint32_t pos = (uint32_t)in.pos + token;
            if (row < a.q_rows + a.kv_rows) {
                if ((row & 1) == 0) {
                    int32_t x0 = v, x1 = partner;
                    // mistral.rs:114-126: pair j of each head, position * f_j.
                    if (pos != 0) {
                        if (a.rope_sc) dn::rotate_pair_sc(x0, x1, in.s, in.c);
                        else dn::rotate_pair_q30(x0, x1, (int64_t)pos * in.s);
                    }
                    if (row < a.q_rows) {
                        a.out[(size_t)token * a.out_stride + row] = x0;
                        a.out[(size_t)token * a.out_stride + row + 1] = x1;
                    } else {
                        int32_t* kc = a.k_cache + (size_t)(row - a.q_rows) * a.k_pos_stride + pos;
                        kc[0] = x0;
                        kc[a.k_pos_stride] = x1;
                    }
                }
            } else {
                a.v_cache[(size_t)pos * a.kv_rows + (row - a.q_rows - a.kv_rows)] = v;
            }
            break;
        }
        default:
            a.out[(size_t)token * a.out_stride + row] = v;
    }
}

__device__ __forceinline__ void store_output(const GemvArgs& a, uint32_t row, uint32_t token, int32_t v,
                                             int32_t partner) {
    store_output_in(a, row, token, v, partner, epilogue_inputs(a, row, token));
}
