// The per-value epilogue of a Q8_0 product, shared by the GEMV and the GEMM:
// one finished output (row, token) with the value of its pair partner
// (row ^ 1), written as the launch's epilogue asks.
#pragma once

#include "detnum_dev.h"
#include "q8_internal.h"

__device__ __forceinline__ void store_output(const GemvArgs& a, uint32_t row, uint32_t token, int32_t v,
                                             int32_t partner) {
    switch (a.epilogue) {
        case EPI_RESIDUAL:
            a.out[(size_t)token * a.out_stride + row] =
                dn::add_sat(v, a.residual[(size_t)token * a.residual_stride + row]);
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
            const uint32_t pos = (uint32_t)(*a.d_pos) + token;
            if (row < a.q_rows + a.kv_rows) {
                if ((row & 1) == 0) {
                    int32_t x0 = v, x1 = partner;
                    // mistral.rs:114-126: pair j of each head, position * f_j.
                    const uint32_t j = (row % a.head_dim) >> 1;
                    if (pos != 0) {
                        if (a.rope_sc) {
                            const int64_t* sc = a.rope_sc + ((size_t)token * (a.head_dim >> 1) + j) * 2;
                            dn::rotate_pair_sc(x0, x1, sc[0], sc[1]);
                        } else {
                            dn::rotate_pair_q30(x0, x1, (int64_t)pos * a.inv_freq[j]);
                        }
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
