/*
 * CPU oracle: a plain-C restatement of iris's det-num fixed-point arithmetic
 * (crates/det-num) and of the layer kernels built on it.
 *
 * TEST INFRASTRUCTURE ONLY. This code gives the expected results the HIP path is
 * compared against, and the timed CPU baseline. Nothing in the shipped library links,
 * loads or calls it; only tests, the smoke check and the benchmark's CPU
 * baseline leg do.
 *
 * Types follow det-num: Act = Q16.16 in int32_t, Acc = Q32.32 in int64_t,
 * Q8_0 blocks = 2-byte little-endian f16 scale + 32 signed bytes.
 * Every function cites the reference function it restates.
 *
 * Pinning: the rounding, saturation, MAC, f32->fixed, scale_q24, dot_row,
 * RoPE, attention-scale, YaRN and SiLU special values are pinned by the
 * reference's own test vectors; inv_sqrt_acc by exhaustive neighbour checks;
 * the embedding, final norm, head and first-maximum selection by the
 * reference's direct-executor fixtures (expected tokens [2], [2, 0], the tie
 * to 0). softmax_exp_term, exp_neg_q32, sigmoid_q32/silu, sin_cos_q30,
 * sin_cos_acc and tanh_act are pinned bit for bit only at the inputs where
 * the reference's arithmetic fixes every bit (zero and unit remainders,
 * small angles in each quadrant, the linear and saturated ranges) and
 * elsewhere against their truncation-error bounds; nth_root_acc and gelu
 * only against bounds. Parity unpinned at the last bit between those points
 * (no reference vectors exist for them).
 */
#ifndef IRIS_ORACLE_DETNUM_H
#define IRIS_ORACLE_DETNUM_H

#include <stddef.h>
#include <stdint.h>

typedef __int128 dn_i128;
typedef unsigned __int128 dn_u128;

#define DN_ONE_ACT ((int32_t)1 << 16)
#define DN_ONE_ACC ((int64_t)1 << 32)
#define DN_Q8_BLOCK 32
#define DN_Q8_BLOCK_BYTES 34

/* ---- core rounding / saturation (crates/det-num/src/ops.rs) ---- */
int64_t dn_rshift_round_ties_even(int64_t x, uint32_t shift);
int32_t dn_requantize(int64_t acc);
int32_t dn_add_sat(int32_t a, int32_t b);
int32_t dn_sub_sat(int32_t a, int32_t b);
int32_t dn_mul_sat(int32_t a, int32_t b);
int64_t dn_acc_add_sat(int64_t a, int64_t b);
dn_i128 dn_round_ties_even_division(dn_i128 dividend, dn_i128 divisor);
int32_t dn_div_act(int32_t numerator, int32_t denominator);
int64_t dn_div_acc(int64_t numerator, int64_t denominator);
int64_t dn_div_acc_by_u32(int64_t value, uint32_t divisor);
int64_t dn_acc_mul(int64_t lhs, int64_t rhs);
int32_t dn_inv_sqrt_acc(int64_t x);
int32_t dn_rms_norm_scale(const int32_t* v, size_t n, int64_t eps);
void dn_rms_norm(int32_t* v, const int32_t* w, size_t n, int64_t eps);
void dn_value_rms_norm(int32_t* v, size_t n, int64_t eps);
size_t dn_argmax_first(const int32_t* xs, size_t n);
int64_t dn_softmax_exp_term(int64_t delta);
void dn_attention_softmax(const int32_t* logits, size_t n, int64_t* exp_scratch, int32_t* weights);
int32_t dn_tanh_act(int32_t x);
int32_t dn_softcap_act(int32_t x, int32_t cap);
int32_t dn_gelu(int32_t x);
int64_t dn_nth_root_acc(int64_t value, uint32_t degree);
int64_t dn_pow_acc_u32(int64_t base, uint32_t exponent);
int64_t dn_rope_frequency_step(int64_t base, size_t freq_base_dim);
void dn_sin_cos_acc(int64_t angle, int32_t* cos_out, int32_t* sin_out);
void dn_rope_rotate_pairs(int32_t* v, size_t n, size_t rotary_dim, size_t freq_base_dim, int64_t base,
                          size_t position);
int32_t dn_dot_bits(const int32_t* a, const int32_t* b, size_t n);

/* ---- Q8_0 (crates/det-num/src/q8.rs) ---- */
/* Returns 0 and the exact Q.24 value, or -1 for inf/NaN scales. */
int dn_scale_q24(uint16_t bits, int64_t* out);
/* 0 on success, -1 for a non-finite scale. */
int dn_q8_dot_row(const int32_t* act, const uint8_t* row, size_t cols, int32_t* out);
int dn_q8_dequantize_row(const uint8_t* row, size_t cols, int32_t* out);
int32_t dn_round_to_i32(dn_i128 value, uint32_t shift);

/* ---- mistral-dense (crates/det-num/src/mistral.rs) ---- */
uint64_t dn_exp_neg_q32(uint64_t a);
uint64_t dn_sigmoid_q32(int32_t x);
int32_t dn_silu(int32_t x);
void dn_sin_cos_q30(int64_t angle, int64_t* sin_out, int64_t* cos_out);
void dn_rotate_consecutive_pairs(int32_t* v, size_t n, const int64_t* inv_freq, size_t pairs,
                                 uint32_t position);
int32_t dn_scaled_score(const int32_t* q, const int32_t* k, size_t n, uint32_t scale_q32);
uint32_t dn_attention_scale_q32(uint32_t head_dim);
/* Returns 0 and fills out[pairs], or -1 where the reference returns None. */
int dn_yarn_inverse_frequencies(uint64_t base, uint32_t pairs, uint32_t factor, uint32_t low,
                                uint32_t high, int64_t* out);

/* ---- float -> fixed conversion (crates/det-num/src/convert.rs) ---- */
int32_t dn_f32_to_act_bits(float x);
int64_t dn_f32_to_acc_bits(float x);

#endif
