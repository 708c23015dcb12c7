/*
 * CPU oracle: det-num restated in C. TEST INFRASTRUCTURE ONLY (see detnum.h).
 *
 * Each function names the reference function and lines it follows. Rust's
 * i128 `/` and `%` truncate toward zero and `>>` on signed values is
 * arithmetic; GCC's __int128 and int64_t behave the same way, so the
 * restatement keeps the reference's operations one for one.
 */
#include "detnum.h"

#include <string.h>

static const int64_t I64_MAX = INT64_MAX;
static const int64_t I64_MIN = INT64_MIN;

static int32_t clamp_i128_to_i32(dn_i128 v) {  /* ops.rs:488-490 */
    if (v < (dn_i128)INT32_MIN) return INT32_MIN;
    if (v > (dn_i128)INT32_MAX) return INT32_MAX;
    return (int32_t)v;
}

static int64_t clamp_i128_to_i64(dn_i128 v) {  /* ops.rs:492-494 */
    if (v < (dn_i128)I64_MIN) return I64_MIN;
    if (v > (dn_i128)I64_MAX) return I64_MAX;
    return (int64_t)v;
}

static int32_t sat_neg_i32(int32_t v) { return v == INT32_MIN ? INT32_MAX : -v; }
static int64_t sat_neg_i64(int64_t v) { return v == I64_MIN ? I64_MAX : -v; }

/* ops.rs:773-803 rshift_round_ties_even_bits */
int64_t dn_rshift_round_ties_even(int64_t x, uint32_t shift) {
    if (shift == 0) return x;
    dn_i128 divisor = (dn_i128)1 << shift;
    dn_i128 xx = x;
    dn_i128 q = xx / divisor;
    dn_i128 r = xx % divisor;
    if (r == 0) return (int64_t)q;
    dn_i128 twice = (r < 0 ? -r : r) * 2;
    dn_i128 step = xx < 0 ? -1 : 1;
    dn_i128 rounded;
    if (twice < divisor) rounded = q;
    else if (twice > divisor) rounded = q + step;
    else if ((q & 1) == 0) rounded = q;
    else rounded = q + step;
    return (int64_t)rounded;
}

/* ops.rs:448-451 requantize + ops.rs:483-486 narrow_act_sat */
int32_t dn_requantize(int64_t acc) {
    int64_t r = dn_rshift_round_ties_even(acc, 16);
    if (r < INT32_MIN) return INT32_MIN;
    if (r > INT32_MAX) return INT32_MAX;
    return (int32_t)r;
}

/* ops.rs:36-38 */
int32_t dn_add_sat(int32_t a, int32_t b) {
    int64_t s = (int64_t)a + b;
    if (s > INT32_MAX) return INT32_MAX;
    if (s < INT32_MIN) return INT32_MIN;
    return (int32_t)s;
}

/* ops.rs:431-433 */
int32_t dn_sub_sat(int32_t a, int32_t b) {
    int64_t s = (int64_t)a - b;
    if (s > INT32_MAX) return INT32_MAX;
    if (s < INT32_MIN) return INT32_MIN;
    return (int32_t)s;
}

/* ops.rs:41-45 */
int32_t dn_mul_sat(int32_t a, int32_t b) { return dn_requantize((int64_t)a * (int64_t)b); }

/* ops.rs:436-438 */
int64_t dn_acc_add_sat(int64_t a, int64_t b) {
    int64_t s;
    if (__builtin_add_overflow(a, b, &s)) return a < 0 ? I64_MIN : I64_MAX;
    return s;
}

/* ops.rs:691-720 */
dn_i128 dn_round_ties_even_division(dn_i128 dividend, dn_i128 divisor) {
    dn_i128 q = dividend / divisor;
    dn_i128 r = dividend % divisor;
    if (r == 0) return q;
    dn_i128 twice = (r < 0 ? -r : r) * 2;
    dn_i128 absd = divisor < 0 ? -divisor : divisor;
    dn_i128 step = ((dividend < 0) ^ (divisor < 0)) ? -1 : 1;
    if (twice < absd) return q;
    if (twice > absd) return q + step;
    if ((q & 1) == 0) return q;
    return q + step;
}

/* ops.rs:53-64 */
int32_t dn_div_act(int32_t numerator, int32_t denominator) {
    dn_i128 dividend = (dn_i128)numerator * ((dn_i128)1 << 16);
    return clamp_i128_to_i32(dn_round_ties_even_division(dividend, (dn_i128)denominator));
}

/* ops.rs:67-78 */
int64_t dn_div_acc(int64_t numerator, int64_t denominator) {
    dn_i128 dividend = (dn_i128)numerator * ((dn_i128)1 << 32);
    return clamp_i128_to_i64(dn_round_ties_even_division(dividend, (dn_i128)denominator));
}

/* ops.rs:81-88 */
int64_t dn_div_acc_by_u32(int64_t value, uint32_t divisor) {
    return clamp_i128_to_i64(dn_round_ties_even_division((dn_i128)value, (dn_i128)divisor));
}

/* ops.rs:685-689 */
int64_t dn_acc_mul(int64_t lhs, int64_t rhs) {
    dn_i128 p = (dn_i128)lhs * (dn_i128)rhs;
    return clamp_i128_to_i64(dn_round_ties_even_division(p, (dn_i128)1 << 32));
}

/* ops.rs:768-771 */
static dn_u128 inv_sqrt_product(uint32_t c, dn_u128 divisor) {
    dn_u128 cc = (dn_u128)c * (dn_u128)c; /* < 2^62, cannot saturate */
    dn_u128 p;
    if (__builtin_mul_overflow(cc, divisor, &p)) return ~(dn_u128)0;
    return p;
}

/* ops.rs:722-766 */
int32_t dn_inv_sqrt_acc(int64_t x) {
    if (x == 0) return INT32_MAX;
    dn_u128 target = (dn_u128)1 << 64;
    dn_u128 divisor = (dn_u128)(uint64_t)x;
    uint32_t max_bits = (uint32_t)INT32_MAX;
    if (inv_sqrt_product(max_bits, divisor) <= target) return INT32_MAX;
    uint32_t low = 0, high = max_bits;
    while (low < high) {
        uint32_t mid = low + ((high - low + 1) / 2);
        if (inv_sqrt_product(mid, divisor) <= target) low = mid;
        else high = mid - 1;
    }
    uint32_t lower = low;
    uint32_t upper = lower == UINT32_MAX ? UINT32_MAX : lower + 1;
    if (upper > max_bits) upper = max_bits;
    dn_u128 lp = inv_sqrt_product(lower, divisor);
    dn_u128 up = inv_sqrt_product(upper, divisor);
    dn_u128 lower_error = target - lp;
    dn_u128 upper_error = up > target ? up - target : 0;
    uint32_t r;
    if (upper == lower || lower_error < upper_error) r = lower;
    else if (upper_error < lower_error) r = upper;
    else if ((lower & 1) == 0) r = lower;
    else r = upper;
    return (int32_t)r;
}

/* ops.rs:409-428 */
int32_t dn_rms_norm_scale(const int32_t* v, size_t n, int64_t eps) {
    int64_t sum = 0;
    for (size_t i = 0; i < n; i++) sum = dn_acc_add_sat(sum, (int64_t)v[i] * (int64_t)v[i]);
    int64_t mean = dn_div_acc_by_u32(sum, (uint32_t)n);
    int64_t adjusted = dn_acc_add_sat(mean, eps);
    return dn_inv_sqrt_acc(adjusted);
}

/* ops.rs:98-114 */
void dn_rms_norm(int32_t* v, const int32_t* w, size_t n, int64_t eps) {
    int32_t scale = dn_rms_norm_scale(v, n, eps);
    for (size_t i = 0; i < n; i++) v[i] = dn_mul_sat(dn_mul_sat(v[i], scale), w[i]);
}

/* ops.rs:124-134 */
void dn_value_rms_norm(int32_t* v, size_t n, int64_t eps) {
    int32_t scale = dn_rms_norm_scale(v, n, eps);
    for (size_t i = 0; i < n; i++) v[i] = dn_mul_sat(v[i], scale);
}

/* ops.rs:466-481 */
size_t dn_argmax_first(const int32_t* xs, size_t n) {
    size_t best = 0;
    int32_t bv = xs[0];
    for (size_t i = 1; i < n; i++)
        if (xs[i] > bv) { best = i; bv = xs[i]; }
    return best;
}

/* ops.rs:508-556 */
int64_t dn_softmax_exp_term(int64_t delta) {
    const int64_t LN_2_BITS = 2977044472LL;
    const int64_t MIN_DELTA = -((int64_t)16 << 32);
    if (delta <= MIN_DELTA) return 0;
    int64_t positive = sat_neg_i64(delta);
    int64_t shift = positive / LN_2_BITS;
    int64_t r = positive % LN_2_BITS;
    int64_t r2 = dn_acc_mul(r, r);
    int64_t r3 = dn_acc_mul(r2, r);
    int64_t r4 = dn_acc_mul(r3, r);
    int64_t r5 = dn_acc_mul(r4, r);
    int64_t approx = dn_acc_add_sat(
        dn_acc_add_sat(DN_ONE_ACC, sat_neg_i64(r)),
        dn_acc_add_sat(dn_div_acc_by_u32(r2, 2),
                       dn_acc_add_sat(sat_neg_i64(dn_div_acc_by_u32(r3, 6)),
                                      dn_acc_add_sat(dn_div_acc_by_u32(r4, 24),
                                                     sat_neg_i64(dn_div_acc_by_u32(r5, 120))))));
    if (approx <= 0) return 0;
    if (shift >= 0 && shift < 64) return dn_rshift_round_ties_even(approx, (uint32_t)shift);
    return 0;
}

/* ops.rs:233-261 attention_softmax_into, with :264-276 for the terms */
void dn_attention_softmax(const int32_t* logits, size_t n, int64_t* exp_scratch, int32_t* weights) {
    size_t mi = dn_argmax_first(logits, n);
    int32_t mx = logits[mi];
    int64_t sum = 0;
    for (size_t i = 0; i < n; i++) {
        int64_t delta = (int64_t)dn_sub_sat(logits[i], mx) * ((int64_t)1 << 16);
        exp_scratch[i] = dn_softmax_exp_term(delta);
        sum = dn_acc_add_sat(sum, exp_scratch[i]);
    }
    int32_t summed = 0;
    for (size_t i = 0; i < n; i++) {
        weights[i] = dn_requantize(dn_div_acc(exp_scratch[i], sum));
        summed = dn_add_sat(summed, weights[i]);
    }
    int32_t residual = dn_sub_sat(DN_ONE_ACT, summed);
    weights[mi] = dn_add_sat(weights[mi], residual);
}

/* ops.rs:357-377 */
int32_t dn_tanh_act(int32_t x) {
    const int32_t LIN = 27 << 16, QUAD = 9 << 16, SAT = 3 << 16;
    if (x >= SAT) return DN_ONE_ACT;
    if (x <= -SAT) return sat_neg_i32(DN_ONE_ACT);
    int32_t x2 = dn_mul_sat(x, x);
    int32_t num_scale = dn_add_sat(LIN, x2);
    int32_t den_scale = dn_add_sat(LIN, dn_mul_sat(QUAD, x2));
    int32_t numerator = dn_mul_sat(x, num_scale);
    return dn_div_act(numerator, den_scale);
}

/* ops.rs:380-388 */
int32_t dn_softcap_act(int32_t x, int32_t cap) {
    int32_t normalized = dn_div_act(x, cap);
    return dn_mul_sat(cap, dn_tanh_act(normalized));
}

/* ops.rs:391-406 */
int32_t dn_gelu(int32_t x) {
    const int32_t HALF = 1 << 15, INNER = 52290, CUBIC = 2930;
    int32_t x2 = dn_mul_sat(x, x);
    int32_t x3 = dn_mul_sat(x2, x);
    int32_t cubic = dn_mul_sat(CUBIC, x3);
    int32_t inner = dn_add_sat(x, cubic);
    int32_t t = dn_tanh_act(dn_mul_sat(INNER, inner));
    return dn_mul_sat(dn_mul_sat(HALF, x), dn_add_sat(DN_ONE_ACT, t));
}

/* ops.rs:608-614 */
int64_t dn_pow_acc_u32(int64_t base, uint32_t exponent) {
    int64_t r = DN_ONE_ACC;
    for (uint32_t i = 0; i < exponent; i++) r = dn_acc_mul(r, base);
    return r;
}

/* ops.rs:564-606 */
int64_t dn_nth_root_acc(int64_t value, uint32_t degree) {
    if (degree == 1 || value == DN_ONE_ACC) return value;
    int64_t low = 0;
    int64_t high = value > DN_ONE_ACC ? value : DN_ONE_ACC;
    while (low < high) {
        int64_t mid = low + ((high - low + 1) / 2);
        if (dn_pow_acc_u32(mid, degree) <= value) low = mid;
        else high = mid - 1;
    }
    int64_t lower = low;
    int64_t upper = lower == I64_MAX ? I64_MAX : lower + 1;
    int64_t lv = dn_pow_acc_u32(lower, degree);
    int64_t uv = dn_pow_acc_u32(upper, degree);
    dn_i128 le = (dn_i128)value - (dn_i128)lv;
    if (le < 0) le = -le;
    dn_i128 ue = (dn_i128)uv - (dn_i128)value;
    if (ue < 0) ue = -ue;
    if (ue < le) return upper;
    if (le < ue) return lower;
    return (lower & 1) == 0 ? lower : upper;
}

/* ops.rs:558-562 */
int64_t dn_rope_frequency_step(int64_t base, size_t freq_base_dim) {
    uint32_t degree = (uint32_t)(freq_base_dim / 2);
    return dn_div_acc(DN_ONE_ACC, dn_nth_root_acc(base, degree));
}

/* ops.rs:650-666 */
static int64_t sin_polynomial(int64_t x) {
    int64_t x2 = dn_acc_mul(x, x);
    int64_t x3 = dn_acc_mul(x2, x);
    int64_t x5 = dn_acc_mul(x3, x2);
    int64_t x7 = dn_acc_mul(x5, x2);
    return dn_acc_add_sat(dn_acc_add_sat(x, sat_neg_i64(dn_div_acc_by_u32(x3, 6))),
                          dn_acc_add_sat(dn_div_acc_by_u32(x5, 120),
                                         sat_neg_i64(dn_div_acc_by_u32(x7, 5040))));
}

/* ops.rs:668-683 */
static int64_t cos_polynomial(int64_t x) {
    int64_t x2 = dn_acc_mul(x, x);
    int64_t x4 = dn_acc_mul(x2, x2);
    int64_t x6 = dn_acc_mul(x4, x2);
    return dn_acc_add_sat(dn_acc_add_sat(DN_ONE_ACC, sat_neg_i64(dn_div_acc_by_u32(x2, 2))),
                          dn_acc_add_sat(dn_div_acc_by_u32(x4, 24),
                                         sat_neg_i64(dn_div_acc_by_u32(x6, 720))));
}

static int64_t rem_euclid_i64(int64_t a, int64_t m) {
    int64_t r = a % m;
    return r < 0 ? r + m : r;
}

/* ops.rs:622-648 */
void dn_sin_cos_acc(int64_t angle, int32_t* cos_out, int32_t* sin_out) {
    const int64_t HALF_PI = 6746518852LL, PI = 13493037705LL, THREE_HALF_PI = 20239556557LL,
                  TWO_PI = 26986075409LL;
    int64_t reduced = rem_euclid_i64(angle, TWO_PI);
    int64_t qa;
    int ss, cs;
    if (reduced <= HALF_PI) { qa = reduced; ss = 1; cs = 1; }
    else if (reduced <= PI) { qa = PI - reduced; ss = 1; cs = -1; }
    else if (reduced <= THREE_HALF_PI) { qa = reduced - PI; ss = -1; cs = -1; }
    else { qa = TWO_PI - reduced; ss = -1; cs = 1; }
    int32_t s = dn_requantize(sin_polynomial(qa));
    int32_t c = dn_requantize(cos_polynomial(qa));
    if (ss < 0) s = sat_neg_i32(s);
    if (cs < 0) c = sat_neg_i32(c);
    *cos_out = c;
    *sin_out = s;
}

/* ops.rs:154-199 (with mul_usize_by_acc ops.rs:616-620) */
void dn_rope_rotate_pairs(int32_t* v, size_t n, size_t rotary_dim, size_t freq_base_dim, int64_t base,
                          size_t position) {
    (void)n;
    if (rotary_dim == 0) return;
    if (position == 0) return;
    size_t half = rotary_dim / 2;
    int64_t inv_f = DN_ONE_ACC;
    int64_t step = dn_rope_frequency_step(base, freq_base_dim);
    for (size_t i = 0; i < half; i++) {
        int64_t angle = clamp_i128_to_i64((dn_i128)position * (dn_i128)inv_f);
        int32_t c, s;
        dn_sin_cos_acc(angle, &c, &s);
        int32_t lhs = v[i], rhs = v[i + half];
        v[i] = dn_sub_sat(dn_mul_sat(lhs, c), dn_mul_sat(rhs, s));
        v[i + half] = dn_add_sat(dn_mul_sat(rhs, c), dn_mul_sat(lhs, s));
        inv_f = dn_acc_mul(inv_f, step);
    }
}

/* crates/inference/kernels/src/tensor.rs:522-528 dot_bits (mac_bits ops.rs:17-19) */
int32_t dn_dot_bits(const int32_t* a, const int32_t* b, size_t n) {
    uint64_t acc = 0; /* wrapping i64 */
    for (size_t i = 0; i < n; i++) acc += (uint64_t)((int64_t)a[i] * (int64_t)b[i]);
    return dn_requantize((int64_t)acc);
}

/* ---------------- Q8_0: crates/det-num/src/q8.rs ---------------- */

/* q8.rs:27-42 */
int dn_scale_q24(uint16_t bits, int64_t* out) {
    uint32_t exponent = (bits >> 10) & 0x1f;
    int64_t mantissa = bits & 0x3ff;
    int64_t magnitude;
    if (exponent == 0x1f) return -1;
    if (exponent == 0) magnitude = mantissa;
    else magnitude = (1024 + mantissa) << (exponent - 1);
    *out = (bits & 0x8000) ? -magnitude : magnitude;
    return 0;
}

/* q8.rs:94-104 */
int32_t dn_round_to_i32(dn_i128 value, uint32_t shift) {
    dn_i128 floor = value >> shift;
    dn_i128 rem = value - (floor << shift);
    dn_i128 half = (dn_i128)1 << (shift - 1);
    dn_i128 rounded = (rem > half || (rem == half && (floor & 1) == 1)) ? floor + 1 : floor;
    return clamp_i128_to_i32(rounded);
}

/* q8.rs:56-72 (the i128 total wraps; two's complement addition in unsigned
 * __int128 is the wrapping_add the reference uses) */
int dn_q8_dot_row(const int32_t* act, const uint8_t* row, size_t cols, int32_t* out) {
    if (cols == 0 || cols % DN_Q8_BLOCK) return -1;
    dn_u128 total = 0;
    for (size_t b = 0; b < cols / DN_Q8_BLOCK; b++) {
        const uint8_t* blk = row + b * DN_Q8_BLOCK_BYTES;
        int64_t scale;
        if (dn_scale_q24((uint16_t)(blk[0] | (blk[1] << 8)), &scale)) return -1;
        int64_t sum = 0;
        const int32_t* a = act + b * DN_Q8_BLOCK;
        for (int j = 0; j < DN_Q8_BLOCK; j++) sum += (int64_t)(int8_t)blk[2 + j] * (int64_t)a[j];
        total += (dn_u128)((dn_i128)sum * (dn_i128)scale);
    }
    *out = dn_round_to_i32((dn_i128)total, 24);
    return 0;
}

/* q8.rs:76-92 */
int dn_q8_dequantize_row(const uint8_t* row, size_t cols, int32_t* out) {
    if (cols == 0 || cols % DN_Q8_BLOCK) return -1;
    for (size_t b = 0; b < cols / DN_Q8_BLOCK; b++) {
        const uint8_t* blk = row + b * DN_Q8_BLOCK_BYTES;
        int64_t scale;
        if (dn_scale_q24((uint16_t)(blk[0] | (blk[1] << 8)), &scale)) return -1;
        for (int j = 0; j < DN_Q8_BLOCK; j++)
            out[b * DN_Q8_BLOCK + j] = dn_round_to_i32((dn_i128)(int8_t)blk[2 + j] * scale, 8);
    }
    return 0;
}

/* ---------------- mistral-dense: crates/det-num/src/mistral.rs ---------------- */

static const uint64_t ONE_Q32 = (uint64_t)1 << 32;
static const uint64_t LN_2_Q32 = 2977044472ULL;

/* mistral.rs:23-32 */
static int64_t m_shift_round_ties_even(int64_t value, uint32_t shift) {
    int64_t floor = value >> shift;
    int64_t rem = value - (int64_t)((uint64_t)floor << shift);
    int64_t half = (int64_t)1 << (shift - 1);
    return (rem > half || (rem == half && (floor & 1) == 1)) ? floor + 1 : floor;
}

/* mistral.rs:34-36 */
static int32_t m_saturate(int64_t v) {
    if (v < INT32_MIN) return INT32_MIN;
    if (v > INT32_MAX) return INT32_MAX;
    return (int32_t)v;
}

/* mistral.rs:43-56 */
uint64_t dn_exp_neg_q32(uint64_t a) {
    uint64_t k = a / LN_2_Q32;
    if (k >= 32) return 0;
    uint64_t r = a % LN_2_Q32;
    uint64_t acc = ONE_Q32;
    for (uint64_t n = 14; n >= 1; n--) acc = ONE_Q32 - ((r * acc) >> 32) / n;
    return acc >> k;
}

/* mistral.rs:59-69 */
uint64_t dn_sigmoid_q32(int32_t x) {
    uint64_t magnitude = x < 0 ? (uint64_t)(-(int64_t)x) : (uint64_t)x;
    uint64_t divisor = ONE_Q32 + dn_exp_neg_q32(magnitude << 16);
    uint64_t positive = (((uint64_t)1 << 63) / divisor) << 1;
    return x < 0 ? ONE_Q32 - positive : positive;
}

/* mistral.rs:72-77 */
int32_t dn_silu(int32_t x) {
    int64_t product = (int64_t)x * (int64_t)dn_sigmoid_q32(x);
    return m_saturate(m_shift_round_ties_even(product, 32));
}

/* mistral.rs:84-109 */
void dn_sin_cos_q30(int64_t angle, int64_t* sin_out, int64_t* cos_out) {
    const int64_t ONE_Q30 = (int64_t)1 << 30;
    const int64_t HALF_PI = 6746518852LL, PI = 13493037705LL, THREE_HALF_PI = 20239556557LL,
                  TWO_PI = 26986075409LL;
    int64_t reduced = rem_euclid_i64(angle, TWO_PI);
    int64_t quarter;
    int64_t ss, cs;
    if (reduced <= HALF_PI) { quarter = reduced; ss = 1; cs = 1; }
    else if (reduced <= PI) { quarter = PI - reduced; ss = 1; cs = -1; }
    else if (reduced <= THREE_HALF_PI) { quarter = reduced - PI; ss = -1; cs = -1; }
    else { quarter = TWO_PI - reduced; ss = -1; cs = 1; }
    int64_t t = quarter >> 2;
    int64_t u = (t * t) >> 30;
    static const int64_t SIN_DIV[7] = {210, 156, 110, 72, 42, 20, 6};
    static const int64_t COS_DIV[8] = {240, 182, 132, 90, 56, 30, 12, 2};
    int64_t s = ONE_Q30;
    for (int i = 0; i < 7; i++) s = ONE_Q30 - ((u * s) >> 30) / SIN_DIV[i];
    s = (t * s) >> 30;
    int64_t c = ONE_Q30;
    for (int i = 0; i < 8; i++) c = ONE_Q30 - ((u * c) >> 30) / COS_DIV[i];
    *sin_out = ss * s;
    *cos_out = cs * c;
}

/* mistral.rs:114-126 */
void dn_rotate_consecutive_pairs(int32_t* v, size_t n, const int64_t* inv_freq, size_t pairs,
                                 uint32_t position) {
    if (position == 0) return;
    size_t np = n / 2 < pairs ? n / 2 : pairs;
    for (size_t j = 0; j < np; j++) {
        int64_t angle = (int64_t)position * inv_freq[j];
        int64_t s, c;
        dn_sin_cos_q30(angle, &s, &c);
        int64_t a = v[2 * j], b = v[2 * j + 1];
        v[2 * j] = m_saturate(m_shift_round_ties_even(a * c - b * s, 30));
        v[2 * j + 1] = m_saturate(m_shift_round_ties_even(a * s + b * c, 30));
    }
}

/* mistral.rs:130-145 */
int32_t dn_scaled_score(const int32_t* q, const int32_t* k, size_t n, uint32_t scale_q32) {
    uint64_t sum = 0; /* wrapping i64 */
    for (size_t i = 0; i < n; i++) sum += (uint64_t)((int64_t)q[i] * (int64_t)k[i]);
    dn_i128 scaled = ((dn_i128)(int64_t)sum * (dn_i128)scale_q32) >> 32;
    dn_i128 half = (dn_i128)1 << 15;
    dn_i128 floor = scaled >> 16;
    dn_i128 rem = scaled - (floor << 16);
    dn_i128 rounded = (rem > half || (rem == half && (floor & 1) == 1)) ? floor + 1 : floor;
    return clamp_i128_to_i32(rounded);
}

/* mistral.rs:148-160 */
uint32_t dn_attention_scale_q32(uint32_t head_dim) {
    dn_u128 target = ((dn_u128)1 << 64) / (dn_u128)(head_dim > 1 ? head_dim : 1);
    dn_u128 low = 0, high = UINT32_MAX;
    while (low < high) {
        dn_u128 mid = (low + high + 1) / 2;
        if (mid * mid <= target) low = mid;
        else high = mid - 1;
    }
    return (uint32_t)low;
}

/* mistral.rs:162-175 */
static dn_u128 integer_sqrt(dn_u128 value) {
    if (value < 2) return value;
    dn_u128 low = 1, high = (dn_u128)1 << 64;
    while (low < high) {
        dn_u128 mid = (low + high + 1) / 2;
        if (mid <= value / mid) low = mid;
        else high = mid - 1;
    }
    return low;
}

/* mistral.rs:185-214 */
int dn_yarn_inverse_frequencies(uint64_t base, uint32_t pairs, uint32_t factor, uint32_t low,
                                uint32_t high, int64_t* out) {
    if (pairs == 0 || (pairs & (pairs - 1)) != 0 || base == 0 || factor == 0 || high <= low) return -1;
    dn_u128 root = (dn_u128)base << 32;
    for (uint32_t i = 0; i < (uint32_t)__builtin_ctz(pairs); i++) root = integer_sqrt(root << 32);
    dn_u128 step = (((dn_u128)1 << 64) + root / 2) / root;
    dn_u128 span = high - low;
    dn_u128 plain = (dn_u128)1 << 32;
    for (uint32_t pair = 0; pair < pairs; pair++) {
        uint32_t hs = high > pair ? high - pair : 0;
        dn_u128 kept = (dn_u128)hs < span ? (dn_u128)hs : span;
        dn_u128 numerator = plain * (span + (dn_u128)(factor - 1) * kept);
        dn_u128 denominator = (dn_u128)factor * span;
        out[pair] = (int64_t)((numerator + denominator / 2) / denominator);
        plain = (plain * step + ((dn_u128)1 << 31)) >> 32;
    }
    return 0;
}

/* ---------------- convert: crates/det-num/src/convert.rs ---------------- */

/* convert.rs:94-107 */
static dn_u128 saturating_shift_left(dn_u128 value, uint32_t shift, dn_u128 max_mag) {
    if (value == 0) return 0;
    if (shift >= 128) return max_mag;
    dn_u128 threshold = max_mag >> shift;
    return value > threshold ? max_mag : value << shift;
}

/* convert.rs:110-127 */
static dn_u128 round_ties_even_div_pow2(dn_u128 value, uint32_t shift) {
    if (shift == 0) return value;
    if (shift >= 128) return 0;
    dn_u128 q = value >> shift;
    dn_u128 mask = ((dn_u128)1 << shift) - 1;
    dn_u128 r = value & mask;
    dn_u128 half = (dn_u128)1 << (shift - 1);
    return (r > half || (r == half && (q & 1) == 1)) ? q + 1 : q;
}

/* convert.rs:47-92 */
static dn_i128 f32_to_fixed_bits(float x, uint32_t frac, dn_u128 max_pos, dn_u128 max_neg) {
    uint32_t bits;
    memcpy(&bits, &x, 4);
    int neg = (bits >> 31) != 0;
    int32_t exponent_bits = (int32_t)((bits >> 23) & 0xff);
    uint32_t fraction = bits & 0x7fffff;
    if (exponent_bits == 0 && fraction == 0) return 0;
    dn_u128 significand;
    int32_t exponent;
    if (exponent_bits == 0) { significand = fraction; exponent = -149; }
    else { significand = (dn_u128)((1u << 23) | fraction); exponent = exponent_bits - 127 - 23; }
    int32_t scaled = exponent + (int32_t)frac;
    dn_u128 max_mag = neg ? max_neg : max_pos;
    dn_u128 mag;
    if (scaled >= 0) mag = saturating_shift_left(significand, (uint32_t)scaled, max_mag);
    else {
        mag = round_ties_even_div_pow2(significand, (uint32_t)(-scaled));
        if (mag > max_mag) mag = max_mag;
    }
    if (neg) return mag >= max_neg ? -(dn_i128)max_neg : -(dn_i128)mag;
    return (dn_i128)mag;
}

/* convert.rs:21-32 */
int32_t dn_f32_to_act_bits(float x) {
    dn_i128 b = f32_to_fixed_bits(x, 16, (dn_u128)INT32_MAX, (dn_u128)1 << 31);
    return clamp_i128_to_i32(b);
}

/* convert.rs:34-45 */
int64_t dn_f32_to_acc_bits(float x) {
    dn_i128 b = f32_to_fixed_bits(x, 32, (dn_u128)I64_MAX, (dn_u128)1 << 63);
    return clamp_i128_to_i64(b);
}
