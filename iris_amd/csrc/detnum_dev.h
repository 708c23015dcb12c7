// Device-side det-num: the fixed-point arithmetic of crates/det-num restated
// for gfx950. Every function returns the same bits as the reference function
// it names; where operand ranges allow, the 128-bit steps are narrowed to
// 64-bit ones that give the identical result (the narrowing is noted).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dn {

typedef __int128 i128;
typedef unsigned __int128 u128;

constexpr int32_t ONE_ACT = 1 << 16;
constexpr int64_t ONE_ACC = (int64_t)1 << 32;

__device__ __forceinline__ int32_t clamp_i64_to_i32(int64_t v) {
    return v < INT32_MIN ? INT32_MIN : (v > INT32_MAX ? INT32_MAX : (int32_t)v);
}
__device__ __forceinline__ int32_t clamp_i128_to_i32(i128 v) {
    return v < (i128)INT32_MIN ? INT32_MIN : (v > (i128)INT32_MAX ? INT32_MAX : (int32_t)v);
}
__device__ __forceinline__ int64_t clamp_i128_to_i64(i128 v) {
    return v < (i128)INT64_MIN ? INT64_MIN : (v > (i128)INT64_MAX ? INT64_MAX : (int64_t)v);
}
__device__ __forceinline__ int32_t sat_neg_i32(int32_t v) { return v == INT32_MIN ? INT32_MAX : -v; }
__device__ __forceinline__ int64_t sat_neg_i64(int64_t v) { return v == INT64_MIN ? INT64_MAX : -v; }

// ops.rs:773-803. Round-half-even of x / 2^shift; the floor form below is the
// same rounding as the reference's truncate-then-step form.
//
// Every ties-to-even step in this file is written as one comparison,
// rem + (q & 1) > half (the remainder above half, or at half with q odd),
// which compiles to a select; the two-clause form became divergent branches
// with exec-mask bookkeeping around each rounding.
__device__ __forceinline__ int64_t rshift_rte(int64_t x, uint32_t shift) {
    if (shift == 0) return x;
    const int64_t fl = x >> shift;
    const uint64_t rem = (uint64_t)x & ((((uint64_t)1) << shift) - 1);
    const uint64_t half = (uint64_t)1 << (shift - 1);
    return fl + (int64_t)(rem + (uint64_t)(fl & 1) > half);
}

// ops.rs:448-451 + :483-486
__device__ __forceinline__ int32_t requantize(int64_t acc) { return clamp_i64_to_i32(rshift_rte(acc, 16)); }
// ops.rs:41-45
__device__ __forceinline__ int32_t mul_sat(int32_t a, int32_t b) { return requantize((int64_t)a * (int64_t)b); }
// ops.rs:36-38, :431-433
__device__ __forceinline__ int32_t add_sat(int32_t a, int32_t b) { return clamp_i64_to_i32((int64_t)a + b); }
__device__ __forceinline__ int32_t sub_sat(int32_t a, int32_t b) { return clamp_i64_to_i32((int64_t)a - b); }
// ops.rs:436-438
__device__ __forceinline__ int64_t acc_add_sat(int64_t a, int64_t b) {
    int64_t s;
    if (__builtin_add_overflow(a, b, &s)) return a < 0 ? INT64_MIN : INT64_MAX;
    return s;
}

// ops.rs:691-720 on 64-bit operands (the callers below never exceed them).
__device__ __forceinline__ int64_t rte_div_i64(int64_t dividend, int64_t divisor) {
    int64_t q = dividend / divisor;
    int64_t r = dividend % divisor;
    if (r == 0) return q;
    uint64_t twice = (uint64_t)(r < 0 ? -r : r) * 2;
    uint64_t absd = (uint64_t)(divisor < 0 ? -divisor : divisor);
    int64_t step = ((dividend < 0) != (divisor < 0)) ? -1 : 1;
    if (twice < absd) return q;
    if (twice > absd) return q + step;
    return (q & 1) == 0 ? q : q + step;
}

// ops.rs:691-720, full width.
__device__ __forceinline__ i128 rte_div_i128(i128 dividend, i128 divisor) {
    i128 q = dividend / divisor;
    i128 r = dividend % divisor;
    if (r == 0) return q;
    i128 twice = (r < 0 ? -r : r) * 2;
    i128 absd = divisor < 0 ? -divisor : divisor;
    i128 step = ((dividend < 0) != (divisor < 0)) ? -1 : 1;
    if (twice < absd) return q;
    if (twice > absd) return q + step;
    return (q & 1) == 0 ? q : q + step;
}

// ops.rs:81-88: an i64 over a u32 never needs more than 64 bits.
__device__ __forceinline__ int64_t div_acc_by_u32(int64_t value, uint32_t divisor) {
    return rte_div_i64(value, (int64_t)divisor);
}

// ops.rs:53-64: (n << 16) fits in 48 bits.
__device__ __forceinline__ int32_t div_act(int32_t n, int32_t d) {
    return clamp_i64_to_i32(rte_div_i64((int64_t)n * 65536, (int64_t)d));
}

// ops.rs:685-689: round-half-even of a*b / 2^32, clamped.
__device__ __forceinline__ int64_t acc_mul(int64_t a, int64_t b) {
    i128 p = (i128)a * (i128)b;
    const i128 fl = p >> 32;
    const uint64_t rem = (uint64_t)p & 0xffffffffull;
    const i128 r = fl + (i128)(rem + (uint64_t)(fl & 1) > 0x80000000ull);
    return clamp_i128_to_i64(r);
}

// ops.rs:67-78: round-half-even of (n << 32) / d, clamped.
__device__ inline int64_t div_acc(int64_t n, int64_t d) {
    return clamp_i128_to_i64(rte_div_i128((i128)n * ((i128)1 << 32), (i128)d));
}

// ops.rs:608-614: base^exponent by repeated acc_mul, from ONE.
__device__ inline int64_t pow_acc_u32(int64_t base, uint32_t exponent) {
    int64_t r = ONE_ACC;
    for (uint32_t i = 0; i < exponent; i++) r = acc_mul(r, base);
    return r;
}

// ops.rs:564-606: the Q32.32 value whose degree-th power is closest to
// `value` (binary search for the largest r with r^degree <= value, then the
// nearer of r and r + 1, ties to the even one).
__device__ inline int64_t nth_root_acc(int64_t value, uint32_t degree) {
    if (degree == 1 || value == ONE_ACC) return value;
    int64_t low = 0, high = value > ONE_ACC ? value : ONE_ACC;
    while (low < high) {
        const int64_t mid = low + (high - low + 1) / 2;
        if (pow_acc_u32(mid, degree) <= value) low = mid;
        else high = mid - 1;
    }
    const int64_t lower = low, upper = lower == INT64_MAX ? INT64_MAX : lower + 1;
    i128 le = (i128)value - pow_acc_u32(lower, degree);
    i128 ue = (i128)pow_acc_u32(upper, degree) - value;
    if (le < 0) le = -le;
    if (ue < 0) ue = -ue;
    if (ue < le) return upper;
    if (le < ue) return lower;
    return (lower & 1) == 0 ? lower : upper;
}

// ops.rs:722-771. The reference binary-searches the largest r in
// [0, i32::MAX] with r*r*x <= 2^64; that r is found here from a double
// estimate corrected with the same exact u128 test (the test is monotone in
// r, so the corrected value is the one the search returns), then the same
// nearest-with-ties-to-even choice between r and r + 1.
__device__ inline int32_t inv_sqrt_acc(int64_t x) {
    if (x == 0) return INT32_MAX;
    const u128 target = (u128)1 << 64;
    const u128 divisor = (u128)(uint64_t)x;
    const uint32_t max_bits = (uint32_t)INT32_MAX;
    auto prod = [&](uint32_t c) -> u128 { return (u128)((uint64_t)c * (uint64_t)c) * divisor; };
    if (prod(max_bits) <= target) return INT32_MAX;
    // Estimate 2^32 / sqrt(x) from the hardware reciprocal square root and
    // one Newton step; the exact search below does not depend on its quality.
    const double xd = (double)(uint64_t)x;
    double y = __builtin_amdgcn_rsq(xd);
    y = y * (1.5 - 0.5 * xd * y * y);
    double est = floor(4294967296.0 * y);
    if (!(est >= 0.0)) est = 0.0;
    uint32_t low = est >= (double)max_bits ? max_bits : (uint32_t)est;
    while (low < max_bits && prod(low + 1) <= target) low++;
    while (low > 0 && prod(low) > target) low--;
    uint32_t lower = low;
    uint32_t upper = lower + 1 > max_bits ? max_bits : lower + 1;
    u128 le = target - prod(lower);
    u128 up = prod(upper);
    u128 ue = up > target ? up - target : 0;
    uint32_t r;
    if (upper == lower || le < ue) r = lower;
    else if (ue < le) r = upper;
    else r = (lower & 1) == 0 ? lower : upper;
    return (int32_t)r;
}

// ops.rs:81-88 div_acc_by_u32 for a non-negative dividend: the floor
// quotient from a refined hardware reciprocal, made exact by integer
// correction, then rounded half to even. (The generic 64-bit division is a
// long software sequence; this is the hot case, the mean of a sum of squares.)
__device__ __forceinline__ int64_t div_nonneg_by_u32(int64_t value, uint32_t n) {
    const uint64_t u = (uint64_t)value;
    const double nd = (double)n;
    double r = __builtin_amdgcn_rcp(nd);
    r = r * (2.0 - nd * r);
    r = r * (2.0 - nd * r);
    uint64_t q = (uint64_t)((double)u * r);
    int64_t rem = (int64_t)(u - q * (uint64_t)n);
    q = (uint64_t)((int64_t)q + (int64_t)((double)rem * r));
    rem = (int64_t)(u - q * (uint64_t)n);
    while (rem < 0) {
        q--;
        rem += n;
    }
    while (rem >= (int64_t)n) {
        q++;
        rem -= n;
    }
    const uint64_t twice = (uint64_t)rem * 2;
    if (twice > n || (twice == n && (q & 1))) q++;
    return (int64_t)q;
}

// ops.rs:409-428 after the (order-free, saturating) sum of squares.
__device__ __forceinline__ int32_t rms_scale_from_sum(int64_t sum_squares, uint32_t n, int64_t eps) {
    int64_t mean = div_nonneg_by_u32(sum_squares, n);
    return inv_sqrt_acc(acc_add_sat(mean, eps));
}

// rte(x / c) (ops.rs:691-720) for a non-negative dividend below 2^32.
__device__ __forceinline__ uint32_t rte_div_u32(uint32_t x, uint32_t c) {
    const uint32_t q = x / c;
    return q + (uint32_t)(2 * (x - q * c) + (q & 1) > c);
}

// acc_mul (ops.rs:685-689) of 0 <= a, b < 2^32: the product fits 64 bits,
// and the rounded result stays below 2^32 when a or b is below 2^32 - 1.
// (p + 2^31 - 1 + (floor & 1)) carries into the high word exactly when the
// rounding steps up; p <= (2^32 - 1)^2 leaves room for the addend.
__device__ __forceinline__ uint32_t acc_mul_u32(uint32_t a, uint32_t b) {
    const uint64_t p = (uint64_t)a * b;
    return (uint32_t)((p + 0x7fffffffull + ((p >> 32) & 1)) >> 32);
}

// softmax_exp_term (ops.rs:508-556) of delta = -(diff << 16), diff >= 0:
// the only deltas the softmax forms (a logit minus the row's maximum).
// diff >= 2^20 is at or below the -16 cut: zero; diff = 0 gives exactly one.
// Otherwise 0 < r < ln 2 < 1 in Q32.32: every power and quotient of the
// Taylor terms is below 2^32, none of the saturating sums can saturate, the
// result of the nested sums lies in (0, 2^32), and the shift is at most 23,
// so the general routine's integers come out of 32-bit operations. The
// quotient by ln 2 starts from a float estimate (off by at most one, as
// diff < 2^20 is exact in a float) and is corrected on the remainder.
// The body is branch-free (selects only), so a wave's lanes run it together.
__device__ __forceinline__ uint64_t softmax_exp_diff(uint32_t diff) {
    if (diff >= (1u << 20)) return 0;
    const int64_t LN_2_BITS = 2977044472LL;
    const int64_t positive = (int64_t)diff << 16;
    uint32_t shift = (uint32_t)((float)diff * (65536.0f / 2977044472.0f));
    int64_t rl = positive - (int64_t)shift * LN_2_BITS;
    const bool below = rl < 0;
    shift -= (uint32_t)below;
    rl += below ? LN_2_BITS : 0;
    const bool above = rl >= LN_2_BITS;
    shift += (uint32_t)above;
    rl -= above ? LN_2_BITS : 0;
    const uint32_t r = (uint32_t)rl;
    const uint32_t r2 = acc_mul_u32(r, r), r3 = acc_mul_u32(r2, r);
    const uint32_t r4 = acc_mul_u32(r3, r), r5 = acc_mul_u32(r4, r);
    // 1 - r + r2/2 - r3/6 + r4/24 - r5/120, modulo 2^32 (the true value is
    // in (0, 2^32)).
    const uint32_t approx = 0u - r + rte_div_u32(r2, 2) - rte_div_u32(r3, 6) + rte_div_u32(r4, 24) -
                            rte_div_u32(r5, 120);
    const uint32_t fl = approx >> shift;
    const uint32_t rem = approx & ((1u << shift) - 1), half = (1u << shift) >> 1;
    const uint32_t rounded = fl + (uint32_t)(rem + (fl & 1) > half);
    // diff = 0: r = 0 and the sum is 2^32, which wraps to 0 above.
    return diff == 0 ? (uint64_t)ONE_ACC : (uint64_t)(shift == 0 ? approx : rounded);
}

// attention_softmax_raw_weight (ops.rs:269-271), requantize(div_acc(e, sum)),
// for 0 <= e <= 2^32 <= sum < 2^62 and q_scale = 2^32 / sum in double: the
// quotient (e << 32) / sum from the double estimate e * q_scale (within
// 2^-20 of the true quotient, so its floor is off by at most one), made
// exact on the integer remainder (exact modulo 2^64, |remainder| < 2 * sum),
// rounded half to even as div_acc does, then requantized (the quotient is at
// most 2^32, the weight at most 2^16).
__device__ __forceinline__ int32_t softmax_weight(uint64_t e, uint64_t sum, double q_scale) {
    uint64_t q = (uint64_t)((double)e * q_scale);
    int64_t rem = (int64_t)((e << 32) - q * sum);
    if (rem < 0) {
        q--;
        rem += (int64_t)sum;
    } else if ((uint64_t)rem >= sum) {
        q++;
        rem -= (int64_t)sum;
    }
    const uint64_t twice = (uint64_t)rem << 1;
    if (twice > sum || (twice == sum && (q & 1))) q++;
    uint64_t w = q >> 16;
    const uint32_t lo = (uint32_t)q & 0xffff;
    if (lo > 0x8000 || (lo == 0x8000 && (w & 1))) w++;
    return (int32_t)w;
}

// softmax_weight from a double estimate: y = e * 2^16 / sum (w_scale =
// 2^16 / sum) is within 2^-30 of the real quotient, the Q32.32 rounding
// moves it by at most 2^-17, so unless y lies within 2^-15 of a half
// integer both roundings together give the integer nearest y; those rare
// cases take the exact routine.
__device__ __forceinline__ int32_t softmax_weight_fast(uint64_t e, uint64_t sum, double w_scale, double q_scale) {
    const double t = (double)e * w_scale + 0.5;
    const double fl = floor(t);
    // The fraction t - fl below 2^-15 or above 1 - 2^-15, as one comparison.
    if (fabs(t - fl - 0.5) > 0.5 - 0x1p-15) return softmax_weight(e, sum, q_scale);
    return (int32_t)fl;
}

// ops.rs:357-377
__device__ inline int32_t tanh_act(int32_t x) {
    const int32_t LIN = 27 << 16, QUAD = 9 << 16, SAT = 3 << 16;
    if (x >= SAT) return ONE_ACT;
    if (x <= -SAT) return -ONE_ACT;
    int32_t x2 = mul_sat(x, x);
    int32_t num_scale = add_sat(LIN, x2);
    int32_t den_scale = add_sat(LIN, mul_sat(QUAD, x2));
    return div_act(mul_sat(x, num_scale), den_scale);
}

// ops.rs:380-388 (with sequence-check's cap <= 0 passthrough)
__device__ inline int32_t softcap(int32_t x, int32_t cap) {
    if (cap <= 0) return x;
    return mul_sat(cap, tanh_act(div_act(x, cap)));
}

// ops.rs:391-406
__device__ inline int32_t gelu(int32_t x) {
    int32_t x2 = mul_sat(x, x);
    int32_t x3 = mul_sat(x2, x);
    int32_t inner = add_sat(x, mul_sat(2930, x3));
    int32_t t = tanh_act(mul_sat(52290, inner));
    return mul_sat(mul_sat(1 << 15, x), add_sat(ONE_ACT, t));
}

__device__ __forceinline__ int64_t rem_euclid(int64_t a, int64_t m) {
    int64_t r = a % m;
    return r < 0 ? r + m : r;
}

// ops.rs:622-683 sin_cos_acc (returns cos, sin)
__device__ inline void sin_cos_acc(int64_t angle, int32_t& cos_out, int32_t& sin_out) {
    const int64_t HALF_PI = 6746518852LL, PI = 13493037705LL, THREE_HALF_PI = 20239556557LL,
                  TWO_PI = 26986075409LL;
    int64_t reduced = rem_euclid(angle, TWO_PI);
    int64_t x;
    bool sneg = false, cneg = false;
    if (reduced <= HALF_PI) { x = reduced; }
    else if (reduced <= PI) { x = PI - reduced; cneg = true; }
    else if (reduced <= THREE_HALF_PI) { x = reduced - PI; sneg = true; cneg = true; }
    else { x = TWO_PI - reduced; sneg = true; }
    int64_t x2 = acc_mul(x, x);
    int64_t x3 = acc_mul(x2, x);
    int64_t x5 = acc_mul(x3, x2);
    int64_t x7 = acc_mul(x5, x2);
    int64_t sp = acc_add_sat(acc_add_sat(x, sat_neg_i64(div_acc_by_u32(x3, 6))),
                             acc_add_sat(div_acc_by_u32(x5, 120), sat_neg_i64(div_acc_by_u32(x7, 5040))));
    int64_t x4 = acc_mul(x2, x2);
    int64_t x6 = acc_mul(x4, x2);
    int64_t cp = acc_add_sat(acc_add_sat(ONE_ACC, sat_neg_i64(div_acc_by_u32(x2, 2))),
                             acc_add_sat(div_acc_by_u32(x4, 24), sat_neg_i64(div_acc_by_u32(x6, 720))));
    int32_t s = requantize(sp), c = requantize(cp);
    sin_out = sneg ? sat_neg_i32(s) : s;
    cos_out = cneg ? sat_neg_i32(c) : c;
}

// ---- mistral-dense (crates/det-num/src/mistral.rs) ----

// mistral.rs:23-32
__device__ __forceinline__ int64_t m_shift_rte(int64_t value, uint32_t shift) {
    const int64_t fl = value >> shift;
    const int64_t rem = value - (int64_t)((uint64_t)fl << shift);
    const int64_t half = (int64_t)1 << (shift - 1);
    return fl + (int64_t)(rem + (fl & 1) > half);
}

// mistral.rs:43-56. r < ln 2 < 2^32 and acc <= 2^32 throughout, so each
// Horner step's (r * acc) >> 32 is one 32 x 32-bit product (r itself while
// acc is exactly 2^32), and its quotient by n a 32-bit one.
__device__ inline uint64_t exp_neg_q32(uint64_t a) {
    const uint64_t ONE_Q32 = (uint64_t)1 << 32, LN2 = 2977044472ULL;
    const uint64_t k = a / LN2;
    if (k >= 32) return 0;
    const uint32_t r = (uint32_t)(a - k * LN2);
    uint64_t acc = ONE_Q32;
#pragma unroll
    for (uint32_t n = 14; n >= 1; n--) {
        const uint32_t prod = acc == ONE_Q32 ? r : (uint32_t)(((uint64_t)r * (uint32_t)acc) >> 32);
        acc = ONE_Q32 - prod / n;
    }
    return acc >> k;
}

// floor(2^63 / d) for 2^32 <= d <= 2^33: a double estimate (within 2^-22 of
// the quotient, so its floor is off by at most one) corrected on the exact
// remainder.
__device__ __forceinline__ uint64_t floor_2p63_over(uint64_t d) {
    const uint64_t q = (uint64_t)(9223372036854775808.0 / (double)d);
    const int64_t rem = (int64_t)(((uint64_t)1 << 63) - q * d);
    return q - (uint64_t)(rem < 0) + (uint64_t)(rem >= 0 && (uint64_t)rem >= d);
}

// mistral.rs:59-77
__device__ inline int32_t silu(int32_t x) {
    const uint64_t ONE_Q32 = (uint64_t)1 << 32;
    uint64_t mag = x < 0 ? (uint64_t)(-(int64_t)x) : (uint64_t)x;
    uint64_t divisor = ONE_Q32 + exp_neg_q32(mag << 16);
    uint64_t positive = floor_2p63_over(divisor) << 1;
    uint64_t sig = x < 0 ? ONE_Q32 - positive : positive;
    int64_t product = (int64_t)x * (int64_t)sig;
    return clamp_i64_to_i32(m_shift_rte(product, 32));
}

// silu by table. exp_neg_q32(|x| << 16) is zero once the quotient by ln 2
// reaches 32, i.e. for |x| >= SILU_TAB_HALF; there the divisor is 2^32, the
// sigmoid 2^32 (or 0 for x < 0) and silu(x) is exactly x (or 0). Inside,
// silu(x) = tab[x + SILU_TAB_HALF - 1], a table of dn::silu itself.
constexpr int32_t SILU_TAB_HALF = 1453635;
constexpr uint32_t SILU_TAB_N = 2u * SILU_TAB_HALF - 1;

// The table index of x (clamped, so the load is always in bounds).
__device__ __forceinline__ uint32_t silu_tab_index(int32_t x) {
    const uint32_t u = (uint32_t)x + (uint32_t)(SILU_TAB_HALF - 1);
    return u < SILU_TAB_N ? u : SILU_TAB_N - 1;
}

// silu(x) given tab[silu_tab_index(x)].
__device__ __forceinline__ int32_t silu_from_tab(int32_t x, int32_t looked_up) {
    const uint32_t u = (uint32_t)x + (uint32_t)(SILU_TAB_HALF - 1);
    return u < SILU_TAB_N ? looked_up : (x > 0 ? x : 0);
}

// mistral.rs:84-109 (returns sin, cos in Q30)
__device__ inline void sin_cos_q30(int64_t angle, int64_t& sin_out, int64_t& cos_out) {
    const int64_t ONE_Q30 = (int64_t)1 << 30;
    const int64_t HALF_PI = 6746518852LL, PI = 13493037705LL, THREE_HALF_PI = 20239556557LL,
                  TWO_PI = 26986075409LL;
    int64_t reduced = rem_euclid(angle, TWO_PI);
    int64_t quarter, ss = 1, cs = 1;
    if (reduced <= HALF_PI) { quarter = reduced; }
    else if (reduced <= PI) { quarter = PI - reduced; cs = -1; }
    else if (reduced <= THREE_HALF_PI) { quarter = reduced - PI; ss = -1; cs = -1; }
    else { quarter = TWO_PI - reduced; ss = -1; }
    int64_t t = quarter >> 2;
    int64_t u = (t * t) >> 30;
    int64_t s = ONE_Q30;
    s = ONE_Q30 - ((u * s) >> 30) / 210;
    s = ONE_Q30 - ((u * s) >> 30) / 156;
    s = ONE_Q30 - ((u * s) >> 30) / 110;
    s = ONE_Q30 - ((u * s) >> 30) / 72;
    s = ONE_Q30 - ((u * s) >> 30) / 42;
    s = ONE_Q30 - ((u * s) >> 30) / 20;
    s = ONE_Q30 - ((u * s) >> 30) / 6;
    s = (t * s) >> 30;
    int64_t c = ONE_Q30;
    c = ONE_Q30 - ((u * c) >> 30) / 240;
    c = ONE_Q30 - ((u * c) >> 30) / 182;
    c = ONE_Q30 - ((u * c) >> 30) / 132;
    c = ONE_Q30 - ((u * c) >> 30) / 90;
    c = ONE_Q30 - ((u * c) >> 30) / 56;
    c = ONE_Q30 - ((u * c) >> 30) / 30;
    c = ONE_Q30 - ((u * c) >> 30) / 12;
    c = ONE_Q30 - ((u * c) >> 30) / 2;
    sin_out = ss * s;
    cos_out = cs * c;
}

// mistral.rs:114-126 for one pair (a, b) at angle position * f.
__device__ __forceinline__ void rotate_pair_q30(int32_t& a, int32_t& b, int64_t angle) {
    int64_t s, c;
    sin_cos_q30(angle, s, c);
    int64_t x = a, y = b;
    a = clamp_i64_to_i32(m_shift_rte(x * c - y * s, 30));
    b = clamp_i64_to_i32(m_shift_rte(x * s + y * c, 30));
}

// The same rotation with (sin, cos) already formed.
__device__ __forceinline__ void rotate_pair_sc(int32_t& a, int32_t& b, int64_t s, int64_t c) {
    int64_t x = a, y = b;
    a = clamp_i64_to_i32(m_shift_rte(x * c - y * s, 30));
    b = clamp_i64_to_i32(m_shift_rte(x * s + y * c, 30));
}

// mistral.rs:130-145 after the wrapping sum.
__device__ __forceinline__ int32_t scaled_score_from_sum(int64_t sum, uint32_t scale_q32) {
    // floor(sum * scale / 2^32) = hi * scale + floor(lo * scale / 2^32) for
    // sum = hi * 2^32 + lo (hi signed, lo unsigned); |.| < 2^63.
    const int64_t hi = sum >> 32;
    const uint64_t lo = (uint32_t)sum;
    const int64_t scaled = hi * (int64_t)scale_q32 + (int64_t)((lo * scale_q32) >> 32);
    return clamp_i64_to_i32(rshift_rte(scaled, 16));
}

// q8.rs:94-104: value / 2^shift, ties to even, saturated to i32.
__device__ __forceinline__ int32_t round_to_i32(i128 value, uint32_t shift) {
    const i128 fl = value >> shift;
    const uint64_t rem = (uint64_t)(value - (fl << shift));  // in [0, 2^shift), shift < 64
    const uint64_t half = (uint64_t)1 << (shift - 1);
    const i128 r = fl + (i128)(rem + (uint64_t)(fl & 1) > half);
    return clamp_i128_to_i32(r);
}

// q8.rs:27-42: exact Q.24 of finite f16 bits (callers reject exponent 0x1f).
__device__ __forceinline__ int64_t scale_q24(uint32_t bits) {
    uint32_t e = (bits >> 10) & 0x1f;
    int64_t m = bits & 0x3ff;
    int64_t mag = e == 0 ? m : ((1024 + m) << (e - 1));
    return (bits & 0x8000) ? -mag : mag;
}

}  // namespace dn
