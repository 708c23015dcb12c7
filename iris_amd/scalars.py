"""Import-time scalar derivations: the integer constants a model's shape carries.

These run once on the host when a model is described, never on the token
path. Each one restates the reference's import-time arithmetic in Python
integers, so the committed bits are the same:

- ``f32_to_act_bits`` / ``f32_to_acc_bits``: crates/det-num/src/convert.rs:21-92
- ``attention_scale_q32``: crates/det-num/src/mistral.rs:148-160
- ``yarn_inverse_frequencies``: crates/det-num/src/mistral.rs:162-214
- ``mistral_yarn_bounds``: crates/model/import/src/mistral.rs:189-247
- ``f32_to_q16``: crates/model/import/src/main.rs:1214-1218
"""
from __future__ import annotations

import math
import struct

I32_MIN, I32_MAX = -(1 << 31), (1 << 31) - 1
I64_MIN, I64_MAX = -(1 << 63), (1 << 63) - 1
ONE = 1 << 16


def _f32_to_fixed_bits(x: float, frac: int, max_pos: int, max_neg: int) -> int:
    bits = struct.unpack("<I", struct.pack("<f", x))[0]
    neg = bits >> 31
    exp_bits = (bits >> 23) & 0xFF
    fraction = bits & 0x7FFFFF
    if exp_bits == 0xFF:
        raise ValueError("fixed-point conversion requires a finite source value")
    if exp_bits == 0 and fraction == 0:
        return 0
    if exp_bits == 0:
        significand, exponent = fraction, -149
    else:
        significand, exponent = (1 << 23) | fraction, exp_bits - 127 - 23
    scaled = exponent + frac
    max_mag = max_neg if neg else max_pos
    if scaled >= 0:
        mag = max_mag if significand > (max_mag >> scaled) else significand << scaled
    else:
        shift = -scaled
        q = significand >> shift
        r = significand & ((1 << shift) - 1)
        half = 1 << (shift - 1)
        mag = q + 1 if (r > half or (r == half and q & 1)) else q
        mag = min(mag, max_mag)
    if neg:
        return -max_neg if mag >= max_neg else -mag
    return mag


def f32_to_act_bits(x: float) -> int:
    """Q16.16 bits of an f32 value (the value is first rounded to f32)."""
    return max(I32_MIN, min(I32_MAX, _f32_to_fixed_bits(x, 16, I32_MAX, 1 << 31)))


def f32_to_acc_bits(x: float) -> int:
    """Q32.32 bits of an f32 value (the value is first rounded to f32)."""
    return max(I64_MIN, min(I64_MAX, _f32_to_fixed_bits(x, 32, I64_MAX, 1 << 63)))


def f32_to_q16(value: float) -> int:
    """The importer's float-to-Q16.16 for config floats (f64 round, clamp)."""
    scaled = value * ONE
    return int(max(I32_MIN, min(I32_MAX, _round_half_away(scaled))))


def _round_half_away(v: float) -> float:
    # Rust's f64::round rounds half away from zero.
    return math.floor(v + 0.5) if v >= 0 else -math.floor(-v + 0.5)


def attention_scale_q32(head_dim: int) -> int:
    """floor(2^32 / sqrt(head_dim)) by binary search on the square."""
    target = (1 << 64) // max(head_dim, 1)
    low, high = 0, (1 << 32) - 1
    while low < high:
        mid = (low + high + 1) // 2
        if mid * mid <= target:
            low = mid
        else:
            high = mid - 1
    return low


def _integer_sqrt(value: int) -> int:
    if value < 2:
        return value
    low, high = 1, 1 << 64
    while low < high:
        mid = (low + high + 1) // 2
        if mid <= value // mid:
            low = mid
        else:
            high = mid - 1
    return low


def yarn_inverse_frequencies(base: int, pairs: int, factor: int, low: int, high: int):
    """Per-pair rotation angle per position in Q32.32, or None where the
    reference refuses (pairs not a power of two, zero base or factor,
    high <= low)."""
    if pairs <= 0 or pairs & (pairs - 1) or base == 0 or factor == 0 or high <= low:
        return None
    root = base << 32
    for _ in range(pairs.bit_length() - 1):
        root = _integer_sqrt(root << 32)
    step = ((1 << 64) + root // 2) // root
    span = high - low
    plain = 1 << 32
    out = []
    for pair in range(pairs):
        kept = min(max(high - pair, 0), span)
        numerator = plain * (span + (factor - 1) * kept)
        denominator = factor * span
        out.append((numerator + denominator // 2) // denominator)
        plain = (plain * step + (1 << 31)) >> 32
    return out


def _correction_dim(dims: float, original: float, rotations: float, base: float) -> float:
    return dims * math.log(original / (rotations * 2.0 * math.pi)) / (2.0 * math.log(base))


def mistral_yarn_bounds(head_dim: int, original: float, beta_fast: float, beta_slow: float,
                        base: float):
    """YaRN's ramp bounds (low, high) as the importer derives them."""
    dims = float(head_dim)
    lo = _correction_dim(dims, original, beta_fast, base)
    hi = _correction_dim(dims, original, beta_slow, base)
    for v in (lo, hi):
        if abs(v - round(v)) < 1e-6:
            raise ValueError(f"a YaRN bound of {v} is too close to a whole number")
    return int(max(math.floor(lo), 0.0)), int(min(math.ceil(hi), dims - 1.0))


def plain_rope_inverse_frequencies(base: int, head_dim: int):
    """Plain RoPE as the importer writes it: YaRN with factor 1, where the
    ramp bounds drop out of the formula."""
    freqs = yarn_inverse_frequencies(base, head_dim // 2, 1, 0, 1)
    if freqs is None:
        raise ValueError("plain RoPE needs head_dim / 2 to be a power of two")
    return freqs
