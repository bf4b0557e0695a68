"""Exact bf16 / f16 conversions in numpy (oracle; test infrastructure only).

numpy has no bfloat16, so bf16 values travel as uint16 bit patterns.

to_bf16_bits restates the round-to-nearest-even rule of the reference's
constant encoder, src/jam/ops/structural.mm:33-38 (`x += 0x7FFF +
((x >> 16) & 1); return x >> 16`), with one deliberate difference: NaN inputs
are kept NaN (quiet bit set, sign kept).  The reference formula turns some
NaN payloads into ±Inf (0x7F800001 + 0x7FFF carries into the exponent and
truncates to 0x7F80); XLA and the HIP kernels keep NaN, so the oracle does.

to_f16_bits is IEEE round-to-nearest-even with subnormals, as XLA converts;
the reference's FloatToHalf (structural.mm:22-31) truncates and flushes
subnormals — that difference is documented, not mirrored.
"""

from __future__ import annotations

import numpy as np


def to_bf16_bits(x) -> np.ndarray:
    """float32 (or anything castable) -> uint16 bf16 bits, RNE, NaN kept."""
    f = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    is_nan = (u & 0x7FFFFFFF) > 0x7F800000
    nan_bits = ((u >> 16) | 0x0040) & 0xFFFF
    return np.where(is_nan, nan_bits, rounded).astype(np.uint16)


def to_bf16_bits_f64(x) -> np.ndarray:
    """float64 -> bf16 bits with ONE rounding (RNE).

    Going through float32 first can double-round: when the float32 result
    sits exactly on a bf16 halfway point but the float64 value was not, the
    direction must come from the float64 value, not from ties-to-even."""
    x = np.asarray(x, dtype=np.float64)
    f = x.astype(np.float32)
    bits = to_bf16_bits(f)
    u = np.ascontiguousarray(f).view(np.uint32)
    tie = ((u & 0xFFFF) == 0x8000) & np.isfinite(f)
    with np.errstate(invalid="ignore"):
        above = (x - f.astype(np.float64)) * np.sign(f)
    trunc = (u >> 16).astype(np.uint16)
    fixed = np.where(above > 0, trunc + np.uint16(1), np.where(above < 0, trunc, bits))
    return np.where(tie, fixed, bits).astype(np.uint16)


def from_bf16_bits(b) -> np.ndarray:
    """uint16 bf16 bits -> float32 (exact)."""
    b = np.asarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(x) -> np.ndarray:
    """float -> nearest bf16 value, returned as float32."""
    return from_bf16_bits(to_bf16_bits(x))


def to_f16_bits(x) -> np.ndarray:
    """float32 -> IEEE half bits (numpy's cast is RNE with subnormals)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def from_f16_bits(b) -> np.ndarray:
    return np.asarray(b, dtype=np.uint16).view(np.float16).astype(np.float32)


def bf16_ulp_distance(a_bits, b_bits) -> np.ndarray:
    """Distance in units of last place between two bf16 bit arrays (same sign
    class ordering; NaNs compare as distance 0 to each other)."""
    a = np.asarray(a_bits, dtype=np.uint16).astype(np.int32)
    b = np.asarray(b_bits, dtype=np.uint16).astype(np.int32)

    def ordered(v):
        # map sign-magnitude to a monotone integer line
        return np.where(v & 0x8000, -(v & 0x7FFF), v & 0x7FFF)

    d = np.abs(ordered(a) - ordered(b))
    both_nan = np.isnan(from_bf16_bits(a.astype(np.uint16))) & np.isnan(
        from_bf16_bits(b.astype(np.uint16)))
    return np.where(both_nan, 0, d)
