"""Exact-arithmetic helpers for pinning the oracle (independent of its C code).

Every operation is done on exact rationals and rounded once, correctly, to
binary32 / binary64, so fma and per-operation rounding can be restated
without trusting any fused instruction or compiler.
"""
from fractions import Fraction

import numpy as np


def round_f32(q: Fraction) -> np.float32:
    """Round an exact rational to the nearest binary32 (ties to even)."""
    x = np.float32(float(q))  # within one binary32 ulp of the answer
    best = None
    for c in (np.nextafter(x, np.float32(-np.inf)), x, np.nextafter(x, np.float32(np.inf))):
        if not np.isfinite(c):
            continue
        err = abs(Fraction(float(c)) - q)
        if best is None or err < best[0] or (
            err == best[0] and (int(c.view(np.uint32)) & 1) == 0
        ):
            best = (err, c)
    return best[1]


def round_f64(q: Fraction) -> float:
    return float(q)  # Fraction.__float__ rounds correctly


def f32_sub(a, b):
    return round_f32(Fraction(float(a)) - Fraction(float(b)))


def f32_mul(a, b):
    return round_f32(Fraction(float(a)) * Fraction(float(b)))


def f32_fma(a, b, c):
    return round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def f64_fma(a, b, c):
    return round_f64(Fraction(a) * Fraction(b) + Fraction(c))


def sq3_f32(dx, dy, dz):
    """fma(dz,dz, fma(dx,dx, dy*dy)) in binary32 (chamfer.cu:67, fps.cu:145 under -fmad)."""
    return f32_fma(dz, dz, f32_fma(dx, dx, f32_mul(dy, dy)))


def knn_l2_f32(diffs):
    """d0*d0 then fma(dk,dk,acc) in binary32 (knn.cu:148-158 under -fmad)."""
    acc = f32_mul(diffs[0], diffs[0])
    for d in diffs[1:]:
        acc = f32_fma(d, d, acc)
    return acc


def sq3_f64(dx, dy, dz):
    return f64_fma(dz, dz, f64_fma(dx, dx, dy * dy))


def sq3_f16(dx, dy, dz):
    """c10::Half arithmetic: every op rounded to binary16; numpy's float16
    operators compute in float32 and round, the same thing."""
    dx, dy, dz = np.float16(dx), np.float16(dy), np.float16(dz)
    return (dx * dx + dy * dy) + dz * dz
