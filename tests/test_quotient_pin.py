"""Pin of the router softmax's quotient (slotstream_spark_amd/csrc/ss_verify_dev.hpp, router_tail_wave).

The kernel forms v / z for every entry from one division: rz = RN(1/z), q = RN(v * rz), rem = RN(v - q * z) (a
fused multiply-add, exact here), result RN(q + rem * rz), and takes the division itself for v in (0, 2^-64). The
oracle divides (oracle/ssmoe_oracle.c or_router_topk). This test replays the kernel's sequence with exact rational
arithmetic and correctly rounded binary32 (ties to even) and requires the IEEE quotient bit for bit over the kernel's
domain (v in [0, 1], z in [1, 512]): random binary32 patterns and the values next to powers of two, where a wrong
rounding would show first.
"""
from fractions import Fraction

import numpy as np
import pytest

_HALF = Fraction(1, 2)


def _rn32(x: Fraction) -> np.float32:
    """x rounded to the nearest binary32, ties to even (normal range, as in the kernel's domain)."""
    if x == 0:
        return np.float32(0.0)
    sign = -1 if x < 0 else 1
    x = abs(x)
    e = x.numerator.bit_length() - x.denominator.bit_length()
    if Fraction(2) ** e > x:
        e -= 1
    assert e >= -126, "outside the normal range"
    scale = Fraction(2) ** (23 - e)
    m = x * scale
    mi = m.numerator // m.denominator
    rest = m - mi
    if rest > _HALF or (rest == _HALF and mi % 2 == 1):
        mi += 1
    return np.float32(sign * float(Fraction(mi) / scale))


def _fma(a, b, c) -> np.float32:
    return _rn32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def _kernel_quotient(v: np.float32, z: np.float32) -> np.float32:
    rz = np.float32(1.0) / z
    if 0.0 < v < 2.0 ** -64:
        return v / z
    q = _rn32(Fraction(float(v)) * Fraction(float(rz)))
    rem = _fma(-q, z, v)
    return _fma(rem, rz, q)


def _bits(f: np.float32) -> int:
    return int(np.array(f, dtype=np.float32).view(np.uint32))


def _step(x: float, k: int) -> float:
    """The binary32 k representable values above (k < 0: below) x."""
    b = int(np.array([x], dtype=np.float32).view(np.uint32)[0]) + k
    return float(np.array([b], dtype=np.uint32).view(np.float32)[0])


def _cases():
    rng = np.random.default_rng(20261202)
    one, lo, z_hi = 0x3F800000, 0x1F800000, 0x44000000  # 1.0, 2^-64, 512.0
    v = rng.integers(lo, one + 1, 2500, dtype=np.uint32).view(np.float32)
    z = rng.integers(one, z_hi + 1, 2500, dtype=np.uint32).view(np.float32)
    out = list(zip(v.tolist(), z.tolist()))
    # next to powers of two: v = 2^e +- k ulp, z = 2^f +- j ulp
    for e in (0, -1, -7, -23, -40, -63):
        for k in (-3, -1, 0, 1, 2):
            vv = _step(2.0 ** e, k)
            if not 0.0 <= vv <= 1.0:
                continue
            for f in range(0, 10):
                for j in (-2, -1, 0, 1, 3):
                    zz = _step(2.0 ** f, j)
                    if 1.0 <= zz <= 512.0:
                        out.append((vv, zz))
    out += [(0.0, 1.0), (1.0, 1.0), (1.0, 512.0), (0.5, 3.0), (1.0, 3.0), (2.0 ** -70, 7.0)]
    return out


def test_markstein_quotient_equals_ieee_division():
    bad = []
    for v, z in _cases():
        v32, z32 = np.float32(v), np.float32(z)
        got, want = _kernel_quotient(v32, z32), v32 / z32
        if _bits(got) != _bits(want):
            bad.append((v, z, float(got), float(want)))
    assert not bad, bad[:5]


def test_planted_mistake_is_caught():
    """Without the remainder step (q = RN(v * RN(1/z)) alone) the comparison finds differences."""
    diff = 0
    for v, z in _cases()[:2500]:
        v32, z32 = np.float32(v), np.float32(z)
        rz = np.float32(1.0) / z32
        if _bits(_rn32(Fraction(float(v32)) * Fraction(float(rz)))) != _bits(v32 / z32):
            diff += 1
    assert diff > 0


@pytest.mark.parametrize("v,z", [(float("nan"), 3.0), (0.25, float("nan"))])
def test_nan_propagates(v, z):
    v32, z32 = np.float32(v), np.float32(z)
    rz = np.float32(1.0) / z32
    q = v32 * rz
    with np.errstate(invalid="ignore"):
        rem = np.float32(-q * z32 + v32)  # NaN in, NaN out, with or without fusion
        assert np.isnan(np.float32(rem * rz + q))
