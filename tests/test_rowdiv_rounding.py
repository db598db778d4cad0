"""The per-row division of k_row_softmax / k_row_layernorm (RowDiv in
csrc/pt_reduce.hip): with rb = RN(1/b), q0 = RN(a rb), r = RN(a - b q0)
(one fma) and q = RN(q0 + r rb) (one fma), q equals the correctly rounded
fp32 quotient RN(a/b) whenever a, b and a/b are normal (Markstein's
theorem); a quotient with |q0| <= FLT_MIN takes the IEEE division instead.
Checked here in exact rational arithmetic, every rounding done once and to
nearest-even on the binary32 grid (subnormals included), on the operand
ranges the kernels see: softmax divides exp values in (0, 1] by a row sum
in [1, n], layerNorm divides centred values by sqrt(var + eps), and
softmax values down to the subnormal range.  Pure CPU; no GPU code runs."""
from fractions import Fraction

import numpy as np
import pytest


FLT_MIN = Fraction(2) ** -126


def rn32(x):
    """Round an exact rational to the nearest binary32 (ties to even),
    subnormals included (quantum 2^-149 below 2^-126); no overflow."""
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    x = abs(x)
    e = x.numerator.bit_length() - x.denominator.bit_length()
    if Fraction(2) ** e > x:
        e -= 1
    assert Fraction(2) ** e <= x < Fraction(2) ** (e + 1)
    assert e <= 127, "no overflow"
    e = max(e, -126)                                # subnormal: fixed quantum
    m = x / Fraction(2) ** (e - 23)
    q, r = divmod(m.numerator, m.denominator)
    if 2 * r > m.denominator or (2 * r == m.denominator and q % 2 == 1):
        q += 1
    return sign * Fraction(q) * Fraction(2) ** (e - 23)


def markstein(a, b):
    rb = rn32(1 / b)
    q0 = rn32(a * rb)
    r = rn32(a - b * q0)
    return q0, rn32(q0 + r * rb)


def rowdiv(a, b):
    """RowDiv::operator(): the IEEE quotient when |q0| <= FLT_MIN."""
    q0, q = markstein(a, b)
    return rn32(a / b) if abs(q0) <= FLT_MIN else q


def f32(v):
    return Fraction(float(np.float32(v)))


@pytest.mark.parametrize("case", ["softmax", "layernorm", "wide"])
def test_rowdiv_is_correctly_rounded(case):
    rng = np.random.default_rng({"softmax": 1, "layernorm": 2, "wide": 3}[case])
    count = 1500
    if case == "softmax":
        # exp values down to e^-60, so that quotient and remainder stay normal
        a = np.exp(-rng.uniform(0, 60, count)).astype(np.float32)
        b = rng.uniform(1, 4096, count).astype(np.float32)
    elif case == "layernorm":
        a = rng.normal(0, 3, count).astype(np.float32)
        b = np.sqrt(rng.uniform(1e-4, 50, count)).astype(np.float32)
    else:
        a = (rng.uniform(1, 2, count) * 2.0 ** rng.integers(-60, 60, count)).astype(np.float32)
        b = (rng.uniform(1, 2, count) * 2.0 ** rng.integers(-60, 60, count)).astype(np.float32)
    for x, y in zip(a, b):
        fa, fb = f32(x), f32(y)
        if fa == 0:
            continue
        assert rowdiv(fa, fb) == rn32(fa / fb), (float(fa), float(fb))


def test_rowdiv_halfway_quotients():
    """Quotients whose exact value lies on or next to a rounding boundary:
    a = b * (m + 1/2 ulp) rounded, around every power of two of b."""
    for eb in range(0, 13):
        for mb in (1, 3, 5, 7, 1023, 4095, (1 << 23) - 1):
            b = Fraction((1 << 23) + mb, 1 << 23) * Fraction(2) ** eb
            for mq in (0, 1, 2, (1 << 22), (1 << 23) - 1):
                q = Fraction((1 << 23) + mq, 1 << 23) * Fraction(2) ** -3
                half = Fraction(1, 1 << 27)             # half an ulp of q
                for t in (q, q + half, q - half):
                    a = rn32(b * t)
                    assert rowdiv(a, b) == rn32(a / b)


def test_rowdiv_subnormal_quotients():
    """Softmax values whose quotient by the row sum is subnormal or at the
    normal boundary (exp arguments from about -87 to -104): the guard takes
    the IEEE division there, so every quotient is correctly rounded; the
    unguarded three-instruction form is off by an ulp on some of these,
    which is what the guard is for."""
    rng = np.random.default_rng(4)
    off = 0
    for _ in range(1500):
        b = f32(rng.uniform(1, 4096))
        # a / b between 2^-149 and 2^-125
        a = f32(float(b) * 2.0 ** rng.uniform(-148, -125))
        if a == 0:
            continue
        assert rowdiv(a, b) == rn32(a / b), (float(a), float(b))
        off += markstein(a, b)[1] != rn32(a / b)
    assert off > 0
    # q0 exactly at FLT_MIN: the guard is inclusive
    b = Fraction(3)
    a = rn32(FLT_MIN * b)
    assert rowdiv(a, b) == rn32(a / b)
