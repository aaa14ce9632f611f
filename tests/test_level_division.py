"""The leave grid's division (quant_step, app_core.c:1930-1940, as
rint(y / leave)) is computed on the GPU as q = fl(y r), r = fl(1 / leave), then
fl(q + fl(y - q leave) r) with two fused multiply-adds (div_leave in
igl_gemm_level.hip).  This pins that sequence to the correctly rounded binary32
quotient in exact rational arithmetic: near-ties at every half-integer quotient
of the clamp range, random quotients, and leave values including all-ones
mantissas, powers of two and the grids the tests use."""
from fractions import Fraction

import numpy as np


def rn32(x: Fraction) -> Fraction:
    """x rounded to the nearest binary32 (ties to even), normal range."""
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    elif Fraction(2) ** (e + 1) <= a:
        e += 1
    scale = Fraction(2) ** (23 - e)
    m = a * scale
    whole = m.numerator // m.denominator
    rest = m - whole
    if rest > Fraction(1, 2) or (rest == Fraction(1, 2) and whole % 2 == 1):
        whole += 1
    return sign * Fraction(whole) / scale


def f32(v) -> Fraction:
    return Fraction(float(np.float32(v)))


def device_div(y: Fraction, leave: Fraction) -> Fraction:
    r = rn32(1 / leave)
    q = rn32(y * r)
    e = rn32(y - q * leave)
    return rn32(e * r + q)


def test_rn32_matches_numpy():
    rng = np.random.default_rng(0)
    for _ in range(2000):
        a, b = np.float32(rng.normal()), np.float32(rng.normal() + 3.0)
        assert rn32(Fraction(float(a)) / Fraction(float(b))) == Fraction(float(a / b))
        assert rn32(Fraction(float(a)) * Fraction(float(b))) == Fraction(float(a * b))


def test_corrected_division_is_correctly_rounded():
    rng = np.random.default_rng(1)
    leaves = [0.02, 2.5 / 127, 0.0625, 1.0 / 3.0, 0.1, 7.0e-4, 3.0]
    ones = np.float32(2.0)
    for _ in range(4):
        ones = np.nextafter(ones, np.float32(0.0))  # mantissas of all ones and neighbours
        leaves.append(float(ones) * 0.01)
    leaves += [float(np.float32(abs(rng.normal()) * 0.05 + 1e-4)) for _ in range(6)]
    checked = 0
    for lv in leaves:
        leave = f32(lv)
        ys = []
        # near-ties: quotients k + 1/2 for every level of the clamp range and beyond
        for k in range(-135, 135):
            t = np.float32((k + 0.5) * float(leave))
            ys.append(t)
            for _ in range(3):
                t_up = np.nextafter(ys[-1], np.float32(np.inf))
                ys.append(t_up)
            t = np.float32((k + 0.5) * float(leave))
            for _ in range(3):
                t = np.nextafter(t, np.float32(-np.inf))
                ys.append(t)
        ys += list((rng.normal(size=600) * 60.0 * float(leave)).astype(np.float32))
        for y in ys:
            yf = Fraction(float(y))
            if yf == 0:
                continue
            assert device_div(yf, leave) == rn32(yf / leave), (float(y), lv)
            checked += 1
    assert checked > 20000
