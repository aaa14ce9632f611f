"""The grid divisions (quant_step, app_core.c:1930-1940, as rint(y / leave)
and rint(x / step)) are computed on the GPU as q = fl(y r), r = fl(1 / leave),
then fl(q + fl(y - q leave) r) with two fused multiply-adds (quot_near in
igl_device.h: the fused GEMV's activation levels, and div_leave in
igl_gemm_level.hip: the leave grid), for steps in [2^-96, 2^96] (level_recip;
outside it the kernels divide), with fl(y r) first clamped to [-256, 256]
(beyond it the level clamps alike).  This pins that sequence to the
correctly rounded binary32 quotient in exact rational arithmetic: near-ties at
every half-integer quotient of the clamp range, random quotients, and leave
values including all-ones mantissas, powers of two, both ends of the range
and the grids the tests use."""
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


def quot_near(x: Fraction, step: Fraction):
    """quot_near of igl_device.h in exact arithmetic, each operation rounded
    once; returns (value, corrected): corrected is False where q0 was clamped
    (the quotient's magnitude is then at least 256)."""
    inv = rn32(1 / step)
    q0 = rn32(x * inv)
    clamped = abs(q0) > 256
    q0 = max(min(q0, Fraction(256)), Fraction(-256))
    r = rn32(x - q0 * step)
    return rn32(r * inv + q0), not clamped


def clamp_level(q: float) -> float:
    return min(max(float(np.rint(q)), -128.0), 127.0)


def test_quot_near_range_ends():
    """Steps at both ends of [2^-96, 2^96] (powers of two and all-ones
    mantissas) and the usual grids: below 256 the corrected quotient is the
    correctly rounded one; at and above it the level clamps as the quotient's."""
    ones = float(np.nextafter(np.float32(2.0), np.float32(0.0)))  # 2 - 2^-23
    steps = [2.0 ** -96, ones * 2.0 ** -96, 2.0 ** 96, ones * 2.0 ** 95, 2.5 / 127, 0.02, 3.0]
    rng = np.random.default_rng(3)
    checked = 0
    for st in steps:
        step = f32(st)
        xs = []
        for k in list(range(-131, 131, 3)) + [-129, -128, 126, 127, 255, 256]:
            t = np.float32((k + 0.5) * float(step))
            xs += [t, np.nextafter(t, np.float32(np.inf)), np.nextafter(t, np.float32(-np.inf))]
        xs += list((rng.normal(size=200) * 90.0 * float(step)).astype(np.float32))
        xs += list((rng.normal(size=40) * 5000.0 * float(step)).astype(np.float32))
        for x in xs:
            xf = Fraction(float(x))
            if xf == 0:
                continue
            got, corrected = quot_near(xf, step)
            want = rn32(xf / step)
            if corrected:
                assert got == want, (float(x), st)
            else:
                assert clamp_level(float(got)) == clamp_level(float(want)), (float(x), st)
            checked += 1
    assert checked > 3000


def device_quot_f32(x, st):
    """quot_near in binary32 with numpy, each fma as a float64 product (exact
    for two binary32 values) and sum rounded to binary32; only the clamped
    levels of these special cases are compared."""
    inv = np.float32(1.0) / st
    q0 = np.float32(np.clip(np.float32(x * inv), -256.0, 256.0)) if not np.isnan(x * inv) else np.float32(256.0)
    r = np.float32(np.float64(x) - np.float64(q0) * np.float64(st))
    return np.float32(np.float64(r) * np.float64(inv) + np.float64(q0))


def test_quot_near_specials_clamp_alike():
    """Overflowing and non-finite quotients in binary32: fl(x r) overflowing
    to infinity is clamped to 256 and the result clamps to the same level as
    the quotient; NaN stays NaN (whatever the clamp gives for it); zero stays
    zero."""
    with np.errstate(over="ignore", invalid="ignore"):
        for x, st in [(3.0e38, 0.01), (-3.0e38, 0.01), (np.inf, 0.5), (-np.inf, 0.5), (np.nan, 0.5),
                      (0.0, 2.0 ** -96), (300.0, 1.0), (-1000.0, 1.0), (255.75, 1.0), (-128.5, 1.0)]:
            x, st = np.float32(x), np.float32(st)
            got = device_quot_f32(x, st)
            want = x / st
            if np.isnan(want):
                assert np.isnan(got)
            else:
                assert clamp_level(got) == clamp_level(want), (float(x), float(st), float(got))
