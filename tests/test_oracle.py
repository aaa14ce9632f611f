"""Pins the oracle (oracle/igl_oracle.c) before anything is held against it.

Each check is chosen so that a plausible slip in the restatement (nibble
order, a dropped bias term, a wrong sign, a transposed index, a changed
summation order) fails:
  * the reference's own known-answer vectors (app_test.c test_gemma, test_cache);
  * an independent bit writer and closed forms in float64;
  * the reference itself, compiled from its source into oracle/_ref, to the bit.
"""
import ctypes
import math

import numpy as np
import pytest

import oracle_lib as ol

rng = np.random.default_rng(1234)


def pack_fields(values, bits):
    """Independent little-endian bit writer (the role of test_pack_write,
    app_test.c:378-385)."""
    total = len(values) * bits
    out = bytearray((total + 7) // 8 + 8)
    for i, v in enumerate(values):
        for b in range(bits):
            if (int(v) >> b) & 1:
                pos = i * bits + b
                out[pos // 8] |= 1 << (pos % 8)
    return np.frombuffer(bytes(out), dtype=np.uint8).copy()


# ---- quant layer --------------------------------------------------------------

def quant_step_inputs():
    """Values for the activation grid: normals at several scales, exact ties
    (k + 1/2) step for a power-of-two step, values past both clamps, signed
    zeros, infinities and NaN."""
    rng = np.random.default_rng(5)
    vals = [rng.normal(size=400) * s for s in (0.01, 1.0, 30.0)]
    vals.append((np.arange(-140, 140) + 0.5) * 0.0625)
    vals.append(np.array([-1e9, 1e9, -8.03, 7.97, 0.0, -0.0, np.inf, -np.inf, np.nan]))
    return np.concatenate(vals).astype(np.float32)


def quant_step_closed(x, step):
    """rint(x / step) in float32, clamped by comparisons (NaN passes), times step."""
    x = np.asarray(x, dtype=np.float32)
    if not step > 0:
        return x.copy()
    with np.errstate(invalid="ignore", over="ignore"):
        level = np.rint(x / np.float32(step)).astype(np.float32)
    level = np.where(level < -128, np.float32(-128), level)
    level = np.where(level > 127, np.float32(127), level)
    return (level * np.float32(step)).astype(np.float32)


@pytest.mark.parametrize("step", [0.0625, 0.1, 3.7, 1e-30, 0.0, -1.0, float("nan")])
def test_quant_step_pinned(step):
    """oracle_quant_step (app_core.c:1930-1940) against numpy's float32 closed
    form (ties to even, both clamps, NaN through, non-positive steps inert) and,
    where it was built, the reference's own quant_step."""
    x = quant_step_inputs()
    want = quant_step_closed(x, step)
    got = np.array([ol.oracle().oracle_quant_step(float(v), step) for v in x], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    ref = ol.ref("plain")
    if ref is not None:
        got_ref = np.array([ref.ref_quant_step(float(v), step) for v in x], dtype=np.float32)
        assert np.array_equal(got_ref.view(np.uint32), want.view(np.uint32))
    if step == 0.0625:
        # the ties went to even levels
        ties = x[1200:1480]
        assert np.all(np.rint(ties / np.float32(step)) % 2 == 0)


def test_nibble_kat():
    """app_test.c:593-594: {0x98,0xBA,0x21,0x0F} are 0,1,2,3,-7,-6,7,-8 (code - 8)."""
    row = np.array([0x98, 0xBA, 0x21, 0x0F], dtype=np.uint8)
    vals = [int(ol.oracle().oracle_pack_read(ol.p(row), i, 4)) - 8 for i in range(8)]
    assert vals == [0, 1, 2, 3, -7, -6, 7, -8]


def test_plane_row_kat():
    """app_test.c:651-658: three rows of the same bytes, one scale a row (0.5, 1, 2)."""
    codes = np.tile(np.array([0x98, 0xBA, 0x21, 0x0F], dtype=np.uint8), (3, 1))
    gains = np.array([[0.5], [1.0], [2.0]], dtype=np.float32)
    d = ol.plane_desc(codes, gains, 8, group_size=8)
    row = np.zeros(8, dtype=np.float32)
    ol.oracle().oracle_plane_row(ctypes.byref(d), 0, ol.p(row))
    assert row[0] == 0.0 and row[3] == 1.5 and row[4] == -3.5 and row[7] == -4.0
    ol.oracle().oracle_plane_row(ctypes.byref(d), 2, ol.p(row))
    assert row[6] == 14.0


def test_signed_byte_kat():
    """app_test.c:663-686: signed bytes with flip 128 / bias 128; row_code -149.25, -298.5."""
    codes = np.tile(np.array([0x00, 0x01, 0x7F, 0xFF, 0x80, 0xC8], dtype=np.uint8), (2, 1))
    gains = np.array([[0.25], [0.5]], dtype=np.float32)
    d = ol.plane_desc(codes, gains, 6, group_size=6, bits=8, code_bias=128, code_flip=128)
    row = np.zeros(6, dtype=np.float32)
    ol.oracle().oracle_plane_row(ctypes.byref(d), 0, ol.p(row))
    assert (row[2], row[3], row[4], row[5]) == (31.75, -0.25, -32.0, -14.0)
    act = np.arange(1, 7, dtype=np.float32)
    sums = np.array([act.sum()], dtype=np.float32)
    assert abs(ol.oracle().oracle_row_code(ctypes.byref(d), 0, ol.p(act), ol.p(sums)) + 149.25) < 1e-4
    assert abs(ol.oracle().oracle_row_code(ctypes.byref(d), 1, ol.p(act), ol.p(sums)) + 298.5) < 1e-4


def test_two_bit_kat():
    """app_test.c:688-702: two-bit codes, group 4, per-group scales."""
    codes = np.tile(np.array([0x1B, 0xE4], dtype=np.uint8), (2, 1))
    gains = np.array([[1.0, 4.0], [0.5, 2.0]], dtype=np.float32)
    d = ol.plane_desc(codes, gains, 8, group_size=4, bits=2, code_bias=2)
    row = np.zeros(8, dtype=np.float32)
    ol.oracle().oracle_plane_row(ctypes.byref(d), 0, ol.p(row))
    assert (row[0], row[3], row[4], row[7]) == (1.0, -2.0, -8.0, 4.0)
    ol.oracle().oracle_plane_row(ctypes.byref(d), 1, ol.p(row))
    assert row[4] == -4.0


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 7, 8, 13])
def test_pack_read_vs_writer(bits):
    vals = rng.integers(0, 1 << bits, size=301)
    stream = pack_fields(vals, bits)
    got = [ol.oracle().oracle_pack_read(ol.p(stream), i, bits) for i in range(len(vals))]
    assert got == [int(v) for v in vals]


# ---- projection ---------------------------------------------------------------

def closed_form(codes, gains, act, K, group, bits=4, bias=8):
    """y = sum_g s[n,g] * sum_{k in g} (c - bias) x, in float64."""
    N = codes.shape[0]
    c = np.empty((N, K), dtype=np.float64)
    for k in range(K):
        byte = codes[:, (k * bits) // 8].astype(np.int64)
        if bits == 4:
            c[:, k] = (byte >> (4 * (k & 1))) & 15
        else:
            c[:, k] = [ol.oracle().oracle_pack_read(ol.p(codes[n]), k, bits) for n in range(N)]
    w = (c - bias) * np.repeat(gains.astype(np.float64), group, axis=1)[:, :K]
    return act.astype(np.float64) @ w.T


@pytest.mark.parametrize("N,K,lanes", [(70, 128, 1), (70, 128, 5), (33, 2048, 3), (64, 96, 19)])
def test_mat_mat_closed_form(N, K, lanes):
    codes = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    gains = np.abs(rng.normal(0, 0.02, size=(N, K // 32))).astype(np.float32)
    act = rng.normal(size=(lanes, K)).astype(np.float32)
    got = ol.oracle_mat_mat(codes, gains, act, K, 32, threads=3)
    want = closed_form(codes, gains, act, K, 32)
    scale = np.sqrt(np.mean(want ** 2))
    assert np.max(np.abs(got - want)) <= 1e-5 * scale * math.sqrt(K / 32) + 1e-7


def test_planted_bias_slip_is_caught():
    """A restatement that dropped the code_bias term would miss the closed form."""
    N, K = 16, 64
    codes = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    gains = np.abs(rng.normal(0, 0.02, size=(N, K // 32))).astype(np.float32)
    act = rng.normal(size=(1, K)).astype(np.float32)
    wrong = ol.oracle_mat_mat(codes, gains, act, K, 32, code_bias=0)
    want = closed_form(codes, gains, act, K, 32)
    assert np.max(np.abs(wrong - want)) > 1e-2


@pytest.mark.parametrize("N,K,group,bits,lanes,threads", [
    (70, 128, 32, 4, 1, 1), (70, 128, 32, 4, 4, 3), (70, 130, 48, 4, 19, 3),
    (96, 2048, 32, 4, 8, 4), (40, 8192, 32, 4, 2, 2), (70, 128, 32, 2, 3, 1),
    (70, 128, 32, 8, 5, 3), (33, 96, 32, 3, 2, 1),
])
def test_mat_mat_bitexact_vs_reference(ref_plain, N, K, group, bits, lanes, threads):
    """The oracle and the reference's own back_mat_mat (plain build) agree to the bit."""
    stride = (K * bits + 7) // 8
    codes = rng.integers(0, 256, size=(N, stride), dtype=np.uint8)
    G = (K + group - 1) // group
    gains = np.abs(rng.normal(0, 0.02, size=(N, G))).astype(np.float32)
    act = rng.normal(size=(lanes, K)).astype(np.float32)
    kw = dict(bits=bits, code_bias=1 << (bits - 1))
    got = ol.oracle_mat_mat(codes, gains, act, K, group, threads=threads, **kw)
    want = ol.ref_mat_mat(ref_plain, codes, gains, act, K, group, threads=threads, **kw)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# The shipped export's kinds: one gain a row (group = K), signed I8 (flip 128),
# 2-bit MLP / head planes, 4-bit per-channel attention planes.
SHIPPED_KINDS = [
    (70, 1536, 1536, 8, 128, 3), (40, 256, 256, 8, 128, 1), (64, 1536, 1536, 2, 0, 2),
    (33, 6144, 6144, 2, 0, 1), (50, 1536, 1536, 4, 0, 4), (24, 8960, 256, 4, 0, 2),
    (20, 96, 96, 2, 1, 3), (20, 96, 32, 8, 0, 2), (20, 96, 96, 4, 5, 1),
]


@pytest.mark.parametrize("N,K,group,bits,flip,lanes", SHIPPED_KINDS)
def test_shipped_kinds_closed_form(N, K, group, bits, flip, lanes):
    """y = sum_g s[n,g] sum_{k in g} ((c ^ flip) - bias) x in float64."""
    stride = (K * bits + 7) // 8
    codes = rng.integers(0, 256, size=(N, stride), dtype=np.uint8)
    G = (K + group - 1) // group
    gains = np.abs(rng.normal(0, 0.02, size=(N, G))).astype(np.float32)
    act = rng.normal(size=(lanes, K)).astype(np.float32)
    bias = 1 << (bits - 1)
    got = ol.oracle_mat_mat(codes, gains, act, K, group, threads=2, bits=bits, code_bias=bias,
                            code_flip=flip)
    fields = np.unpackbits(codes, axis=1, bitorder="little")[:, :K * bits].reshape(N, K, bits)
    c = (fields.astype(np.int64) << np.arange(bits)).sum(axis=2) ^ flip
    w = (c - bias).astype(np.float64) * np.repeat(gains.astype(np.float64), group, axis=1)[:, :K]
    want = act.astype(np.float64) @ w.T
    scale = np.sqrt(np.mean(want ** 2))
    assert np.max(np.abs(got - want)) <= 2e-6 * scale * math.sqrt(K / 32) + 1e-7
    if flip:  # a restatement that dropped the flip misses the closed form
        wrong = ol.oracle_mat_mat(codes, gains, act, K, group, bits=bits, code_bias=bias)
        assert np.max(np.abs(wrong - want)) > 1e-3 * scale


@pytest.mark.parametrize("N,K,group,bits,flip,lanes", SHIPPED_KINDS)
def test_shipped_kinds_bitexact_vs_reference(ref_plain, N, K, group, bits, flip, lanes):
    stride = (K * bits + 7) // 8
    codes = rng.integers(0, 256, size=(N, stride), dtype=np.uint8)
    G = (K + group - 1) // group
    gains = np.abs(rng.normal(0, 0.02, size=(N, G))).astype(np.float32)
    act = rng.normal(size=(lanes, K)).astype(np.float32)
    kw = dict(bits=bits, code_bias=1 << (bits - 1), code_flip=flip)
    got = ol.oracle_mat_mat(codes, gains, act, K, group, threads=2, **kw)
    want = ol.ref_mat_mat(ref_plain, codes, gains, act, K, group, threads=2, **kw)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ---- zero points (asymmetric planes) -------------------------------------------

ZERO_CASES = [(70, 128, 32, 4, 1), (70, 256, 32, 4, 5), (40, 1536, 128, 4, 3), (33, 256, 32, 2, 2),
              (33, 512, 64, 2, 1), (24, 256, 32, 8, 4), (24, 512, 512, 8, 1), (70, 130, 48, 4, 19)]


def zero_inputs(N, K, group, bits, lanes, seed=11):
    r = np.random.default_rng(seed)
    stride = (K * bits + 7) // 8
    codes = r.integers(0, 256, size=(N, stride), dtype=np.uint8)
    G = (K + group - 1) // group
    gains = np.abs(r.normal(0, 0.02, size=(N, G))).astype(np.float32)
    half = 1 << (bits - 1)
    zeros = r.integers(-half, half, size=(N, G)).astype(np.int8)
    act = r.normal(size=(lanes, K)).astype(np.float32)
    return codes, gains, zeros, act


def zero_closed(codes, gains, zeros, act, K, group, bits, sign=1):
    """sum_g s[n,g] sum_{k in g} (c - bias - zero[n,g]) x in float64 (sign=-1
    plants the slip of adding the zero point instead)."""
    N = codes.shape[0]
    fields = np.unpackbits(codes, axis=1, bitorder="little")[:, :K * bits].reshape(N, K, bits)
    c = (fields.astype(np.int64) << np.arange(bits)).sum(axis=2).astype(np.float64)
    z = np.repeat(zeros.astype(np.float64), group, axis=1)[:, :K]
    w = (c - (1 << (bits - 1)) - sign * z) * np.repeat(gains.astype(np.float64), group, axis=1)[:, :K]
    return act.astype(np.float64) @ w.T


@pytest.mark.parametrize("N,K,group,bits,lanes", ZERO_CASES)
def test_zero_points_closed_form(N, K, group, bits, lanes):
    """plane_row's (code - bias - zero) gain (app_core.c:1849-1852) summed in
    float64; a restatement that added the zero point misses it."""
    codes, gains, zeros, act = zero_inputs(N, K, group, bits, lanes)
    kw = dict(bits=bits, code_bias=1 << (bits - 1), zeros=zeros)
    got = ol.oracle_mat_mat(codes, gains, act, K, group, threads=2, **kw)
    want = zero_closed(codes, gains, zeros, act, K, group, bits)
    scale = np.sqrt(np.mean(want ** 2))
    assert np.max(np.abs(got - want)) <= 2e-6 * scale * math.sqrt(K / 32) + 1e-7
    wrong = zero_closed(codes, gains, zeros, act, K, group, bits, sign=-1)
    assert np.max(np.abs(wrong - want)) > 1e-2 * scale


@pytest.mark.parametrize("N,K,group,bits,lanes", ZERO_CASES)
def test_zero_points_bitexact_vs_reference(ref_plain, N, K, group, bits, lanes):
    """With zero points the oracle and the reference's own back_mat_mat (plain
    build, kern_row_code / kern_row_code_many: (bias + zero) sum per group)
    agree to the bit."""
    codes, gains, zeros, act = zero_inputs(N, K, group, bits, lanes)
    kw = dict(bits=bits, code_bias=1 << (bits - 1), zeros=zeros)
    got = ol.oracle_mat_mat(codes, gains, act, K, group, threads=2, **kw)
    want = ol.ref_mat_mat(ref_plain, codes, gains, act, K, group, threads=2, **kw)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("bits,rows,groups", [(2, 70, 3), (4, 33, 5), (8, 24, 2), (4, 8, 1), (3, 50, 4)])
def test_zero_unpack_matches_reference_zero_read(ref_plain, bits, rows, groups):
    """The engine's loader unpacks weight_zero_point (I32, each group's zero
    points packed along the rows) as the reference's zero_read
    (app_core.c:7855-7866) reads it, row by row and group by group; 3-bit
    fields straddle words."""
    from igllm_amd import native

    r = np.random.default_rng(bits * 100 + rows)
    words = r.integers(0, 1 << 32, size=((rows * bits + 31) // 32 + 1, groups), dtype=np.uint64).astype(np.uint32)
    out = np.zeros((rows, groups), dtype=np.int8)
    native.load().igl_zero_unpack(ol.p(words), groups, rows, bits, ol.p(out))
    want = np.array([[ref_plain.ref_zero_read(ol.p(words), groups, g, n, bits) for g in range(groups)]
                     for n in range(rows)])
    assert np.array_equal(out.astype(np.int64), want)
    assert want.min() >= -(1 << (bits - 1)) and want.max() < (1 << (bits - 1))


# ---- calibrated planes: the integer level path --------------------------------

LEVEL_CASES = [
    (70, 1536, 1536, 4, 0, 1), (70, 1536, 1536, 4, 0, 3), (40, 1536, 1536, 2, 0, 2),
    (40, 256, 256, 8, 128, 5), (33, 6144, 6144, 2, 0, 1), (20, 512, 128, 4, 0, 2),
    (24, 1536, 1536, 8, 0, 17), (20, 96, 32, 4, 0, 1),
]


def level_inputs(N, K, group, bits, lanes, seed=5):
    r = np.random.default_rng(seed)
    stride = (K * bits + 7) // 8
    codes = r.integers(0, 256, size=(N, stride), dtype=np.uint8)
    gains = np.abs(r.normal(0, 0.02, size=(N, (K + group - 1) // group))).astype(np.float32)
    act = r.normal(size=(lanes, K)).astype(np.float32)
    return codes, gains, act, np.float32(2.5 / 127)  # values past 2.5 clip to the ends


def level_closed(codes, gains, act, K, group, bits, flip, step):
    """sum over groups of gain * step * sum ((c ^ flip) - bias) L in float64,
    L the numpy float32 quant_step level."""
    N = codes.shape[0]
    fields = np.unpackbits(codes, axis=1, bitorder="little")[:, :K * bits].reshape(N, K, bits)
    c = (fields.astype(np.int64) << np.arange(bits)).sum(axis=2) ^ flip
    L = np.clip(np.rint(act / step), -128, 127).astype(np.float64)
    w = (c - (1 << (bits - 1))).astype(np.float64) * np.repeat(gains.astype(np.float64), group, axis=1)[:, :K]
    return (L * float(step)) @ w.T


@pytest.mark.parametrize("N,K,group,bits,flip,lanes", LEVEL_CASES)
def test_level_closed_form(N, K, group, bits, flip, lanes):
    codes, gains, act, step = level_inputs(N, K, group, bits, lanes)
    kw = dict(bits=bits, code_bias=1 << (bits - 1), code_flip=flip)
    got = ol.oracle_mat_mat_level(codes, gains, act, K, group, float(step), **kw)
    want = level_closed(codes, gains, act, K, group, bits, flip, step)
    scale = np.sqrt(np.mean(want ** 2))
    assert np.max(np.abs(got - want)) <= 1e-6 * scale * math.sqrt(K / group)
    # a restatement that took x instead of its level misses it
    plain = ol.oracle_mat_mat(codes, gains, act, K, group, **kw)
    assert np.max(np.abs(plain - want)) > 1e-4 * scale


def test_level_one_group_is_one_rounding():
    """One gain a row: y = fl(fl(gain * step) * fl(part)), part the exact integer sum."""
    N, K, bits = 50, 1536, 4
    codes, gains, act, step = level_inputs(N, K, K, bits, 2)
    got = ol.oracle_mat_mat_level(codes, gains, act, K, K, float(step), bits=bits, code_bias=8)
    fields = np.unpackbits(codes, axis=1, bitorder="little")[:, :K * bits].reshape(N, K, bits)
    c = (fields.astype(np.int64) << np.arange(bits)).sum(axis=2) - 8
    L = np.clip(np.rint(act / step), -128, 127).astype(np.int64)
    part = L @ c.T
    want = (gains[:, 0] * step)[None, :] * part.astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))


def test_level_off_grid_takes_float_path():
    """Groups of 32 are not level-ready, and a NaN puts a chunk off the grid:
    both go to the float path on the quant_step values."""
    codes, gains, act, step = level_inputs(20, 96, 32, 4, 2)
    want = ol.oracle_mat_mat(codes, gains, ol.quant_step(act, float(step)), 96, 32)
    got = ol.oracle_mat_mat_level(codes, gains, act, 96, 32, float(step))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    codes, gains, act, step = level_inputs(20, 1536, 1536, 4, 3)
    act[1, 7] = np.nan
    want = ol.oracle_mat_mat(codes, gains, ol.quant_step(act, float(step)), 1536, 1536)
    got = ol.oracle_mat_mat_level(codes, gains, act, 1536, 1536, float(step))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.all(np.isnan(got[1]))


@pytest.mark.parametrize("N,K,group,bits,flip,lanes", [c for c in LEVEL_CASES if c[2] % 64 == 0])
def test_level_bitexact_vs_reference(N, K, group, bits, flip, lanes):
    """The oracle against the reference's own VNNI build on quant_step'd lanes
    (level-ready planes: off the grid, that build's float path is its AVX-512
    one, not the SSE2 order the oracle restates)."""
    lib = ol.ref("level")
    if lib is None:
        pytest.skip("level build of oracle/_ref absent, or this host has no AVX-512 VNNI")
    codes, gains, act, step = level_inputs(N, K, group, bits, lanes)
    kw = dict(bits=bits, code_bias=1 << (bits - 1), code_flip=flip)
    got = ol.oracle_mat_mat_level(codes, gains, act, K, group, float(step), **kw)
    want = ol.ref_mat_mat_step(lib, codes, gains, ol.quant_step(act, float(step)), K, group, float(step),
                               threads=2, **kw)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def real_rows(N, K, real_type):
    """Rows of a real plane and their values in float64."""
    w = rng.normal(0, 0.05, size=(N, K)).astype(np.float32)
    if real_type == ol.REAL_F32:
        return w, w.astype(np.float64)
    if real_type == ol.REAL_F16:
        h = w.astype(np.float16)
        return h.view(np.uint16), h.astype(np.float64)
    b = (w.view(np.uint32) >> 16).astype(np.uint16)
    return b, (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


@pytest.mark.parametrize("real_type", [ol.REAL_F32, ol.REAL_F16, ol.REAL_BF16])
@pytest.mark.parametrize("N,K,lanes", [(70, 1536, 1), (33, 1541, 3), (20, 7, 2)])
def test_real_plane_closed_form(real_type, N, K, lanes):
    raw, w64 = real_rows(N, K, real_type)
    act = rng.normal(size=(lanes, K)).astype(np.float32)
    got = ol.oracle_mat_mat_real(raw, real_type, act)
    want = act.astype(np.float64) @ w64.T
    scale = np.sqrt(np.mean(want ** 2))
    assert np.max(np.abs(got - want)) <= 2e-6 * scale * math.sqrt(K)
    if real_type == ol.REAL_BF16:  # reading the bits as binary16 misses it
        wrong = ol.oracle_mat_mat_real(raw, ol.REAL_F16, act)
        assert not np.allclose(wrong, want, rtol=1e-2)


@pytest.mark.parametrize("real_type", [ol.REAL_F32, ol.REAL_F16, ol.REAL_BF16])
@pytest.mark.parametrize("N,K,lanes", [(70, 1536, 1), (33, 1541, 3), (96, 8960, 2)])
def test_real_plane_bitexact_vs_reference(ref_plain, real_type, N, K, lanes):
    raw, _ = real_rows(N, K, real_type)
    act = rng.normal(size=(lanes, K)).astype(np.float32)
    got = ol.oracle_mat_mat_real(raw, real_type, act)
    want = ol.ref_mat_mat_real(ref_plain, raw, real_type, act, threads=2)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ---- FP8 codec ----------------------------------------------------------------

def e4m3_definition(code):
    sign = -1.0 if code & 0x80 else 1.0
    e, m = (code >> 3) & 15, code & 7
    return sign * (m * 2.0 ** -9 if e == 0 else (8 + m) * 2.0 ** (e - 10))


def test_real8_all_codes():
    for c in range(256):
        assert ol.oracle().oracle_real8(c) == e4m3_definition(c)
    assert ol.oracle().oracle_real8(0x7F) == 480.0 and ol.oracle().oracle_real8(0xFF) == -480.0


def test_real8_matches_torch_e4m3fn():
    torch = pytest.importorskip("torch")
    codes = torch.arange(256, dtype=torch.uint8)
    vals = codes.view(torch.float8_e4m3fn).float().numpy()
    for c in range(256):
        if c in (0x7F, 0xFF):
            assert math.isnan(vals[c])  # OCP e4m3fn spends these on NaN; the reference reads 480
        else:
            assert ol.oracle().oracle_real8(c) == vals[c]


def test_code8_round_trip_and_saturation():
    lib = ol.oracle()
    for c in range(256):
        if c in (0x7F, 0xFF, 0x80):
            continue
        assert lib.oracle_code8(lib.oracle_real8(c)) == c
    assert lib.oracle_code8(1e9) == 0x7E and lib.oracle_code8(-1e9) == 0xFE
    assert lib.oracle_code8(float("nan")) == 0x7E
    assert lib.oracle_code8(-0.0) == 0x00


def test_code8_matches_torch_rounding():
    torch = pytest.importorskip("torch")
    x = np.concatenate([rng.normal(0, 30, 20000), rng.normal(0, 0.01, 20000),
                        rng.uniform(-448, 448, 20000)]).astype(np.float32)
    x = x[np.abs(x) <= 448.0]  # torch does not saturate (NaN); the reference does, tested above
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = ol.encode(x, 1.0, 0)
    # The one deliberate difference: a negative value that rounds to zero is
    # stored as +0 by the reference (cache_code8 tests `size < 0` on -0.0,
    # app_core.c:11010) and as -0 (0x80) by torch.
    differ = got != want
    assert np.all((got[differ] == 0x00) & (want[differ] == 0x80))
    assert np.all(x[differ] < 0) and np.all(np.abs(x[differ]) <= 2.0 ** -10)


def test_codec_bitexact_vs_reference(ref_plain):
    x = np.concatenate([rng.normal(0, 50, 50000), rng.normal(0, 1e-3, 20000),
                        np.array([0.0, -0.0, 448.0, 449.0, 464.0, -1e30, 2.0 ** -10, 1.5 * 2.0 ** -9])])
    x = x.astype(np.float32)
    lib = ol.oracle()
    for v in x[:5000]:
        assert lib.oracle_code8(float(v)) == ref_plain.ref_cache_code8(float(v))
        a, b = lib.oracle_pack8(float(v)), ref_plain.ref_cache_pack8(float(v))
        assert a == b or (math.isnan(a) and math.isnan(b))
    for c in range(256):
        assert lib.oracle_real8(c) == ref_plain.ref_cache_real8(c)
    for scale in (2.686925, 21.165359, 0.0371):
        g1 = ol.grid8(scale)
        g2 = np.empty(256, dtype=np.float32)
        ref_plain.ref_cache_grid_fill(ol.p(g2), scale)
        assert np.array_equal(g1, g2)


def test_int8_codec():
    lib = ol.oracle()
    s = 4.0 / 127.0
    for v in (0.0, 1.0, -1.0, 4.0, -4.0, 10.0, -10.0):
        c = lib.oracle_code_i8(v, s)
        assert np.int8(np.uint8(c)) == np.clip(np.rint(np.float32(v) / np.float32(s)), -127, 127)
    g = ol.grid_i8(s)
    assert g[1] == np.float32(s) and g[255] == -np.float32(s) and g[0x81] == np.float32(-127) * np.float32(s)


# ---- softmax ------------------------------------------------------------------

def test_exp_near_against_libm():
    xs = np.linspace(-87.0, 0.0, 20001).astype(np.float32)
    got = np.array([ol.oracle().oracle_exp_near(float(x)) for x in xs], dtype=np.float64)
    want = np.exp(xs.astype(np.float64))
    assert np.max(np.abs(got - want) / want) < 4e-7


def test_exp_near_and_soft_max_bitexact_vs_reference(ref_plain):
    xs = rng.uniform(-90, 0, 5000).astype(np.float32)
    for x in xs:
        assert ol.oracle().oracle_exp_near(float(x)) == ref_plain.ref_exp_near(float(x))
    for n in (1, 3, 4, 7, 64, 513, 4096):
        v = (rng.normal(size=n) * 5).astype(np.float32)
        a, b = v.copy(), v.copy()
        ol.oracle().oracle_soft_max(ol.p(a), n)
        ref_plain.ref_soft_max(ol.p(b), n)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        e = np.exp(v.astype(np.float64) - v.max())
        assert np.max(np.abs(a - e / e.sum())) < 1e-6


# ---- attention ----------------------------------------------------------------

def make_cache(span_rows, kv_width, fmt, scale, seed):
    r = np.random.default_rng(seed)
    k = np.clip(r.normal(size=(span_rows, kv_width)), -4, 4).astype(np.float32)
    v = np.clip(r.normal(size=(span_rows, kv_width)), -4, 4).astype(np.float32)
    return ol.encode(k, scale, fmt), ol.encode(v, scale, fmt)


def brute_attention(kb, vb, kgrid, vgrid, q, cache_span, kv_width, kv_index, head_size,
                    start, span, score_scale):
    slots = [(start + t) % cache_span for t in range(span)]
    off = kv_index * head_size
    K = kgrid[kb[slots, off:off + head_size]].astype(np.float64)
    V = vgrid[vb[slots, off:off + head_size]].astype(np.float64)
    s = (q.astype(np.float64) @ K.T) * score_scale
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=1, keepdims=True)
    return p @ V


@pytest.mark.parametrize("fmt,scale,score_scale", [(0, 4.0 / 448.0, 1.0), (1, 4.0 / 127.0, 1.0 / 16.0)])
@pytest.mark.parametrize("cache_span,start,span", [(64, 0, 1), (64, 0, 37), (512, 300, 512), (600, 0, 600)])
def test_attend_against_brute_force(fmt, scale, score_scale, cache_span, start, span):
    head, group = 256, 8
    kb, vb = make_cache(cache_span, head, fmt, scale, 7)
    grid = ol.grid8(scale) if fmt == 0 else ol.grid_i8(scale)
    q = rng.normal(size=(group, head)).astype(np.float32)
    got = ol.oracle_attend(kb, vb, grid, grid, cache_span, head, 0, q, 0, group, head, start, span,
                           score_scale)
    want = brute_attention(kb, vb, grid, grid, q, cache_span, head, 0, head, start, span, score_scale)
    assert np.max(np.abs(got - want)) < 1e-5


@pytest.mark.parametrize("cache_span,start,span,threads", [(64, 0, 37, 1), (512, 300, 512, 3),
                                                           (700, 0, 700, 4), (256, 10, 129, 2)])
def test_attend_bitexact_vs_reference(ref_plain, cache_span, start, span, threads):
    head, group = 256, 8
    scale = 4.0 / 448.0
    kb, vb = make_cache(cache_span, head, 0, scale, 11)
    grid = ol.grid8(scale)
    q = rng.normal(size=(group, head)).astype(np.float32)
    got = ol.oracle_attend(kb, vb, grid, grid, cache_span, head, 0, q, 0, group, head, start, span)
    desk = ref_plain.ref_desk_open(threads, 64, 2048)
    want = np.zeros((group, head), dtype=np.float32)
    try:
        ref_plain.ref_attend(desk, ol.p(kb), ol.p(vb), ol.p(grid), ol.p(grid), cache_span, head, 0,
                             ol.p(q), 0, group, head, start, span, ol.p(want))
    finally:
        ref_plain.ref_desk_close(desk)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ---- the other table entries ----------------------------------------------------

def test_norm_gelu_rope_definitions():
    x = rng.normal(size=1536).astype(np.float32)
    g = rng.normal(size=1536).astype(np.float32)
    out = np.empty_like(x)
    ol.oracle().oracle_norm_rms(ol.p(x), ol.p(g), x.size, 1e-6, ol.p(out))
    want = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * g
    assert np.max(np.abs(out - want)) < 1e-5
    gate = (rng.normal(size=4096) * 3).astype(np.float32)
    rise = rng.normal(size=4096).astype(np.float32)
    got = gate.copy()
    ol.oracle().oracle_gelu_gate(ol.p(got), ol.p(rise), gate.size)
    xd = gate.astype(np.float64)
    gelu = 0.5 * xd * (1 + np.tanh(math.sqrt(2 / math.pi) * (xd + 0.044715 * xd ** 3)))
    assert np.max(np.abs(got - gelu * rise)) < 1e-5
    v = rng.normal(size=256).astype(np.float32)
    ang = rng.uniform(0, 6.28, 128)
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    got = v.copy()
    ol.oracle().oracle_rope_turn(ol.p(got), 256, ol.p(c), ol.p(s))
    lo, hi = v[:128].astype(np.float64), v[128:].astype(np.float64)
    want = np.concatenate([lo * c - hi * s, hi * c + lo * s])
    assert np.max(np.abs(got - want)) < 1e-5
