"""GPU parity of the packed int4 projection: decode GEMV, small-lane verify
GEMV and batched prefill GEMM, against the oracle on the same seeded inputs.

Bars:
  * GEMV (fp32 in/out): every output within relative error 1e-3 of the oracle,
    relative to max(|y_ref|, rms(y_ref)) so that outputs near zero are judged
    against the scale of the row set rather than against themselves.
  * GEMM (bf16 in/out): bf16 output rounding alone is up to 2^-9 relative, so
    |C - y_ref| <= 2^-8 |y_ref| + 2e-3 rms(y_ref), y_ref the oracle (or the
    float64 closed form at the largest sizes) on the bf16-rounded activations.
"""
import ctypes
import math

import numpy as np
import pytest

import oracle_lib as ol
from igllm_amd.backend import make_plane, synth_projection

pytestmark = pytest.mark.gpu


def rel_err(got, want):
    want = want.astype(np.float64)
    floor = np.sqrt(np.mean(want ** 2))
    return float(np.max(np.abs(got.astype(np.float64) - want) / np.maximum(np.abs(want), floor)))


def run_gemv_dev(backend, cp, act, lanes, path="gemv"):
    K, N = cp.K, cp.N
    dev_act = backend.upload(act)
    dev_out = backend.alloc(lanes * N * 4)
    fn = backend.gemv_dev if path == "gemv" else backend.mat_mat_dev
    fn(cp, dev_act, K, lanes, dev_out, N)
    backend.sync()
    out = dev_out.get(np.float32, lanes * N).reshape(lanes, N)
    dev_act.free()
    dev_out.free()
    return out


def print_case(**kw):
    print("case", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def test_decode_gemv_config0(backend):
    """W [8192, 2048] int4 g32, x [2048] ~ N(0,1), seed 0 (the decode projection)."""
    print_case(test="config0", N=8192, K=2048, lanes=1, seed=0)
    codes, gains, act = synth_projection(8192, 2048, 1, seed=0)
    cp = backend.attach(make_plane(codes, gains, 2048))
    got = run_gemv_dev(backend, cp, act, 1)
    want = ol.oracle_mat_mat(codes, gains, act, 2048, threads=8)
    err = rel_err(got, want)
    print("rel_err", err)
    assert err <= 1e-3
    # the table entry (host pointers) is the same launch behind staging
    host = backend.mat_vec(cp, act[0])
    assert np.array_equal(host, got[0])
    backend.detach(cp)


@pytest.mark.parametrize("N,K", [(8192, 2048), (2048, 8192)])
@pytest.mark.parametrize("lanes", [1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 16])
def test_small_lane_sweep(backend, N, K, lanes):
    print_case(test="sweep", N=N, K=K, lanes=lanes)
    codes, gains, act = synth_projection(N, K, lanes, seed=lanes)
    cp = backend.attach(make_plane(codes, gains, K))
    got = run_gemv_dev(backend, cp, act, lanes)
    want = ol.oracle_mat_mat(codes, gains, act, K, threads=8)
    err = rel_err(got, want)
    print("rel_err", err)
    assert err <= 1e-3
    backend.detach(cp)


@pytest.mark.parametrize("N,K,lanes,group", [
    (70, 128, 1, 32), (130, 96, 3, 32), (1, 32, 1, 32), (257, 1536, 2, 32), (64, 12288, 1, 32),
    (33, 12288, 8, 32), (100, 2048, 8, 64), (100, 4096, 4, 128), (512, 256, 16, 32),
    (300, 6144, 12, 32), (40, 8192, 5, 32), (1536, 12288, 1, 32), (1000, 6144, 1, 32),
    (1536, 4096, 1, 32), (999, 2048, 1, 32), (1536, 12288, 2, 32), (37, 9216, 2, 32),
    (1536, 4096, 2, 32), (999, 2048, 2, 32), (1537, 256, 2, 32), (1000, 6144, 2, 32),
])
def test_gemv_edges(backend, N, K, lanes, group):
    """Ragged rows, narrow and odd unit counts, K-chunked launches, wider groups,
    lane counts past one launch; one or two lanes on wide rows in six-row
    tiles (the 1536 x 12288 down projection of a decode step or a two-lane
    block, and a ragged last tile); one
    or two lanes on small planes, one wave a tile, two units a lane past 64;
    two lanes past K 8192 (twelve staged groups a thread, two units a
    lane)."""
    print_case(test="gemv_edges", N=N, K=K, lanes=lanes, group=group)
    codes, gains, act = synth_projection(N, K, lanes, seed=N + K, group_size=group)
    cp = backend.attach(make_plane(codes, gains, K, group_size=group))
    got = run_gemv_dev(backend, cp, act, lanes)
    want = ol.oracle_mat_mat(codes, gains, act, K, group_size=group, threads=8)
    assert rel_err(got, want) <= 1e-3
    host = backend.mat_mat(cp, act)
    assert rel_err(host, want) <= 1e-3
    backend.detach(cp)


def test_gemv_chunked_repeat(backend):
    """K-chunked matrix-core launches (partials summed in chunk order by a
    second launch): launches of different lane counts and planes (full and ragged row blocks)
    interleaved, each repeated, then all of them recorded once and replayed
    three times: every repeat and every replay is bit-identical to the first
    and within the bar of the oracle."""
    cases = [(2048, 8192, 4), (2048, 8192, 8), (40, 8192, 5), (2000, 8192, 3), (33, 12288, 8)]
    planes, firsts = [], []
    for N, K, lanes in cases:
        print_case(test="chunked_repeat", N=N, K=K, lanes=lanes)
        codes, gains, act = synth_projection(N, K, lanes, seed=N + lanes)
        cp = backend.attach(make_plane(codes, gains, K))
        planes.append((cp, act))
        got = run_gemv_dev(backend, cp, act, lanes)
        want = ol.oracle_mat_mat(codes, gains, act, K, threads=8)
        assert rel_err(got, want) <= 1e-3
        firsts.append(got)
    for turn in range(3):
        for (cp, act), first in zip(planes, firsts):
            got = run_gemv_dev(backend, cp, act, act.shape[0])
            assert np.array_equal(got.view(np.uint32), first.view(np.uint32)), f"repeat {turn}"
    bufs = []
    for cp, act in planes:
        bufs.append((backend.upload(act), backend.alloc(act.shape[0] * cp.N * 4)))
    backend.record_begin()
    for (cp, act), (a, o) in zip(planes, bufs):
        backend.gemv_dev(cp, a, cp.K, act.shape[0], o, cp.N)
    handle = backend.record_end()
    try:
        for turn in range(3):
            for _, o in bufs:
                o.put(np.zeros(o.nbytes // 4, np.float32))
            backend.replay_run(handle)
            backend.sync()
            for (cp, act), (a, o), first in zip(planes, bufs, firsts):
                got = o.get(np.float32, act.shape[0] * cp.N).reshape(act.shape[0], cp.N)
                assert np.array_equal(got.view(np.uint32), first.view(np.uint32)), f"replay {turn}"
    finally:
        backend.replay_free(handle)
    for a, o in bufs:
        a.free()
        o.free()
    for cp, _ in planes:
        backend.detach(cp)


@pytest.mark.parametrize("lanes", [1, 3])
def test_gemv_unaligned_activations(backend, lanes):
    """An activation stride that is not a multiple of four floats takes the
    scalar staging path (one lane: the float register form)."""
    N, K = 96, 256
    codes, gains, act = synth_projection(N, K, lanes, seed=9)
    padded = np.zeros((lanes, K + 1), dtype=np.float32)
    padded[:, :K] = act
    cp = backend.attach(make_plane(codes, gains, K))
    dev_act = backend.upload(padded)
    dev_out = backend.alloc(lanes * N * 4)
    backend.gemv_dev(cp, dev_act, K + 1, lanes, dev_out, N)
    backend.sync()
    got = dev_out.get(np.float32, lanes * N).reshape(lanes, N)
    want = ol.oracle_mat_mat(codes, gains, act, K)
    assert rel_err(got, want) <= 1e-3
    backend.detach(cp)


@pytest.mark.parametrize("case", ["zeros", "tiny", "subnormal", "huge", "mixed"])
@pytest.mark.parametrize("lanes", [1, 2])
def test_gemv_activation_range(backend, lanes, case):
    """The one- and two-lane products quantize each 32-element unit of x to 24
    bits against the unit's largest |x|, scaling by exact powers of two: a
    unit of zeros, x at 1e-30, subnormal x, x at 1e30, and units mixing 1e-6
    with 1e3, against the float64 closed form."""
    print_case(test="activation_range", lanes=lanes, case=case)
    N, K = 300, 2048
    codes, gains, act = synth_projection(N, K, lanes, seed=21)
    act = act.astype(np.float64)
    if case == "zeros":
        act[:, 32:96] = 0.0
        act[:, 200] = 0.0
    elif case == "tiny":
        act *= 1e-30
    elif case == "subnormal":
        act *= 1e-40
    elif case == "huge":
        act *= 1e30
    else:
        act[:, 0::2] *= 1e-6
        act[:, 1::64] *= 1e3
    act = act.astype(np.float32)
    cp = backend.attach(make_plane(codes, gains, K))
    got = run_gemv_dev(backend, cp, act, lanes)
    vals = ((codes[:, :, None] >> np.array([0, 4], dtype=np.uint8)) & 15).reshape(N, K).astype(np.float64) - 8
    scale = np.repeat(gains.astype(np.float64), 32, axis=1)
    want = act.astype(np.float64) @ (vals * scale).T
    err = rel_err(got, want)
    print("rel_err", err)
    assert np.all(np.isfinite(got))
    # subnormal x: the closed form's own inputs carry only ~17 bits
    assert err <= (1e-3 if case == "subnormal" else 1e-5)
    backend.detach(cp)


def test_unsupported_plane_is_refused(backend):
    from igllm_amd.backend import BackendError

    codes, gains, act = synth_projection(16, 48, 1, seed=3, group_size=16)
    with pytest.raises(BackendError):
        backend.attach(make_plane(codes, gains, 48, group_size=16))


def bf16_round(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_to_f32(raw):
    return (raw.astype(np.uint32) << 16).view(np.float32)


def closed_form64(codes, gains, act64, K, group=32):
    nib = np.stack([codes & 15, codes >> 4], axis=-1).reshape(codes.shape[0], -1)[:, :K]
    w = (nib.astype(np.float64) - 8.0) * np.repeat(gains.astype(np.float64), group, axis=1)[:, :K]
    return act64 @ w.T


def closed_form64_groups(codes, gains, act64, K, group):
    nib = np.stack([codes & 15, codes >> 4], axis=-1).reshape(codes.shape[0], -1)[:, :K]
    w = (nib.astype(np.float64) - 8.0) * np.repeat(gains.astype(np.float64), group, axis=1)[:, :K]
    return act64 @ w.T


def gemm_form(backend, M, N, K, terms):
    """The tiling form the GEMM launcher picks (0: 256 x 256 tiles .. 4: 16 x 64
    tiles with an eight-way K split inside the workgroup; 5: 64 x 64 tiles in
    four-wave workgroups, two a CU)."""
    fn = backend.lib.igl_gemm_form
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int] * 4
    return fn(M, N, K, terms)


@pytest.mark.parametrize("N,K", [(8192, 2048), (2048, 8192)])
@pytest.mark.parametrize("M", [64, 100, 192, 256, 1024, 2048])
def test_prefill_gemm(backend, N, K, M):
    """BASELINE's prefill lanes (64 .. 2048) and two ragged counts, bf16 in and
    out.  The products are exact and summed in fp32, so the only loss is the
    output's bf16 rounding (unit roundoff 2^-8): |C - y| <= 2^-8 |y| +
    1e-4 rms(y), y the float64 closed form on the same bf16 activations; and C
    is y rounded to bf16 but where y lies within fp32 error of a rounding tie
    (all but a few in ten thousand)."""
    print_case(test="prefill", N=N, K=K, M=M, form=gemm_form(backend, M, N, K, 1))
    codes, gains, act = synth_projection(N, K, M, seed=M)
    a16 = bf16_round(act).reshape(M, K)
    cp = backend.attach(make_plane(codes, gains, K))
    dev_a = backend.upload(a16)
    dev_c = backend.alloc(M * N * 2)
    backend.gemm_bf16_dev(cp, dev_a, K, M, dev_c, N)
    backend.sync()
    got = bf16_to_f32(dev_c.get(np.uint16, M * N)).reshape(M, N).astype(np.float64)
    a32 = bf16_to_f32(a16)
    want = closed_form64(codes, gains, a32.astype(np.float64), K)
    rms = math.sqrt(float(np.mean(want ** 2)))
    excess = np.abs(got - want) - (2.0 ** -8 * np.abs(want) + 1e-4 * rms)
    same = float(np.mean(got == bf16_to_f32(bf16_round(want.astype(np.float32)))))
    print("max_excess", float(excess.max()), "rms", rms, "bf16(y) share", same)
    assert float(excess.max()) <= 0.0
    assert same >= 0.999
    dev_a.free()
    dev_c.free()
    backend.detach(cp)


@pytest.mark.parametrize("N,K", [(8192, 2048), (2048, 8192)])
@pytest.mark.parametrize("M", [64, 256, 2048])
def test_mat_mat_gemm_fp32(backend, N, K, M):
    """fp32 activations with >= 64 lanes take the MFMA GEMM through mat_mat_dev
    with two binary16 terms a value: within 1e-3 of the oracle (the reference's
    fp32 float path) and of the float64 closed form; in practice ~1e-6."""
    print_case(test="mat_mat_fp32", N=N, K=K, M=M, form=gemm_form(backend, M, N, K, 2))
    codes, gains, act = synth_projection(N, K, M, seed=M + 7)
    cp = backend.attach(make_plane(codes, gains, K))
    got = run_gemv_dev(backend, cp, act, M, path="mat_mat")
    exact = closed_form64(codes, gains, act.astype(np.float64), K)
    err = rel_err(got, exact)
    print("rel_err vs float64", err)
    assert err <= 1e-3
    if M <= 256:
        want = ol.oracle_mat_mat(codes, gains, act, K, threads=8)
        err = rel_err(got, want)
        print("rel_err vs oracle", err)
        assert err <= 1e-3
    backend.detach(cp)


# (M, N, K): cases that reach each tiling form, plus ragged tiles in M and N,
# K an odd number of 32-code groups (padded to a whole step with zeros), and K
# a multiple of 128 but not 256 (the two-a-CU form's K split only).
FORM_CASES = [(1024, 8192, 256), (2048, 2048, 512), (256, 4096, 1024), (64, 8192, 1024),
              (64, 2048, 2048), (100, 1000, 1536), (333, 777, 192), (70, 300, 1056), (128, 256, 96),
              (300, 5000, 384), (64, 1024, 640)]


@pytest.mark.parametrize("terms", [1, 2])
def test_gemm_forms(backend, terms):
    """Every tiling form (the intra-workgroup K splits included) and ragged
    tiles, one- and two-term activations, against the oracle at 1e-3 (fp32 x:
    two terms; bf16-valued x: one term is exact)."""
    seen = set()
    for M, N, K in FORM_CASES:
        form = gemm_form(backend, M, N, K, terms)
        seen.add(form)
        print_case(test="forms", M=M, N=N, K=K, terms=terms, form=form)
        codes, gains, act = synth_projection(N, K, M, seed=M + N + K)
        cp = backend.attach(make_plane(codes, gains, K))
        if terms == 1:
            a16 = bf16_round(act).reshape(M, K)
            dev_a = backend.upload(a16)
            dev_c = backend.alloc(M * N * 2)
            backend.gemm_bf16_dev(cp, dev_a, K, M, dev_c, N)
            backend.sync()
            got = bf16_to_f32(dev_c.get(np.uint16, M * N)).reshape(M, N).astype(np.float64)
            want = closed_form64(codes, gains, bf16_to_f32(a16).astype(np.float64), K)
            rms = math.sqrt(float(np.mean(want ** 2)))
            assert float((np.abs(got - want) - (2.0 ** -8 * np.abs(want) + 1e-4 * rms)).max()) <= 0.0
            assert float(np.mean(got == bf16_to_f32(bf16_round(want.astype(np.float32))))) >= 0.999
            dev_a.free()
            dev_c.free()
        else:
            got = run_gemv_dev(backend, cp, act, M, path="mat_mat")
            want = ol.oracle_mat_mat(codes, gains, act, K, threads=8)
            err = rel_err(got, want)
            print("rel_err", err)
            assert err <= 1e-3
        backend.detach(cp)
    assert seen == {0, 1, 2, 3, 4, 5}


@pytest.mark.parametrize("case", ["zeros", "tiny", "huge", "rows", "mixed"])
def test_gemm_activation_range(backend, case):
    """Each activation row is scaled by its own power of two before it is split
    into binary16 terms: rows of zeros, x at 1e-30 and at 1e30, rows spanning
    1e-20 .. 1e20, and rows mixing 1e-6 with 1e3, against the float64 closed
    form (relative to each row's own scale)."""
    print_case(test="gemm_activation_range", case=case)
    M, N, K = 96, 512, 1024
    codes, gains, act = synth_projection(N, K, M, seed=31)
    act = act.astype(np.float64)
    if case == "zeros":
        act[3] = 0.0
        act[:, 64:160] = 0.0
    elif case == "tiny":
        act *= 1e-30
    elif case == "huge":
        act *= 1e30
    elif case == "rows":
        act *= 10.0 ** np.linspace(-20, 20, M)[:, None]
    else:
        act[:, 0::2] *= 1e-6
        act[:, 1::64] *= 1e3
    act = act.astype(np.float32)
    cp = backend.attach(make_plane(codes, gains, K))
    got = run_gemv_dev(backend, cp, act, M, path="mat_mat").astype(np.float64)
    want = closed_form64(codes, gains, act.astype(np.float64), K)
    assert np.all(np.isfinite(got))
    floor = np.sqrt(np.mean(want ** 2, axis=1, keepdims=True))
    floor = np.where(floor > 0, floor, 1.0)
    err = float(np.max(np.abs(got - want) / np.maximum(np.abs(want), floor)))
    print("rel_err", err)
    assert err <= 1e-5
    backend.detach(cp)


@pytest.mark.parametrize("group", [64, 128, 2048])
def test_gemm_group_sizes(backend, group):
    """Groups of 64 and 128 codes (one gain over two or four units) and one
    gain a row (the gain taken once at the store), fp32 activations."""
    M, N, K = 128, 1024, 2048
    print_case(test="gemm_groups", group=group)
    codes, gains, act = synth_projection(N, K, M, seed=group, group_size=group)
    cp = backend.attach(make_plane(codes, gains, K, group_size=group))
    got = run_gemv_dev(backend, cp, act, M, path="mat_mat")
    want = ol.oracle_mat_mat(codes, gains, act, K, group_size=group, threads=8)
    err = rel_err(got, want)
    print("rel_err", err)
    assert err <= 1e-3
    assert rel_err(got, closed_form64_groups(codes, gains, act.astype(np.float64), K, group)) <= 1e-5
    backend.detach(cp)


def test_gemm_repeat_bitwise(backend):
    """Launches of different forms interleaved and repeated are bit-identical
    to their first run (the K split's partial tiles are added in a fixed
    order)."""
    cases = [(64, 2048, 2048), (256, 4096, 1024), (300, 1000, 1536)]
    runs = []
    for M, N, K in cases:
        codes, gains, act = synth_projection(N, K, M, seed=M * 3 + 1)
        cp = backend.attach(make_plane(codes, gains, K))
        runs.append((cp, act, run_gemv_dev(backend, cp, act, M, path="mat_mat")))
    for turn in range(3):
        for cp, act, first in runs:
            got = run_gemv_dev(backend, cp, act, act.shape[0], path="mat_mat")
            assert np.array_equal(got.view(np.uint32), first.view(np.uint32)), f"repeat {turn}"
    for cp, _, _ in runs:
        backend.detach(cp)


def gemm_slices(backend, M, N, K, terms):
    """How many K slices the GEMM launcher splits K into across workgroups
    (1: none)."""
    fn = backend.lib.igl_gemm_slices
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int] * 4
    return fn(M, N, K, terms)


# (M, N, K, group, zero points): long rows at a few hundred lanes or less,
# whose K the launcher splits across workgroups into 2, 4 and 8 slices, with
# ragged tiles in M and N, groups of 64 codes, one gain a row, and zero points.
SLICE_CASES = [(64, 2048, 8192, 32, False), (100, 1000, 4096, 32, False), (192, 2048, 8192, 32, False),
               (70, 4000, 4096, 64, False), (96, 512, 16384, 16384, False), (128, 1536, 6144, 32, True)]


@pytest.mark.parametrize("terms", [1, 2])
def test_gemm_k_slices(backend, terms):
    """K split across workgroups: each slice's fp32 product (row scale
    applied, exactly) written apart and the slices added in slice order by a
    second launch.  bf16 activations (one term) against the float64 closed
    form at the bf16 output's rounding, fp32 ones (two terms) against the
    oracle at 1e-3; each case repeated bit-identical; 2, 4 and 8 slices all
    reached."""
    seen = set()
    for M, N, K, group, zero in SLICE_CASES:
        slices = gemm_slices(backend, M, N, K, terms)
        seen.add(slices)
        print_case(test="k_slices", M=M, N=N, K=K, group=group, zero=zero, terms=terms, slices=slices)
        codes, gains, act = synth_projection(N, K, M, seed=M + K + group, group_size=group)
        zeros = None
        if zero:
            zeros = np.random.default_rng(M + N).integers(-8, 8, size=gains.shape).astype(np.int8)
        cp = backend.attach(make_plane(codes, gains, K, group_size=group, zeros=zeros))
        if terms == 1:
            a16 = bf16_round(act).reshape(M, K)
            dev_a = backend.upload(a16)
            dev_c = backend.alloc(M * N * 2)
            runs = []
            for _ in range(2):
                backend.gemm_bf16_dev(cp, dev_a, K, M, dev_c, N)
                backend.sync()
                runs.append(dev_c.get(np.uint16, M * N))
            assert np.array_equal(runs[0], runs[1])
            got = bf16_to_f32(runs[0]).reshape(M, N).astype(np.float64)
            nib = np.stack([codes & 15, codes >> 4], axis=-1).reshape(N, -1)[:, :K].astype(np.float64)
            sub = 8.0 if zeros is None else 8.0 + np.repeat(zeros.astype(np.float64), group, axis=1)[:, :K]
            w = (nib - sub) * np.repeat(gains.astype(np.float64), group, axis=1)[:, :K]
            want = bf16_to_f32(a16).astype(np.float64) @ w.T
            rms = math.sqrt(float(np.mean(want ** 2)))
            excess = np.abs(got - want) - (2.0 ** -8 * np.abs(want) + 1e-4 * rms)
            same = float(np.mean(got == bf16_to_f32(bf16_round(want.astype(np.float32)))))
            print("max_excess", float(excess.max()), "bf16(y) share", same)
            assert float(excess.max()) <= 0.0
            assert same >= 0.999
            dev_a.free()
            dev_c.free()
        else:
            got = run_gemv_dev(backend, cp, act, M, path="mat_mat")
            again = run_gemv_dev(backend, cp, act, M, path="mat_mat")
            assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
            kw = {} if zeros is None else {"zeros": zeros}
            want = ol.oracle_mat_mat(codes, gains, act, K, group, threads=8, **kw)
            err = rel_err(got, want)
            print("rel_err", err)
            assert err <= 1e-3
        backend.detach(cp)
    assert {2, 4, 8} <= seen


def test_mat_mat_many_lanes_takes_gemm(backend):
    """fp32 activations with >= 64 lanes go to the MFMA GEMM through mat_mat_dev."""
    N, K, M = 384, 1024, 96
    codes, gains, act = synth_projection(N, K, M, seed=5)
    cp = backend.attach(make_plane(codes, gains, K))
    got = run_gemv_dev(backend, cp, act, M, path="mat_mat")
    want = ol.oracle_mat_mat(codes, gains, act, K, threads=8)
    assert rel_err(got, want) <= 1e-3
    backend.detach(cp)
