"""GPU parity of the backend table's elementwise entries (norm_rms, soft_max,
gelu_gate, rope_turn) through the table itself, against the oracle.
Bar: 1e-5 relative to the vector's scale (1e-6 for softmax probabilities)."""
import ctypes

import numpy as np
import pytest

import launch_structs
import oracle_lib as ol

pytestmark = pytest.mark.gpu
r = np.random.default_rng(99)


def test_norm_rms(backend):
    for n, with_gain in ((1536, True), (256, False), (12288, True)):
        x = (r.normal(size=n) * 7).astype(np.float32)
        g = r.normal(size=n).astype(np.float32) if with_gain else None
        got = backend.norm_rms(x, g, 1e-6)
        want = np.empty_like(x)
        ol.oracle().oracle_norm_rms(ol.p(x), None if g is None else ol.p(g), n, 1e-6, ol.p(want))
        assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))


def test_soft_max(backend):
    for n in (1, 5, 512, 16384):
        v = (r.normal(size=n) * 4).astype(np.float32)
        got = backend.soft_max(v)
        want = v.copy()
        ol.oracle().oracle_soft_max(ol.p(want), n)
        assert np.max(np.abs(got - want)) <= 1e-6


def test_gelu_gate(backend):
    n = 12288
    gate = (r.normal(size=n) * 4).astype(np.float32)
    gate[:4] = [-40.0, 40.0, 0.0, -3.0]
    rise = r.normal(size=n).astype(np.float32)
    got = backend.gelu_gate(gate, rise)
    want = gate.copy()
    ol.oracle().oracle_gelu_gate(ol.p(want), ol.p(rise), n)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))


def test_rope_turn(backend):
    for head in (256, 512):
        v = r.normal(size=head).astype(np.float32)
        ang = r.uniform(0, 6.3, head // 2)
        c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
        got = backend.rope_turn(v, c, s)
        want = v.copy()
        ol.oracle().oracle_rope_turn(ol.p(want), head, ol.p(c), ol.p(s))
        assert np.max(np.abs(got - want)) <= 1e-6


@pytest.mark.parametrize("step", [0.0625, 0.1, 3.7, 0.0])
def test_quant_step_dev(backend, step):
    """igl_quant_step_dev against the pinned float32 closed form, bit for bit:
    three lanes at a stride, out of place and in place."""
    from test_oracle import quant_step_closed, quant_step_inputs

    x = quant_step_inputs()
    n, lanes, stride = x.size, 3, x.size + 5
    host = np.zeros((lanes, stride), dtype=np.float32)
    for l in range(lanes):
        host[l, :n] = np.roll(x, 17 * l)
    src = backend.upload(host)
    dst = backend.alloc(host.nbytes)
    backend.quant_step_dev(src, stride, dst, stride, n, lanes, step)
    backend.quant_step_dev(src, stride, src, stride, n, lanes, step)
    backend.sync()
    out = dst.get(np.float32, lanes * stride).reshape(lanes, stride)
    inplace = src.get(np.float32, lanes * stride).reshape(lanes, stride)
    for l in range(lanes):
        want = quant_step_closed(host[l, :n], step)
        assert np.array_equal(out[l, :n].view(np.uint32), want.view(np.uint32))
        assert np.array_equal(inplace[l, :n].view(np.uint32), want.view(np.uint32))
    src.free()
    dst.free()


@pytest.mark.parametrize("lanes", [1, 3, 64])
def test_plane_lift_dev(backend, lanes):
    """plane_lift_many on device (app_core.c:7814-7843): the lanes on the
    enter_gain grid, the product, the outputs on the leave_gain grid.  Below 64
    lanes the product is the fused one on the activation grid (exact integer
    sums), from 64 the steps one by one (grid, MFMA GEMM, grid).  Checked: the
    product against the oracle on the gridded activations, and the leave grid
    to the bit against the closed form applied to that product."""
    from igllm_amd.backend import make_plane, synth_projection
    from test_oracle import quant_step_closed

    N, K = 640, 2048
    codes, gains, act = synth_projection(N, K, lanes, seed=31)
    act = (act * 3).astype(np.float32)
    cp = backend.attach(make_plane(codes, gains, K))
    cp.plane.enter_gain = 0.05
    entered = np.stack([quant_step_closed(a, 0.05) for a in act])
    dev_act = backend.upload(act)
    out = backend.alloc(lanes * N * 4)
    cp.plane.leave_gain = 0.0
    backend.plane_lift_dev(cp, dev_act, K, lanes, out, N)
    backend.sync()
    product = out.get(np.float32, lanes * N).reshape(lanes, N)
    cp.plane.leave_gain = 0.01
    backend.plane_lift_dev(cp, dev_act, K, lanes, out, N)
    backend.sync()
    got = out.get(np.float32, lanes * N).reshape(lanes, N)
    want = np.stack([quant_step_closed(y, 0.01) for y in product])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    ref = ol.oracle_mat_mat(codes, gains, entered, K, threads=8)
    floor = np.sqrt(np.mean(ref.astype(np.float64) ** 2))
    # from 64 lanes the MFMA GEMM on hi + lo binary16 terms: as close as the GEMV
    assert np.max(np.abs(product - ref) / np.maximum(np.abs(ref), floor)) <= 1e-5
    for b in (dev_act, out):
        b.free()
    backend.detach(cp)


LEVEL_KINDS = [
    (2048, 1536, 4, 0, 1), (2048, 1536, 4, 0, 3), (6144, 1536, 2, 0, 1), (1536, 6144, 2, 0, 2),
    (256, 1536, 8, 128, 1), (1536, 256, 8, 128, 4), (1536, 2048, 4, 0, 5), (300, 16384, 4, 0, 1),
    (100, 8192, 8, 128, 2), (70, 96, 2, 1, 1),
    # one lane on wide rows: six-row tiles, four waves a tile (the export-kinds
    # down projections, a ragged last tile, two slots a lane of 8-bit codes)
    (1536, 12288, 2, 0, 1), (1000, 6144, 4, 0, 1), (700, 6144, 8, 128, 1),
    # one lane on small planes: one wave a two-row tile, no K split (two slots
    # a lane for 8-bit codes at K 2048)
    (1536, 2048, 4, 0, 1), (1000, 2048, 8, 128, 1), (257, 1536, 8, 128, 1),
    # from 64 lanes: the int8 MFMA GEMM (levels against codes as int8 operands)
    (2048, 1536, 4, 0, 64), (6144, 1536, 2, 0, 300), (256, 1536, 8, 128, 70), (1536, 256, 8, 128, 256),
    (1536, 6144, 2, 0, 100), (512, 2048, 4, 3, 64),
    # K off that kernel's step (128; 64 for 8-bit codes): the binary16 MFMA on
    # levels and widened codes
    (512, 1056, 4, 0, 64), (384, 1056, 8, 128, 64), (640, 1056, 2, 0, 96),
]


@pytest.mark.parametrize("N,K,bits,flip,lanes", LEVEL_KINDS)
def test_plane_lift_level_bitexact(backend, N, K, bits, flip, lanes):
    """Calibrated per-channel planes (the export's kinds, one gain a row): the
    product on the activation grid (the fused GEMV below 64 lanes; from 64 the
    int8 MFMA GEMM, or the binary16 MFMA on integer-valued operands where K does
    not fit it) equals the oracle's level path
    (the reference's VNNI-tier kern_row_code_level, pinned to the bit against
    that build) to the bit, and so does the leave grid after it."""
    from igllm_amd.backend import make_plane
    from test_oracle import quant_step_closed

    print("case level N=%d K=%d bits=%d flip=%d lanes=%d" % (N, K, bits, flip, lanes), flush=True)
    r = np.random.default_rng(N + K + bits)
    stride = ((K * bits + 7) // 8 + 15) // 16 * 16
    codes = r.integers(0, 256, size=(N, stride), dtype=np.uint8)
    gains = np.abs(r.normal(0, 0.02, size=(N, 1))).astype(np.float32)
    act = r.normal(size=(lanes, K)).astype(np.float32)
    step, leave = float(np.float32(2.5 / 127)), float(np.float32(0.02))
    cp = backend.attach(make_plane(codes, gains, K, group_size=K, bits=bits, code_flip=flip))
    cp.plane.enter_gain = step
    kw = dict(bits=bits, code_bias=1 << (bits - 1), code_flip=flip)
    want = ol.oracle_mat_mat_level(codes, gains, act, K, K, step, **kw)
    dev_act = backend.upload(act)
    out = backend.alloc(lanes * N * 4)
    backend.plane_lift_dev(cp, dev_act, K, lanes, out, N)
    backend.sync()
    got = out.get(np.float32, lanes * N).reshape(lanes, N)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    cp.plane.leave_gain = leave
    backend.plane_lift_dev(cp, dev_act, K, lanes, out, N)
    backend.sync()
    got = out.get(np.float32, lanes * N).reshape(lanes, N)
    assert np.array_equal(got.view(np.uint32), np.stack([quant_step_closed(y, leave) for y in want]).view(np.uint32))
    dev_act.free()
    out.free()
    backend.detach(cp)


NEAR_TIE_STEPS = [2.5 / 127, 2.0 ** -96, 2.0 ** 90, 2.0 ** -100, 2.0 ** 100]


@pytest.mark.parametrize("step_in", NEAR_TIE_STEPS)
@pytest.mark.parametrize("bits,lanes", [(4, 1), (2, 3), (4, 64)])
def test_plane_lift_level_near_ties(backend, step_in, bits, lanes):
    """Activations at and one ulp either side of every half-integer quotient of
    the clamp range, with steps inside [2^-96, 2^96] (the reciprocal and fma
    correction) and outside it (the kernels divide), and a leave grid scaled to
    the products: the levels, the product and the leave grid equal the
    oracle's level path to the bit (the fused GEMV below 64 lanes, the int8
    MFMA GEMM and its close from 64)."""
    from igllm_amd.backend import make_plane
    from test_oracle import quant_step_closed

    N, K = 512, 1536
    print("case near-ties step=%g bits=%d lanes=%d" % (step_in, bits, lanes), flush=True)
    r = np.random.default_rng(bits * 100 + lanes)
    step = float(np.float32(step_in))
    stride = ((K * bits + 7) // 8 + 15) // 16 * 16
    codes = r.integers(0, 256, size=(N, stride), dtype=np.uint8)
    gains = np.abs(r.normal(0, 0.02, size=(N, 1))).astype(np.float32)
    k = r.integers(-140, 140, size=(lanes, K))
    act = ((k + 0.5) * step).astype(np.float32)
    nudge = r.integers(-1, 2, size=(lanes, K))
    act = np.where(nudge > 0, np.nextafter(act, np.float32(np.inf)), act)
    act = np.where(nudge < 0, np.nextafter(act, np.float32(-np.inf)), act).astype(np.float32)
    act[:, ::7] = (r.normal(size=act[:, ::7].shape) * 60.0 * step).astype(np.float32)
    cp = backend.attach(make_plane(codes, gains, K, group_size=K, bits=bits))
    cp.plane.enter_gain = step
    kw = dict(bits=bits, code_bias=1 << (bits - 1), code_flip=0)
    want = ol.oracle_mat_mat_level(codes, gains, act, K, K, step, **kw)
    dev_act = backend.upload(act)
    out = backend.alloc(lanes * N * 4)
    backend.plane_lift_dev(cp, dev_act, K, lanes, out, N)
    backend.sync()
    got = out.get(np.float32, lanes * N).reshape(lanes, N)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    leave = float(np.float32(np.sqrt(np.mean(want.astype(np.float64) ** 2)) / 40.0))
    cp.plane.leave_gain = leave
    backend.plane_lift_dev(cp, dev_act, K, lanes, out, N)
    backend.sync()
    got = out.get(np.float32, lanes * N).reshape(lanes, N)
    assert np.array_equal(got.view(np.uint32), np.stack([quant_step_closed(y, leave) for y in want]).view(np.uint32))
    dev_act.free()
    out.free()
    backend.detach(cp)


def test_plane_lift_level_nan_lane(backend):
    """A NaN activation puts its lane's outputs at NaN and leaves the others on
    the grid.  (The reference sends the whole 16-lane chunk to the float path
    when one lane is off the grid, so its other lanes would carry float-path
    roundings; here each lane keeps the level path.)"""
    from igllm_amd.backend import make_plane

    N, K = 512, 1536
    r = np.random.default_rng(9)
    codes = r.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    gains = np.abs(r.normal(0, 0.02, size=(N, 1))).astype(np.float32)
    act = r.normal(size=(2, K)).astype(np.float32)
    act[1, 100] = np.nan
    step = float(np.float32(2.5 / 127))
    cp = backend.attach(make_plane(codes, gains, K, group_size=K))
    cp.plane.enter_gain = step
    dev_act = backend.upload(act)
    out = backend.alloc(2 * N * 4)
    backend.plane_lift_dev(cp, dev_act, K, 2, out, N)
    backend.sync()
    got = out.get(np.float32, 2 * N).reshape(2, N)
    assert np.all(np.isnan(got[1])) and np.all(np.isfinite(got[0]))
    want = ol.oracle_mat_mat_level(codes, gains, act[:1], K, K, step)
    assert np.array_equal(got[0].view(np.uint32), want[0].view(np.uint32))
    dev_act.free()
    out.free()
    backend.detach(cp)


_CodeView = launch_structs.CodeView
_Prologue = launch_structs.Prologue


@pytest.mark.parametrize("bits,N,K", [(2, 12288, 1536), (4, 6144, 1536), (2, 1001, 1536), (8, 513, 2048),
                                      (4, 77, 1024)])
def test_level_pair_equals_two_launches(backend, bits, N, K):
    """The calibrated gate and up planes of one lane in one launch
    (igl_launch_gemv_level_pair: the residual update as its prologue, both
    row closes on their own leave grids, then gelu(gate) * up) equals, to the
    bit, the two launches it replaces: the gate plane with the prologue
    (igl_launch_gemv_level_pro, x kept) and the up plane with gelu(gate) * up
    fused in its store (igl_launch_gemv_level_epi); and both leave the same
    updated state."""
    print("case level pair bits=%d N=%d K=%d" % (bits, N, K), flush=True)
    lib = backend.lib
    for name, args in (("igl_launch_gemv_level_pro",
                        [ctypes.c_void_p, ctypes.c_float, ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p,
                         ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                         ctypes.c_void_p]),
                       ("igl_launch_gemv_level_epi",
                        [ctypes.c_void_p, ctypes.c_float, ctypes.c_float, ctypes.c_void_p, ctypes.c_int,
                         ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                         ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]),
                       ("igl_launch_gemv_level_pair",
                        [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                         ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p])):
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = args
    lib.igl_desk_stream.restype = ctypes.c_void_p
    lib.igl_desk_stream.argtypes = [ctypes.c_void_p]
    stream = lib.igl_desk_stream(ctypes.byref(backend.desk))
    r = np.random.default_rng(bits * 1000 + N)
    row_bytes = K * bits // 8
    bufs = []

    def up_load(a):
        b = backend.upload(np.ascontiguousarray(a))
        bufs.append(b)
        return b

    planes = []
    for _ in range(2):
        codes = up_load(r.integers(0, 256, size=(N, row_bytes), dtype=np.uint8))
        gains = up_load(np.abs(r.normal(0, 0.02, size=N)).astype(np.float32))
        planes.append(_CodeView(codes.ptr, row_bytes, gains.ptr, 1, 31, bits, 1 << (bits - 1),
                                128 if bits == 8 else 0))
    state = up_load(r.normal(size=K).astype(np.float32))
    lift = up_load(r.normal(size=K).astype(np.float32))
    lift_gain = up_load(r.normal(1.0, 0.1, size=K).astype(np.float32))
    norm_gain = up_load(r.normal(1.0, 0.1, size=K).astype(np.float32))
    s_two, s_pair = backend.alloc(K * 4), backend.alloc(K * 4)
    scrap, y_two, y_pair = backend.alloc(K * 4), backend.alloc(N * 4), backend.alloc(N * 4)
    bufs += [s_two, s_pair, scrap, y_two, y_pair]
    step, leave_g, leave_u = float(np.float32(0.04)), float(np.float32(0.03)), float(np.float32(0.05))
    pro_two = _Prologue(state.ptr, s_two.ptr, lift.ptr, lift_gain.ptr, 1.0, 0, norm_gain.ptr, 1e-6)
    pro_pair = _Prologue(state.ptr, s_pair.ptr, lift.ptr, lift_gain.ptr, 1.0, 0, norm_gain.ptr, 1e-6)
    g, u = planes
    assert lib.igl_launch_gemv_level_pro(ctypes.byref(g), step, leave_g, ctypes.byref(pro_two), scrap.ptr,
                                         y_two.ptr, N, K, 0, None, stream) == 0
    assert lib.igl_launch_gemv_level_epi(ctypes.byref(u), step, leave_u, scrap.ptr, K, 1, y_two.ptr, N, N, K,
                                         1, y_two.ptr, N, stream) == 0
    assert lib.igl_launch_gemv_level_pair(ctypes.byref(g), ctypes.byref(u), step, leave_g, leave_u,
                                          ctypes.byref(pro_pair), y_pair.ptr, N, K, stream) == 0
    backend.sync()
    want, got = y_two.get(np.float32, N), y_pair.get(np.float32, N)
    assert np.all(np.isfinite(want)) and np.any(want != 0)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(s_pair.get(np.float32, K).view(np.uint32), s_two.get(np.float32, K).view(np.uint32))
    for b in bufs:
        b.free()


@pytest.mark.parametrize("bits,rows,K", [(4, (2048, 256, 256), 1536), (4, (2048, 512, 512), 1536),
                                         (2, (1001, 131, 130), 1536), (8, (256, 77), 2048), (4, (300,), 1024)])
def test_level_segments_equal_separate_launches(backend, bits, rows, K):
    """Up to three calibrated planes of one lane that read the same input (a
    layer's q, k and v; igl_launch_gemv_level_segments: the residual update as
    the prologue, each plane's rows on its own leave grid into its own output)
    equal, to the bit, the launches they replace: the first plane with the
    prologue (igl_launch_gemv_level_pro, x kept) and the others reading the
    kept x (igl_launch_gemv_level_epi); odd row counts put plane boundaries
    inside a row tile."""
    print("case level segments bits=%d rows=%s K=%d" % (bits, rows, K), flush=True)
    lib = backend.lib
    for name, args in (("igl_launch_gemv_level_pro",
                        [ctypes.c_void_p, ctypes.c_float, ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p,
                         ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                         ctypes.c_void_p]),
                       ("igl_launch_gemv_level_epi",
                        [ctypes.c_void_p, ctypes.c_float, ctypes.c_float, ctypes.c_void_p, ctypes.c_int,
                         ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                         ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]),
                       ("igl_launch_gemv_level_segments",
                        [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                         ctypes.c_float, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p])):
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = args
    lib.igl_desk_stream.restype = ctypes.c_void_p
    lib.igl_desk_stream.argtypes = [ctypes.c_void_p]
    stream = lib.igl_desk_stream(ctypes.byref(backend.desk))
    r = np.random.default_rng(bits * 1000 + sum(rows))
    row_bytes = K * bits // 8
    bufs = []

    def up_load(a):
        b = backend.upload(np.ascontiguousarray(a))
        bufs.append(b)
        return b

    n = len(rows)
    views = (_CodeView * 3)()
    for i, N in enumerate(rows):
        codes = up_load(r.integers(0, 256, size=(N, row_bytes), dtype=np.uint8))
        gains = up_load(np.abs(r.normal(0, 0.02, size=N)).astype(np.float32))
        views[i] = _CodeView(codes.ptr, row_bytes, gains.ptr, 1, 31, bits, 1 << (bits - 1), 128 if bits == 8 else 0)
    state = up_load(r.normal(size=K).astype(np.float32))
    lift = up_load(r.normal(size=K).astype(np.float32))
    lift_gain = up_load(r.normal(1.0, 0.1, size=K).astype(np.float32))
    norm_gain = up_load(r.normal(1.0, 0.1, size=K).astype(np.float32))
    s_one, s_seg, scrap = backend.alloc(K * 4), backend.alloc(K * 4), backend.alloc(K * 4)
    y_one = [backend.alloc(N * 4) for N in rows]
    y_seg = [backend.alloc(N * 4) for N in rows]
    bufs += [s_one, s_seg, scrap] + y_one + y_seg
    step = float(np.float32(0.04))
    leaves = [float(np.float32(v)) for v in (0.03, 0.05, 0.0)[:n]]
    pro_one = _Prologue(state.ptr, s_one.ptr, lift.ptr, lift_gain.ptr, 1.0, 0, norm_gain.ptr, 1e-6)
    pro_seg = _Prologue(state.ptr, s_seg.ptr, lift.ptr, lift_gain.ptr, 1.0, 0, norm_gain.ptr, 1e-6)
    assert lib.igl_launch_gemv_level_pro(ctypes.byref(views[0]), step, leaves[0], ctypes.byref(pro_one), scrap.ptr,
                                         y_one[0].ptr, rows[0], K, 0, None, stream) == 0
    for i in range(1, n):
        assert lib.igl_launch_gemv_level_epi(ctypes.byref(views[i]), step, leaves[i], scrap.ptr, K, 1, y_one[i].ptr,
                                             rows[i], rows[i], K, 0, None, 0, stream) == 0
    rows_c = (ctypes.c_int * 3)(*rows)
    outs_c = (ctypes.c_void_p * 3)(*[b.ptr for b in y_seg])
    leave_c = (ctypes.c_float * 3)(*leaves)
    assert lib.igl_launch_gemv_level_segments(views, n, rows_c, outs_c, leave_c, step, ctypes.byref(pro_seg), K,
                                              stream) == 0
    backend.sync()
    for i, N in enumerate(rows):
        want, got = y_one[i].get(np.float32, N), y_seg[i].get(np.float32, N)
        assert np.all(np.isfinite(want)) and np.any(want != 0)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"plane {i}"
    assert np.array_equal(s_seg.get(np.float32, K).view(np.uint32), s_one.get(np.float32, K).view(np.uint32))
    for b in bufs:
        b.free()
