"""Lanes as rows of one-lane workgroups (`lane_rows`): a launch of two to four
lanes whose form runs every lane as the one-lane launch (up to eight for the
grouped launches) gives each lane that launch's outputs to the bit.  Checked on the integer-dot GEMV (planes where
gemv_lane_rows_pay takes the rows) and on the grouped decode launches
(igl_launch_gemv_group: q/k/v segments, gate/up with gelu * up and the
residual-update prologue, the per-layer-input gate with gelu * mul), against
the same launch made one lane at a time on the same buffers.  The one-lane
launches themselves are held to the oracle by test_gpu_projection and the
decode streams by test_gpu_e2e.
"""
import ctypes

import numpy as np
import pytest

import launch_structs
from igllm_amd.backend import make_plane, synth_projection

pytestmark = pytest.mark.gpu

GEMV_SEGMENTS, GEMV_GELU_PAIR, GEMV_GELU_MUL = 0, 1, 2


@pytest.mark.parametrize("N,K,lanes", [(1536, 2048, 2), (1536, 2048, 4), (4096, 2048, 3), (1536, 6144, 4),
                                       (1537, 256, 3), (999, 4096, 2)])
def test_gemv_lane_rows_equal_one_lane(backend, N, K, lanes):
    print("case gemv lane rows N=%d K=%d lanes=%d" % (N, K, lanes), flush=True)
    codes, gains, act = synth_projection(N, K, lanes, seed=N + K + lanes)
    cp = backend.attach(make_plane(codes, gains, K))
    d_act = backend.upload(act)
    d_all, d_one = backend.alloc(lanes * N * 4), backend.alloc(lanes * N * 4)
    try:
        backend.gemv_dev(cp, d_act, K, lanes, d_all, N)
        for l in range(lanes):
            backend.gemv_dev(cp, d_act, K, 1, d_one, N, act_off=4 * l * K, out_off=4 * l * N)
        backend.sync()
        got = d_all.get(np.float32, lanes * N)
        one = d_one.get(np.float32, lanes * N)
        assert np.array_equal(got.view(np.uint32), one.view(np.uint32))
    finally:
        for b in (d_act, d_all, d_one):
            b.free()
        backend.detach(cp)


def _bind(lib):
    fn = lib.igl_launch_gemv_group
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                   ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                   ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                   ctypes.c_void_p, ctypes.c_void_p]
    lib.igl_desk_stream.restype = ctypes.c_void_p
    lib.igl_desk_stream.argtypes = [ctypes.c_void_p]
    return fn


@pytest.mark.parametrize("mode,rows,K,lanes,pro", [
    (GEMV_SEGMENTS, (2048, 256, 256), 1536, 3, False),   # a first layer's q/k/v from normed x
    (GEMV_SEGMENTS, (2048, 256, 256), 1536, 2, True),    # q/k/v with the pending update
    (GEMV_GELU_PAIR, (12288, 12288), 1536, 2, True),     # gate/up, two tiles a wave
    (GEMV_GELU_PAIR, (6144, 6144), 1536, 4, True),
    (GEMV_GELU_MUL, (256,), 1536, 3, True),              # the per-layer-input gate, K split four ways
    (GEMV_SEGMENTS, (4096, 512, 512), 2048, 4, True),
    (GEMV_GELU_PAIR, (6144, 6144), 1536, 8, True),       # a block of eight lanes
    (GEMV_GELU_MUL, (256,), 1536, 6, True),
])
def test_group_lane_rows_equal_one_lane(backend, mode, rows, K, lanes, pro):
    print("case group lane rows mode=%d rows=%s K=%d lanes=%d pro=%d" % (mode, rows, K, lanes, pro), flush=True)
    lib = backend.lib
    fn = _bind(lib)
    stream = lib.igl_desk_stream(ctypes.byref(backend.desk))
    r = np.random.default_rng(mode * 100 + lanes * 10 + K)
    segs = len(rows)
    bufs = []

    def up(a):
        b = backend.upload(np.ascontiguousarray(a))
        bufs.append(b)
        return b

    def alloc(n):
        b = backend.alloc(n)
        bufs.append(b)
        return b

    codes = [up(r.integers(0, 256, size=(n, K // 2), dtype=np.uint8)) for n in rows]
    gains = [up(np.abs(r.normal(0, 0.02, size=(n, K // 32))).astype(np.float32)) for n in rows]
    act_stride = K + 32
    act = up(r.normal(size=(lanes, act_stride)).astype(np.float32))
    state = up(r.normal(size=(lanes, act_stride)).astype(np.float32))
    lift = up(r.normal(size=(lanes, act_stride)).astype(np.float32))
    lift_gain = up(r.normal(1.0, 0.1, size=K).astype(np.float32))
    norm_gain = up(r.normal(1.0, 0.1, size=K).astype(np.float32))
    mul_stride = 300
    mul = up(r.normal(size=(lanes, mul_stride)).astype(np.float32))
    out_stride = [n + 16 for n in rows]
    outs_all = [alloc(lanes * s * 4) for s in out_stride]
    outs_one = [alloc(lanes * s * 4) for s in out_stride]
    state_all, state_one = alloc(lanes * act_stride * 4), alloc(lanes * act_stride * 4)

    def launch(l0, n_lanes, outs, state_out):
        off = 4 * l0 * act_stride

        def seg_ptrs(vals):
            return (ctypes.c_void_p * 3)(*([v for v in vals] + [None] * (3 - len(vals))))

        codes_p = seg_ptrs([c.ptr for c in codes])
        gains_p = seg_ptrs([g.ptr for g in gains])
        outs_p = seg_ptrs([o.ptr + 4 * l0 * s for o, s in zip(outs, out_stride)])
        strides = (ctypes.c_longlong * 3)(*([K // 2] * 3))
        gstride = (ctypes.c_int * 3)(*([K // 32] * 3))
        rows_c = (ctypes.c_int * 3)(*(list(rows) + [0] * (3 - segs)))
        ostride = (ctypes.c_int * 3)(*(out_stride + [0] * (3 - segs)))
        p = None
        if pro:
            p = launch_structs.Prologue(state.ptr + off, state_out.ptr + off, lift.ptr + off, lift_gain.ptr, 1.0, 0,
                                        norm_gain.ptr if mode != GEMV_GELU_MUL else None, 1e-6, act_stride)
        rc = fn(mode, n_lanes, segs, codes_p, strides, gains_p, gstride, rows_c, outs_p, ostride, 0, 8,
                None if pro else act.ptr + off, act_stride, K, mul.ptr + 4 * l0 * mul_stride if mode == GEMV_GELU_MUL
                else None, mul_stride, ctypes.byref(p) if p is not None else None, stream)
        assert rc == 0

    try:
        launch(0, lanes, outs_all, state_all)
        for l in range(lanes):
            launch(l, 1, outs_one, state_one)
        backend.sync()
        written = [rows[0]] if mode != GEMV_SEGMENTS else list(rows)
        for s, (oa, oo) in enumerate(zip(outs_all, outs_one)):
            if s >= len(written):
                break
            a = oa.get(np.float32, lanes * out_stride[s]).reshape(lanes, out_stride[s])[:, :written[s]]
            o = oo.get(np.float32, lanes * out_stride[s]).reshape(lanes, out_stride[s])[:, :written[s]]
            assert np.array_equal(a.view(np.uint32), o.view(np.uint32)), s
        if pro:
            a = state_all.get(np.float32, lanes * act_stride).reshape(lanes, act_stride)[:, :K]
            o = state_one.get(np.float32, lanes * act_stride).reshape(lanes, act_stride)[:, :K]
            assert np.array_equal(a.view(np.uint32), o.view(np.uint32))
    finally:
        for b in bufs:
            b.free()
