"""Recording and replay of device entries (igl_record_begin / igl_record_end /
igl_replay_run / igl_replay_free): every replay equals the same entries run
eagerly on the same inputs, bit for bit (the same kernels on the same bytes),
with eager work and synchronizations between the replays; entries that touch
host memory are refused while recording; a desk's scratch is frozen while a
replay of it is alive.  No counterpart in the reference."""
import numpy as np
import pytest

from igllm_amd.backend import Backend, BackendError, make_plane, synth_projection

pytestmark = pytest.mark.gpu


@pytest.fixture()
def desk():
    b = Backend(device=0, sum_limit=1024, col_limit=16384, lane_limit=16)
    yield b
    b.close()


def test_replay_equals_eager(desk):
    print("case replay gemv 8192x2048 M=1, 2048x8192 M=1, 8192x2048 M=4, 2048x8192 M=4", flush=True)
    c1, g1, x1 = synth_projection(8192, 2048, 4, seed=0)
    c2, g2, x2 = synth_projection(2048, 8192, 4, seed=1)
    p1 = desk.attach(make_plane(c1, g1, 2048))
    p2 = desk.attach(make_plane(c2, g2, 8192))
    a1 = desk.upload(x1[:1].copy())
    a4 = desk.upload(x1)
    a2 = desk.upload(x2[:1].copy())
    a24 = desk.upload(x2)
    o1, o2, o4 = desk.alloc(8192 * 4), desk.alloc(2048 * 4), desk.alloc(4 * 8192 * 4)
    e1, e2, e4 = desk.alloc(8192 * 4), desk.alloc(2048 * 4), desk.alloc(4 * 8192 * 4)
    o24, e24 = desk.alloc(4 * 2048 * 4), desk.alloc(4 * 2048 * 4)

    def eager():
        desk.gemv_dev(p1, a1, 2048, 1, e1, 8192)
        desk.gemv_dev(p2, a2, 8192, 1, e2, 2048)
        desk.gemv_dev(p1, a4, 2048, 4, e4, 8192)
        desk.gemv_dev(p2, a24, 8192, 4, e24, 2048)  # K-chunked: partials, then their sum
        desk.sync()
        return (e1.get(np.float32, 8192), e2.get(np.float32, 2048), e4.get(np.float32, 4 * 8192),
                e24.get(np.float32, 4 * 2048))

    want = eager()  # also sizes every scratch buffer the entries use
    desk.record_begin()
    desk.gemv_dev(p1, a1, 2048, 1, o1, 8192)
    desk.gemv_dev(p2, a2, 8192, 1, o2, 2048)
    desk.gemv_dev(p1, a4, 2048, 4, o4, 8192)
    desk.gemv_dev(p2, a24, 8192, 4, o24, 2048)
    replay = desk.record_end()
    try:
        rng = np.random.default_rng(7)
        for turn in range(3):
            if turn:
                # new activations in the same buffers: the replay reads them
                a1.put(rng.normal(size=(1, 2048)).astype(np.float32))
                a2.put(rng.normal(size=(1, 8192)).astype(np.float32))
                a4.put(rng.normal(size=(4, 2048)).astype(np.float32))
                a24.put(rng.normal(size=(4, 8192)).astype(np.float32))
                want = eager()
            desk.replay_run(replay)
            desk.sync()
            got = (o1.get(np.float32, 8192), o2.get(np.float32, 2048), o4.get(np.float32, 4 * 8192),
                   o24.get(np.float32, 4 * 2048))
            for g, w in zip(got, want):
                assert np.array_equal(g, w), f"replay {turn} differs from the eager run"
    finally:
        desk.replay_free(replay)
    desk.detach(p1)
    desk.detach(p2)


def test_recording_refuses_host_entries(desk):
    print("case replay refusals", flush=True)
    codes, gains, x = synth_projection(1024, 512, 1, seed=3)
    cp = desk.attach(make_plane(codes, gains, 512))
    a, o = desk.upload(x), desk.alloc(1024 * 4)
    desk.gemv_dev(cp, a, 512, 1, o, 1024)
    desk.sync()
    want = o.get(np.float32, 1024)
    desk.record_begin()
    desk.gemv_dev(cp, a, 512, 1, o, 1024)
    with pytest.raises(BackendError):
        desk.sync()
    with pytest.raises(BackendError):
        desk.record_end()
    # the stream runs eagerly again
    o2 = desk.alloc(1024 * 4)
    desk.gemv_dev(cp, a, 512, 1, o2, 1024)
    desk.sync()
    assert np.array_equal(o2.get(np.float32, 1024), want)
    desk.detach(cp)


def test_scratch_frozen_while_replay_lives(desk):
    print("case replay frozen scratch", flush=True)
    codes, gains, x = synth_projection(1024, 512, 1, seed=4)
    cp = desk.attach(make_plane(codes, gains, 512))
    a, o = desk.upload(x), desk.alloc(1024 * 4)
    desk.gemv_dev(cp, a, 512, 1, o, 1024)
    desk.record_begin()
    desk.gemv_dev(cp, a, 512, 1, o, 1024)
    replay = desk.record_end()
    # a prefill GEMM would size the desk's binary16 activation copy: refused
    M = 256
    act = desk.upload((np.random.default_rng(5).normal(size=M * 512).astype(np.float32).view(np.uint32)
                       >> 16).astype(np.uint16))
    out = desk.alloc(M * 1024 * 2)
    try:
        with pytest.raises(BackendError):
            desk.gemm_bf16_dev(cp, act, 512, M, out, 1024)
    finally:
        desk.replay_free(replay)
    desk.gemm_bf16_dev(cp, act, 512, M, out, 1024)
    desk.sync()
    desk.detach(cp)
