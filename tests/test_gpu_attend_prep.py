"""GPU parity of the prepared decode attention (igl_launch_attend_prep): a
decode step's or a small speculative block's query, key and value heads
prepared in the attention launch itself, against the oracle on the same
seeded inputs.

For lanes at positions p .. p + lanes - 1 (one key/value head shared by 8
query heads, e4m3 rings, score scale 1.0 as the model runs it):
- each new key row is norm(k) * gain turned by its position's (cos, sin)
  pairs, and each new value row norm(v) (session_attend 11504-11510), encoded
  as e4m3 bytes at the layer's scale (cache_lay 11205-11236) into ring slot
  position % cache_span.  The GPU's own norm step and the host compiler's
  float contraction may each move a value by one ulp, so a byte may land one
  e4m3 step away at a rounding boundary: at most 0.5% of the bytes, and none
  further than one step;
- each lane's blend is the oracle's attention (oracle_attend) over the ring
  as it stands after the launch, lane l seeing the positions up to p + l
  inside its window, with its own prepared query heads.  Bar: 1e-3 max|o| +
  1e-5, as the other attention tests;
- a layer that reads another layer's rings (no raw key or value) writes no
  row and reads the block's own positions from the ring.
"""
import ctypes

import numpy as np
import pytest

import oracle_lib as ol

pytestmark = pytest.mark.gpu

HEADS = 8
EPS = 1e-6


def _bind(lib):
    fn = lib.igl_launch_attend_prep
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float, ctypes.c_float, ctypes.c_int, ctypes.c_int,
                   ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                   ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                   ctypes.c_void_p, ctypes.c_float, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_float,
                   ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.igl_attend_prep_work_floats.restype = ctypes.c_size_t
    lib.igl_attend_prep_work_floats.argtypes = [ctypes.c_int] * 5
    lib.igl_desk_stream.restype = ctypes.c_void_p
    lib.igl_desk_stream.argtypes = [ctypes.c_void_p]
    return fn


def _norm(x, gain):
    out = np.empty_like(x)
    ol.oracle().oracle_norm_rms(ol.p(x), None if gain is None else ol.p(gain), x.size, EPS, ol.p(out))
    return out


def _turned(x, cos_row, sin_row):
    y = x.copy()
    ol.oracle().oracle_rope_turn(ol.p(y), y.size, ol.p(cos_row), ol.p(sin_row))
    return y


@pytest.mark.parametrize("lanes,window,pos,head,writes", [
    (1, 512, 700, 256, True),     # a decode step on a sliding layer past the ring's wrap
    (2, 512, 700, 256, True),     # a two-lane block
    (3, 512, 1030, 256, True),
    (4, 512, 3, 256, True),       # the block's own positions are most of the span
    (2, 0, 300, 512, True),       # a global layer
    (4, 0, 37, 512, True),
    (2, 512, 640, 256, False),    # a layer reading another layer's rings
])
def test_prepared_attention(backend, lanes, window, pos, head, writes):
    print("case prepared attention lanes=%d window=%d pos=%d head=%d writes=%d" % (lanes, window, pos, head,
                                                                                     writes), flush=True)
    lib = backend.lib
    fn = _bind(lib)
    stream = lib.igl_desk_stream(ctypes.byref(backend.desk))
    r = np.random.default_rng(lanes * 1000 + pos + head)
    half = head // 2
    cache_span = window + 16 if window else pos + lanes + 8
    k_scale, v_scale = 0.02, 0.015
    # rings: every position before the block; a reader of another layer's
    # rings also finds the block's own rows there
    filled = pos if writes else pos + lanes
    k_vals = np.clip(r.normal(0, 1.5, size=(cache_span, head)), -8, 8).astype(np.float32)
    v_vals = np.clip(r.normal(0, 1.5, size=(cache_span, head)), -8, 8).astype(np.float32)
    ring_k = ol.encode(k_vals, k_scale, 0)
    ring_v = ol.encode(v_vals, v_scale, 0)
    q_stride, kv_stride, turn_stride = HEADS * head + 64, head + 32, head
    q_raw = r.normal(size=(lanes, q_stride)).astype(np.float32)
    k_raw = r.normal(size=(lanes, kv_stride)).astype(np.float32)
    v_raw = r.normal(size=(lanes, kv_stride)).astype(np.float32)
    q_gain = r.normal(1.0, 0.1, size=head).astype(np.float32)
    k_gain = r.normal(1.0, 0.1, size=head).astype(np.float32)
    steps = (1.0 / np.power(10000.0, np.arange(half, dtype=np.float64) * 2.0 / head)).astype(np.float32)
    angles = (pos + np.arange(lanes, dtype=np.float64))[:, None] * steps.astype(np.float64)[None, :]
    cos_rows, sin_rows = np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)
    turn = np.zeros((lanes, turn_stride), dtype=np.float32)
    turn[:, 0:2 * half:2], turn[:, 1:2 * half:2] = cos_rows, sin_rows

    bound = pos + 5 if window else pos  # a grid sized past the position, as a graph sizes it
    bufs = []

    def up(a):
        b = backend.upload(np.ascontiguousarray(a))
        bufs.append(b)
        return b

    d_k, d_v = up(ring_k), up(ring_v)
    d_q, d_kr, d_vr = up(q_raw), up(k_raw), up(v_raw)
    d_qg, d_kg, d_turn = up(q_gain), up(k_gain), up(turn)
    d_place = up(np.array([pos], dtype=np.int32))
    d_out = backend.alloc(lanes * q_stride * 4)
    d_work = backend.alloc(lib.igl_attend_prep_work_floats(bound, window, head, lanes, 1 if writes else 0) * 4)
    bufs += [d_out, d_work]
    try:
        rc = fn(d_k.ptr, d_v.ptr, k_scale, v_scale, cache_span, head, lanes, d_q.ptr, q_stride, d_qg.ptr,
                d_turn.ptr, turn_stride, d_kr.ptr if writes else None, d_vr.ptr if writes else None, kv_stride,
                d_kg.ptr, d_k.ptr, d_v.ptr, EPS, bound, d_place.ptr, window, 1.0, d_out.ptr, d_work.ptr, stream)
        assert rc == 0
        backend.sync()
        got = d_out.get(np.float32, lanes * q_stride).reshape(lanes, q_stride)
        got_k = d_k.get(np.uint8, cache_span * head).reshape(cache_span, head)
        got_v = d_v.get(np.uint8, cache_span * head).reshape(cache_span, head)
    finally:
        for b in bufs:
            b.free()

    grid_k, grid_v = ol.grid8(k_scale), ol.grid8(v_scale)
    if writes:
        for l in range(lanes):
            slot = (pos + l) % cache_span
            want_k = ol.encode(_turned(_norm(k_raw[l, :head], k_gain), cos_rows[l], sin_rows[l]), k_scale, 0)
            want_v = ol.encode(_norm(v_raw[l, :head], None), v_scale, 0)
            for got_row, want_row, grid in ((got_k[slot], want_k, grid_k), (got_v[slot], want_v, grid_v)):
                off = got_row != want_row
                assert np.mean(off) <= 0.005, (l, int(off.sum()))
                # a byte off sits one e4m3 step from the oracle's: the nearest
                # grid value on one side or the other
                gv, wv = grid[got_row[off]], grid[want_row[off]]
                order = np.sort(grid)
                for a, b in zip(gv, wv):
                    ia, ib = np.searchsorted(order, a), np.searchsorted(order, b)
                    assert abs(int(ia) - int(ib)) <= 1
        # every other slot keeps its bytes
        keep = np.ones(cache_span, dtype=bool)
        keep[[(pos + l) % cache_span for l in range(lanes)]] = False
        assert np.array_equal(got_k[keep], ring_k[keep]) and np.array_equal(got_v[keep], ring_v[keep])
    else:
        assert np.array_equal(got_k, ring_k) and np.array_equal(got_v, ring_v)

    for l in range(lanes):
        q = np.stack([_turned(_norm(q_raw[l, h * head:(h + 1) * head], q_gain), cos_rows[l], sin_rows[l])
                      for h in range(HEADS)])
        span = min(pos + l + 1, window) if window else pos + l + 1
        start = pos + l - span + 1
        want = ol.oracle_attend(got_k, got_v, grid_k, grid_v, cache_span, head, 0, q, 0, HEADS, head, start, span,
                                1.0)
        have = got[l, :HEADS * head].reshape(HEADS, head)
        err = float(np.max(np.abs(have - want)))
        assert err <= 1e-3 * float(np.max(np.abs(want))) + 1e-5, (l, err)
