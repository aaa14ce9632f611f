"""GPU parity of the wide attention launch (igl_launch_attend with 64 lanes or
more, a prefill pass): one workgroup a lane and key/value head walks the
lane's chunks and merges them online, instead of a workgroup a chunk and a
fold launch.

For lanes at positions p .. p + lanes - 1 over a byte ring (e4m3 or int8),
each lane seeing the positions up to its own inside its window:
- every lane's blend against the same lanes launched 63 at a time (the chunk
  workgroups and their fold): the two forms add the same terms in another
  order, bar 1e-5 max|o| + 1e-7;
- sampled lanes against the oracle (oracle_attend over the lane's span), bar
  1e-3 max|o| + 1e-5 as the other attention tests.
"""
import ctypes

import numpy as np
import pytest

import oracle_lib as ol

pytestmark = pytest.mark.gpu

HEADS = 8
NARROW = 63  # lanes a launch below the wide form takes


def _bind(lib):
    fn = lib.igl_launch_attend
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_int,
                   ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                   ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_void_p,
                   ctypes.c_void_p, ctypes.c_void_p]
    lib.igl_attend_work_floats.restype = ctypes.c_size_t
    lib.igl_attend_work_floats.argtypes = [ctypes.c_int] * 5
    lib.igl_desk_stream.restype = ctypes.c_void_p
    lib.igl_desk_stream.argtypes = [ctypes.c_void_p]
    return fn


@pytest.mark.parametrize("lanes,window,place0,head,fmt,kv_count,pad", [
    (64, 0, 65, 512, 0, 1, 0),       # a global layer, two and three chunks
    (100, 0, 37, 256, 1, 1, 0),      # int8 ring, ragged last chunk
    (300, 512, 1000, 256, 0, 1, 0),  # a sliding layer, windows cut mid-chunk
    (130, 512, 2000, 256, 0, 2, 0),  # two key/value heads, the ring wrapped
    (257, 0, 1500, 512, 0, 1, 0),    # a global layer at 1500-1756 positions
    (300, 512, 100, 256, 0, 1, 0),   # a sliding layer whose first spans are shorter than the window
    (96, 0, 200, 256, 1, 1, 1),      # lanes one float off 16-byte alignment (scalar query loads)
])
def test_wide_attention(backend, lanes, window, place0, head, fmt, kv_count, pad):
    print("case wide attention lanes=%d window=%d place0=%d head=%d fmt=%d kv=%d pad=%d" % (
        lanes, window, place0, head, fmt, kv_count, pad), flush=True)
    lib = backend.lib
    fn = _bind(lib)
    stream = lib.igl_desk_stream(ctypes.byref(backend.desk))
    r = np.random.default_rng(lanes + place0 + head + fmt)
    last = place0 + lanes - 1
    cache_span = window + lanes if window else last + 1
    kv_width = kv_count * head
    scale = 4.0 / 127.0 if fmt == 1 else 0.02
    k_bytes = ol.encode(np.clip(r.normal(size=(cache_span, kv_width)), -4, 4).astype(np.float32) *
                        (1.0 if fmt == 1 else 0.05), scale, fmt)
    v_bytes = ol.encode(np.clip(r.normal(size=(cache_span, kv_width)), -4, 4).astype(np.float32) *
                        (1.0 if fmt == 1 else 0.05), scale, fmt)
    q_stride = kv_count * HEADS * head + pad
    query = r.normal(size=(lanes, q_stride)).astype(np.float32)
    score_scale = 1.0 / 16.0
    dk, dv, dq = backend.upload(k_bytes), backend.upload(v_bytes), backend.upload(query)
    wide = backend.alloc(lanes * q_stride * 4)
    narrow = backend.alloc(lanes * q_stride * 4)
    for b in (wide, narrow):  # the pad columns compare equal
        b.put(np.zeros(lanes * q_stride, np.float32))
    work_floats = max([lib.igl_attend_work_floats(place0 + at, window, min(NARROW, lanes - at), kv_count * HEADS,
                                                  head) for at in range(0, lanes, NARROW)] + [1])
    work = backend.alloc(work_floats * 4)
    try:
        rc = fn(dk.ptr, dv.ptr, fmt, scale, scale, cache_span, kv_width, kv_count, HEADS, head, dq.ptr, q_stride,
                place0, None, window, lanes, score_scale, wide.ptr, work.ptr, stream)
        assert rc == 0
        for at in range(0, lanes, NARROW):
            n = min(NARROW, lanes - at)
            rc = fn(dk.ptr, dv.ptr, fmt, scale, scale, cache_span, kv_width, kv_count, HEADS, head,
                    dq.ptr + at * q_stride * 4, q_stride, place0 + at, None, window, n, score_scale,
                    narrow.ptr + at * q_stride * 4, work.ptr, stream)
            assert rc == 0
            backend.sync()  # the next group reuses the partials
        backend.sync()
        got = wide.get(np.float32, lanes * q_stride).reshape(lanes, q_stride)
        ref = narrow.get(np.float32, lanes * q_stride).reshape(lanes, q_stride)
        top = float(np.max(np.abs(ref)))
        err = float(np.max(np.abs(got - ref)))
        print("vs chunk workgroups: max err", err, "max |o|", top)
        assert err <= 1e-5 * top + 1e-7
        grid = ol.grid_i8(scale) if fmt == 1 else ol.grid8(scale)
        for lane in sorted({0, 1, lanes // 2, lanes - 2, lanes - 1}):
            pos = place0 + lane
            span = min(pos + 1, window) if window else pos + 1
            for kv in range(kv_count):
                q = query[lane, kv * HEADS * head:(kv + 1) * HEADS * head].reshape(HEADS, head)
                want = ol.oracle_attend(k_bytes, v_bytes, grid, grid, cache_span, kv_width, kv, q, 0, HEADS, head,
                                        pos - span + 1, span, score_scale)
                have = got[lane, kv * HEADS * head:(kv + 1) * HEADS * head].reshape(HEADS, head)
                e = float(np.max(np.abs(have - want)))
                assert e <= 1e-3 * float(np.max(np.abs(want))) + 1e-5, (lane, kv, e)
    finally:
        for b in (dk, dv, dq, wide, narrow, work):
            b.free()
