"""The attention entry that allocates nothing (igl_attend_lanes_fixed_dev)
against the ordinary one (igl_attend_lanes_dev), through the C ABI.

Both run the same kernels on the same inputs; the fixed entry keeps its chunk
partials in a per-GPU array of IGL_ATTEND_FIXED_FLOATS floats instead of the
desk's workspace, so the outputs must agree bit for bit.  Two calls in a row,
the second smaller (the array keeps the first call's contents), and a call too
large for the array, refused on the host with IGL_FAIL_SUPPORT before any
launch.
"""
import ctypes

import numpy as np
import pytest

import oracle_lib as ol
from igllm_amd import native

pytestmark = pytest.mark.gpu

FIXED_FLOATS = 1 << 21


def ring(rng, span, head, scale):
    return ol.encode(np.clip(rng.normal(size=(span, head)), -4, 4).astype(np.float32), scale, 1)


def run(backend, entry, k, v, scale, span, head, q, lanes, place_first, window):
    lib, desk = backend.lib, ctypes.byref(backend.desk)
    out = backend.alloc(lanes * 8 * head * 4)
    fn = getattr(lib, entry)
    code = fn(desk, k.ptr, v.ptr, native.IGL_CACHE_INT8, scale, scale, span, 1, 8, head, q.ptr, 8 * head,
              place_first, window, lanes, 1.0 / 16, out.ptr)
    assert code == native.IGL_OKAY, (entry, code)
    backend.sync()
    return out.get(np.float32, lanes * 8 * head)


def test_fixed_entry_matches_the_allocating_one(backend):
    rng = np.random.default_rng(7)
    scale = 4.0 / 127.0
    head, span = 256, 4096
    k = backend.upload(ring(rng, span, head, scale))
    v = backend.upload(ring(rng, span, head, scale))
    # first a 4-lane batch ending at position 3003, then one lane at 599 in a
    # 512-position window: fewer partials than the first call left behind
    for lanes, place_first, window in ((4, 3000, 0), (1, 599, 512)):
        q = backend.upload(rng.normal(size=(lanes, 8, head)).astype(np.float32))
        print("case", lanes, place_first, window, flush=True)
        want = run(backend, "igl_attend_lanes_dev", k, v, scale, span, head, q, lanes, place_first, window)
        got = run(backend, "igl_attend_lanes_fixed_dev", k, v, scale, span, head, q, lanes, place_first,
                  window)
        assert np.isfinite(want).all()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_fixed_entry_refuses_what_does_not_fit(backend):
    lib, desk = backend.lib, ctypes.byref(backend.desk)
    head, span, lanes = 512, 16384, 16
    # 16 lanes ending at position 16383 of 512-wide heads need
    # 16 * 128 chunks * 8 heads * 514 floats, past the array
    assert 16 * 128 * 8 * (head + 2) > FIXED_FLOATS
    k = backend.alloc(span * head)
    v = backend.alloc(span * head)
    q = backend.alloc(lanes * 8 * head * 4)
    out = backend.alloc(lanes * 8 * head * 4)
    code = lib.igl_attend_lanes_fixed_dev(desk, k.ptr, v.ptr, native.IGL_CACHE_INT8, 1.0, 1.0, span, 1, 8,
                                          head, q.ptr, 8 * head, span - lanes, 0, lanes, 1.0, out.ptr)
    assert code == native.IGL_FAIL_SUPPORT
    assert lib.igl_desk_error_take(desk) == native.IGL_FAIL_SUPPORT
    assert lib.igl_desk_error_take(desk) == native.IGL_OKAY
