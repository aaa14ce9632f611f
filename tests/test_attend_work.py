"""CPU check of the attention workspace the engine allocates at open.

The decode attention writes one partial per (lane, chunk, head).  Its chunk
count is not monotonic in the span (32-position chunks up to 8192 positions,
64-position chunks beyond, and for every launch of 64 lanes and more), so a
batch whose last position lands just under
8192 needs more partials than a decode step at the last position of a longer
window.  The engine sizes the buffer with igl_attend_work_floats_limit; this
replays every (position, lanes) pair a prime, a speculative block or a decode
step can launch with, and checks each launch's need against that size.  Pure
host arithmetic: no device is touched.
"""
import ctypes

import pytest

HEADS, HEAD = 8, 512


@pytest.fixture(scope="module")
def lib():
    from igllm_amd import native

    lib = native.load()
    for name in ("igl_attend_work_floats", "igl_attend_work_floats_limit", "igl_attend_prep_work_floats"):
        getattr(lib, name).restype = ctypes.c_size_t
    lib.igl_attend_work_floats.argtypes = [ctypes.c_int] * 5
    lib.igl_attend_work_floats_limit.argtypes = [ctypes.c_int] * 4
    lib.igl_attend_prep_work_floats.argtypes = [ctypes.c_int] * 5
    return lib


@pytest.mark.parametrize("window_limit", [4097, 8192, 8193, 12000, 16000])
@pytest.mark.parametrize("lane_limit", [16, 2048])
def test_every_launch_fits_the_engine_allocation(lib, window_limit, lane_limit):
    have = lib.igl_attend_work_floats_limit(window_limit, lane_limit, HEADS, HEAD)
    lane_counts = sorted({1, 2, 3, 15, 16, 63, 64, 255, 2047, 2048} & set(range(1, lane_limit + 1)))
    worst = 0
    for window in (0, 512):  # full layers see every position, sliding ones the last 512
        # decode step: the graph is sized for the last position
        worst = max(worst, lib.igl_attend_work_floats(window_limit - 1, window, 1, HEADS, HEAD))
        for lanes in lane_counts:
            for fill in range(0, window_limit - lanes + 1):
                worst = max(worst, lib.igl_attend_work_floats(fill, window, lanes, HEADS, HEAD))
    assert worst <= have, (worst, have)


def test_longest_span_alone_falls_short(lib):
    """Sizing by a decode step at the last position, or by a full batch ending
    there, is smaller than a 16-lane batch ending at position 8191 of a
    12000-position window: the case the limit covers."""
    W, lanes = 12000, 16
    one = lib.igl_attend_work_floats(W - 1, 0, 1, HEADS, HEAD)
    many = lib.igl_attend_work_floats(W - lanes, 0, lanes, HEADS, HEAD)
    need = lib.igl_attend_work_floats(8192 - lanes, 0, lanes, HEADS, HEAD)
    assert need > max(one, many)
    assert need <= lib.igl_attend_work_floats_limit(W, lanes, HEADS, HEAD)


@pytest.mark.parametrize("window_limit", [1, 33, 4097, 8192, 8193, 12000])
@pytest.mark.parametrize("lane_limit", [1, 16, 2048])
@pytest.mark.parametrize("head", [256, 512])
def test_decode_step_fits_the_engine_allocation(lib, window_limit, lane_limit, head):
    """The prepared attention of a decode step or a small block (up to four
    lanes) writes one partial slot a lane more than its chunks (the new
    positions' own); its graph is sized for the last positions, on full and
    sliding layers, with and without rows to write, and an eager pass or a
    prime's tail launches it at every position before that."""
    have = lib.igl_attend_work_floats_limit(window_limit, lane_limit, HEADS, head)
    for lanes in range(1, min(4, lane_limit, window_limit) + 1):
        for window in (0, 512):
            for writes in (0, 1):
                for bound in sorted({window_limit - lanes, max(0, 8192 - lanes), max(0, window_limit // 2)}):
                    if bound > window_limit - lanes:
                        continue
                    need = lib.igl_attend_prep_work_floats(bound, window, head, lanes, writes)
                    assert need <= have, (lanes, window, writes, bound, need, have)
