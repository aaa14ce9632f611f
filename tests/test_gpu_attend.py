"""GPU parity of decode attention over the byte key/value ring, and of the
cache writer, against the oracle on the same seeded inputs.

Bar: every output within 1e-3 * max|o_ref| + 1e-5 of the oracle (outputs are
convex blends of decoded values ~N(0,1); the GPU reassociates the dot
products and uses the hardware exponential).  The cache writer is bit-exact.
"""
import numpy as np
import pytest

import oracle_lib as ol

pytestmark = pytest.mark.gpu

HEADS, KV = 8, 1


def make_inputs(cache_span, head, fmt, seed):
    r = np.random.default_rng(seed)
    scale = (4.0 / 448.0) if fmt == 0 else (4.0 / 127.0)
    k = np.clip(r.normal(size=(cache_span, KV * head)), -4, 4).astype(np.float32)
    v = np.clip(r.normal(size=(cache_span, KV * head)), -4, 4).astype(np.float32)
    q = r.normal(size=(HEADS * KV, head)).astype(np.float32)
    return scale, ol.encode(k, scale, fmt), ol.encode(v, scale, fmt), q


def run(backend, kb, vb, q, fmt, scale, cache_span, head, start, span, score_scale):
    dk, dv, dq = backend.upload(kb), backend.upload(vb), backend.upload(q)
    do = backend.alloc(q.nbytes)
    backend.attend_dev(dk, dv, fmt, scale, scale, cache_span, KV, HEADS, head, dq, start, span,
                       score_scale, do)
    backend.sync()
    out = do.get(np.float32, q.size).reshape(q.shape)
    for b in (dk, dv, dq, do):
        b.free()
    return out


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("L", [1, 7, 128, 129, 512, 4096, 16384])
def test_attend_full_span(backend, fmt, L):
    head = 256
    score_scale = 1.0 / 16.0
    print("case attend", "fmt", fmt, "L", L, flush=True)
    scale, kb, vb, q = make_inputs(L, head, fmt, seed=L)
    got = run(backend, kb, vb, q, fmt, scale, L, head, 0, L, score_scale)
    grid = ol.grid8(scale) if fmt == 0 else ol.grid_i8(scale)
    want = ol.oracle_attend(kb, vb, grid, grid, L, head, 0, q, 0, HEADS, head, 0, L, score_scale)
    err = float(np.max(np.abs(got - want)))
    print("max_abs_err", err, "max_ref", float(np.max(np.abs(want))))
    assert err <= 1e-3 * float(np.max(np.abs(want))) + 1e-5


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("pos", [512, 700, 1023, 5000])
def test_attend_sliding_ring(backend, fmt, pos):
    """Sliding window 512 over a ring of 512 slots, at positions past the first
    wrap: start = pos - 511, slots (start + t) % 512 (app_core.c:11500, 11516-11526)."""
    head, span_ring = 256, 512
    start = max(0, pos - 512 + 1)
    span = pos - start + 1
    scale, kb, vb, q = make_inputs(span_ring, head, fmt, seed=pos)
    got = run(backend, kb, vb, q, fmt, scale, span_ring, head, start, span, 1.0 / 16.0)
    grid = ol.grid8(scale) if fmt == 0 else ol.grid_i8(scale)
    want = ol.oracle_attend(kb, vb, grid, grid, span_ring, head, 0, q, 0, HEADS, head, start, span,
                            1.0 / 16.0)
    assert float(np.max(np.abs(got - want))) <= 1e-3 * float(np.max(np.abs(want))) + 1e-5


@pytest.mark.parametrize("L", [300, 4096])
def test_attend_reference_graph_head512(backend, L):
    """The reference graph's own setting: score scale 1.0 (q/k norms absorb
    1/sqrt(d)), e4m3 bytes, and the 512-wide heads of the full layers."""
    head = 512
    scale, kb, vb, q = make_inputs(L, head, 0, seed=3)
    q *= 0.05  # normed queries keep unscaled scores in a sane range
    got = run(backend, kb, vb, q, 0, scale, L, head, 0, L, 1.0)
    grid = ol.grid8(scale)
    want = ol.oracle_attend(kb, vb, grid, grid, L, head, 0, q, 0, HEADS, head, 0, L, 1.0)
    assert float(np.max(np.abs(got - want))) <= 1e-3 * float(np.max(np.abs(want))) + 1e-5


@pytest.mark.parametrize("fmt", [0, 1])
def test_cache_lay_bitexact(backend, fmt):
    r = np.random.default_rng(17)
    width = 4096
    scale = (4.0 / 448.0) if fmt == 0 else (4.0 / 127.0)
    row = np.concatenate([
        r.normal(size=width - 16) * 3,
        [0.0, -0.0, 1e9, -1e9, 448 * scale, 449 * scale, 2.0 ** -10 * scale, -2.0 ** -10 * scale,
         1.5 * 2.0 ** -9 * scale, 2.5 * 2.0 ** -9 * scale, 7.5 * 2.0 ** -9 * scale, 15.5 * scale,
         4.0, -4.0, 127.5 * scale, -127.5 * scale]]).astype(np.float32)
    dr = backend.upload(row)
    store = backend.alloc(width + 64)
    backend.cache_lay_dev(dr, width, scale, fmt, store, 32)
    backend.sync()
    got = store.get(np.uint8, width, offset=32)
    want = ol.encode(row, scale, fmt)
    assert np.array_equal(got, want)
    dr.free()
    store.free()


class _At:
    """A device address inside a buffer (an unaligned query)."""

    def __init__(self, buf, offset):
        self.ptr = buf.ptr + offset


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("kv", [1, 2])
@pytest.mark.parametrize("span,aligned", [(33, True), (64, True), (300, False), (511, True), (512, False)])
def test_attend_short_span_kv_heads(backend, fmt, kv, span, aligned):
    """One lane over 2-16 chunks of 32 positions (the sliding-window layers'
    spans), with one and two key/value heads, 16-byte aligned and unaligned
    queries, at a ring offset that wraps."""
    head = 256
    cache_span = 640
    start = 600  # slots (600 + t) % 640: the span wraps
    r = np.random.default_rng(span + 7 * kv + fmt)
    scale = (4.0 / 448.0) if fmt == 0 else (4.0 / 127.0)
    k = np.clip(r.normal(size=(cache_span, kv * head)), -4, 4).astype(np.float32)
    v = np.clip(r.normal(size=(cache_span, kv * head)), -4, 4).astype(np.float32)
    q = r.normal(size=(HEADS * kv, head)).astype(np.float32)
    kb, vb = ol.encode(k, scale, fmt), ol.encode(v, scale, fmt)
    print("case short span", "fmt", fmt, "kv", kv, "span", span, "aligned", aligned, flush=True)
    dk, dv = backend.upload(kb), backend.upload(vb)
    qbuf = backend.alloc(q.nbytes + 16)
    off = 0 if aligned else 4
    qbuf.put(q, off)
    do = backend.alloc(q.nbytes)
    backend.attend_dev(dk, dv, fmt, scale, scale, cache_span, kv, HEADS, head, _At(qbuf, off), start, span,
                       1.0 / 16.0, do)
    backend.sync()
    got = do.get(np.float32, q.size).reshape(q.shape)
    for b in (dk, dv, qbuf, do):
        b.free()
    grid = ol.grid8(scale) if fmt == 0 else ol.grid_i8(scale)
    for j in range(kv):
        want = ol.oracle_attend(kb, vb, grid, grid, cache_span, kv * head, j, q[HEADS * j:HEADS * (j + 1)],
                                0, HEADS, head, start, span, 1.0 / 16.0)
        err = float(np.max(np.abs(got[HEADS * j:HEADS * (j + 1)] - want)))
        assert err <= 1e-3 * float(np.max(np.abs(want))) + 1e-5, (j, err)
