"""GPU parity of the backend table's elementwise entries (norm_rms, soft_max,
gelu_gate, rope_turn) through the table itself, against the oracle.
Bar: 1e-5 relative to the vector's scale (1e-6 for softmax probabilities)."""
import numpy as np
import pytest

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
