"""CPU-side checks of the C ABI: the library loads, exports everything
include/igl_backend.h declares, refuses to open without a device, and its
synthetic generator is the published splitmix64 / xoshiro256** pair."""
import ctypes
import math
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "igl_backend.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set(re.findall(r"\b(igl_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    from igllm_amd import native

    lib = native.load()
    names = declared_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(native.SIGNATURES), set(names) ^ set(native.SIGNATURES)


def test_library_has_no_oracle_dependency():
    """The product must not link or name the checker."""
    lib_path = os.path.join(ROOT, "igllm_amd", "libigl_hip.so")
    blob = open(lib_path, "rb").read()
    assert b"oracle" not in blob and b"liboracle" not in blob and b"ref_harness" not in blob


def test_open_without_device_fails_cleanly():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from igllm_amd import native

    lib = native.load()
    desk = native.Desk()
    code = lib.igl_back_open(ctypes.byref(desk), 0, 64, 2048, 16)
    assert code == native.IGL_FAIL_DEVICE
    assert lib.igl_code_text(code) == b"device error"


def splitmix_stream(seed, count):
    x, out = seed, []
    for _ in range(count):
        x = (x + 0x9E3779B97F4A7C15) & (2 ** 64 - 1)
        z = x
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & (2 ** 64 - 1)
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & (2 ** 64 - 1)
        out.append(z ^ (z >> 31))
    return out


def xoshiro(state, count):
    s = list(state)
    mask = 2 ** 64 - 1
    rotl = lambda x, k: ((x << k) | (x >> (64 - k))) & mask  # noqa: E731
    out = []
    for _ in range(count):
        out.append(rotl((s[1] * 5) & mask, 7) * 9 & mask)
        t = (s[1] << 17) & mask
        s[2] ^= s[0]; s[3] ^= s[1]; s[1] ^= s[2]; s[0] ^= s[3]
        s[2] ^= t
        s[3] = rotl(s[3], 45)
    return out


def test_splitmix64_published_vector():
    # Vigna's splitmix64 from state 0.
    assert splitmix_stream(0, 3) == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_generator_matches_restatement():
    from igllm_amd import native
    from igllm_amd.backend import Synth

    s = Synth(0)
    assert list(s.rng.s) == splitmix_stream(0, 4)
    want = xoshiro(splitmix_stream(0, 4), 1000)
    assert [s.next() for _ in range(1000)] == want


def test_normals_and_codes():
    from igllm_amd.backend import Synth

    s = Synth(42)
    state = list(s.rng.s)
    z = s.normal(5)
    raw = xoshiro(state, 6)
    u = [((raw[2 * i] >> 11) + 1) * 2.0 ** -53 for i in range(3)]
    v = [(raw[2 * i + 1] >> 11) * 2.0 ** -53 for i in range(3)]
    want = []
    for a, b in zip(u, v):
        r = math.sqrt(-2 * math.log(a))
        want += [r * math.cos(2 * math.pi * b), r * math.sin(2 * math.pi * b)]
    assert np.allclose(z, np.float32(want[:5]), rtol=0, atol=1e-6)

    c = Synth(0).codes4(64, 2048)
    nib = np.stack([c & 15, c >> 4], axis=-1).ravel()
    counts = np.bincount(nib, minlength=16)
    assert counts.min() > 0.9 * nib.size / 16 and counts.max() < 1.1 * nib.size / 16
    first = xoshiro(splitmix_stream(0, 4), 2)
    assert c[0, 0] == ((first[0] >> 60) | ((first[1] >> 60) << 4))
