"""The drop-in, proven through the reference's own engine.

oracle/_ref/libigl_ref_dropin.so is the reference engine (app_core.c, SSE2
float tier, built by oracle/Makefile) with the six entries of its backend
table (`back_desk`, app_core.c:5223-5245) forwarded to this backend's
`igl_desk`: the reference loads the checkpoint with its own model_load, opens
its own session and runs its own prime and steps; every projection, norm,
softmax, gated GELU and rotation it asks the table for runs on the GPU.

Bar: the 128-id greedy stream equals the reference's all-CPU stream on the
same checkpoint (tests/golden/e2e_small.json), with each step's top-1/top-2 gap
within 2e-3 of the reference's.  With several pool threads, the reference
calls soft_max from every worker at once (attend_blend_band); the run with 4
threads checks that the backend's table entries serialize those calls.
"""
import ctypes
import json
import os
import tempfile

import numpy as np
import pytest

import oracle_lib
from igllm_amd.engine import SMALL, prompt_ids, write_gemma

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
ENTRIES = ("mat_vec", "mat_mat", "norm_rms", "soft_max", "gelu_gate", "rope_turn")


@pytest.fixture(scope="module")
def dropin():
    if not os.path.exists(oracle_lib.REF_DROPIN_PATH):
        pytest.skip("oracle/_ref/libigl_ref_dropin.so was not built (reference source absent)")
    lib = ctypes.CDLL(oracle_lib.REF_DROPIN_PATH)
    fn = lib.dropin_engine_greedy
    fn.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                   ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                   ctypes.c_void_p]
    fn.restype = ctypes.c_int
    return fn


@pytest.mark.parametrize("threads", [1, 4])
def test_reference_engine_on_the_gpu_table(dropin, threads):
    with open(os.path.join(HERE, "golden", "e2e_small.json")) as f:
        fx = json.load(f)
    folder = os.path.join(tempfile.gettempdir(), f"igl_gemma_dropin_{os.getpid()}")
    write_gemma(folder, seed=fx["seed"], **SMALL)
    prompt = prompt_ids(fx["prompt_count"], fx["shape"]["vocab"], seed=fx["prompt_seed"])
    ids = np.zeros(fx["gen"], np.int32)
    margins = np.zeros(fx["gen"], np.float32)
    calls = np.zeros(7, np.int64)
    code = dropin(folder.encode(), 0, threads, fx["cache_bits"], fx["window_limit"], prompt.ctypes.data,
                  prompt.size, fx["gen"], ids.ctypes.data, margins.ctypes.data, calls.ctypes.data)
    print("entry calls", dict(zip(ENTRIES, calls[:6].tolist())), "unattached products", int(calls[6]))
    assert code == 0, code
    assert calls[6] == 0
    # every entry the text stack uses reached the backend
    for name in ("mat_mat", "norm_rms", "soft_max", "gelu_gate", "rope_turn"):
        assert calls[ENTRIES.index(name)] > 0, name
    want = np.array(fx["plain"]["ids"], dtype=np.int32)
    ref_margin = np.array(fx["plain"]["margin"])
    if not np.array_equal(ids, want):
        first = int(np.nonzero(ids != want)[0][0])
        print("first divergence at step", first, "reference margin there", ref_margin[first])
    assert np.array_equal(ids, want)
    gap = float(np.max(np.abs(margins - ref_margin)))
    print("max gap difference", gap)
    assert gap <= 2e-3
