"""The drop-in, proven through the reference's own engine.

oracle/_ref/libigl_ref_dropin.so is the reference engine (app_core.c, SSE2
float tier, built by oracle/Makefile) with the six entries of its backend
table (`back_desk`, app_core.c:5223-5245) forwarded to this backend's
`igl_desk`: the reference loads the checkpoint with its own model_load, opens
its own session and runs its own prime and steps; every projection, norm,
softmax, gated GELU and rotation it asks the table for runs on the GPU.

Bars:
  * greedy: the 128-id stream equals the reference's all-CPU stream on the
    same checkpoint (tests/golden/e2e_small.json), each step's top-1/top-2 gap
    within 2e-3 of the reference's.  With several pool threads the reference
    calls soft_max from every worker at once (attend_blend_band); the run with
    4 threads checks that the backend's table entries serialize those calls;
  * the CLI's --guess 4 loop (main_answer_guess, app_main.c:520-598): the
    reference's scout, session_guess blocks of up to four lanes through the
    table's mat_mat, session_guess_keep: its stream and its round, drawn and
    taken counts equal the all-CPU run's (tests/golden/e2e_small_guess.json);
  * config.json dimensions (35 layers, the 262144-row head): the 2048-id
    prime and the first 32 greedy steps against the reference's stream
    (tests/golden/e2e_e2b.json), gaps within 2e-3.
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
def dropin_lib():
    if not os.path.exists(oracle_lib.REF_DROPIN_PATH):
        pytest.skip("oracle/_ref/libigl_ref_dropin.so was not built (reference source absent)")
    lib = ctypes.CDLL(oracle_lib.REF_DROPIN_PATH)
    lib.dropin_engine_greedy.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                         ctypes.c_void_p, ctypes.c_void_p]
    lib.dropin_engine_greedy.restype = ctypes.c_int
    lib.dropin_engine_guess.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.dropin_engine_guess.restype = ctypes.c_int
    return lib


@pytest.fixture(scope="module")
def dropin(dropin_lib):
    return dropin_lib.dropin_engine_greedy


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


def test_reference_guess_loop_on_the_gpu_table(dropin_lib):
    with open(os.path.join(HERE, "golden", "e2e_small_guess.json")) as f:
        fx = json.load(f)
    folder = os.path.join(tempfile.gettempdir(), f"igl_gemma_dropin_guess_{os.getpid()}")
    write_gemma(folder, seed=fx["seed"], **SMALL)
    prompt = prompt_ids(fx["prompt_count"], fx["shape"]["vocab"], seed=fx["prompt_seed"],
                        repeat_span=fx["repeat_span"])
    ids = np.zeros(fx["gen"], np.int32)
    stats = np.zeros(3, np.int64)
    calls = np.zeros(7, np.int64)
    code = dropin_lib.dropin_engine_guess(folder.encode(), 0, 4, fx["cache_bits"], fx["window_limit"],
                                          prompt.ctypes.data, prompt.size, fx["gen"], fx["guess_span"],
                                          ids.ctypes.data, stats.ctypes.data, calls.ctypes.data)
    print("entry calls", dict(zip(ENTRIES, calls[:6].tolist())), "rounds, drawn, taken", stats.tolist())
    assert code == 0, code
    assert calls[6] == 0
    assert np.array_equal(ids, np.array(fx["plain"]["ids"], dtype=np.int32))
    assert stats.tolist() == [fx["plain"]["rounds"], fx["plain"]["drawn"], fx["plain"]["taken"]]


def test_reference_engine_e2b_on_the_gpu_table(dropin):
    with open(os.path.join(HERE, "golden", "e2e_e2b.json")) as f:
        fx = json.load(f)
    gen = 32
    root = "/dev/shm" if os.path.isdir("/dev/shm") else tempfile.gettempdir()
    folder = os.path.join(root, f"igl_gemma_dropin_e2b_{os.getpid()}")
    write_gemma(folder, seed=fx["seed"])
    try:
        prompt = prompt_ids(fx["prompt_count"], fx["shape"]["vocab"], seed=fx["prompt_seed"])
        ids = np.zeros(gen, np.int32)
        margins = np.zeros(gen, np.float32)
        calls = np.zeros(7, np.int64)
        code = dropin(folder.encode(), 0, 16, fx["cache_bits"], fx["window_limit"], prompt.ctypes.data,
                      prompt.size, gen, ids.ctypes.data, margins.ctypes.data, calls.ctypes.data)
    finally:
        import shutil
        shutil.rmtree(folder, ignore_errors=True)
    print("entry calls", dict(zip(ENTRIES, calls[:6].tolist())), "unattached products", int(calls[6]))
    assert code == 0, code
    assert calls[6] == 0
    assert np.array_equal(ids, np.array(fx["plain"]["ids"][:gen], dtype=np.int32))
    gap = float(np.max(np.abs(margins - np.array(fx["plain"]["margin"][:gen]))))
    print("max gap difference", gap)
    assert gap <= 2e-3


def test_reference_engine_packed_on_the_gpu_table(dropin):
    """The compressed-tensors pack through the reference's own loader: its
    plane_bind_part unpacks weight_zero_point into bias_data (zero_read), the
    shim copies the plane field for field, and the zero-point products run on
    the GPU (tests/golden/e2e_small_packed.json)."""
    with open(os.path.join(HERE, "golden", "e2e_small_packed.json")) as f:
        fx = json.load(f)
    folder = os.path.join(tempfile.gettempdir(), f"igl_gemma_dropin_packed_{os.getpid()}")
    write_gemma(folder, seed=fx["seed"], **dict(SMALL, kinds=2))
    prompt = prompt_ids(fx["prompt_count"], fx["shape"]["vocab"], seed=fx["prompt_seed"])
    ids = np.zeros(fx["gen"], np.int32)
    margins = np.zeros(fx["gen"], np.float32)
    calls = np.zeros(7, np.int64)
    code = dropin(folder.encode(), 0, 4, fx["cache_bits"], fx["window_limit"], prompt.ctypes.data,
                  prompt.size, fx["gen"], ids.ctypes.data, margins.ctypes.data, calls.ctypes.data)
    print("entry calls", dict(zip(ENTRIES, calls[:6].tolist())), "unattached products", int(calls[6]))
    assert code == 0, code
    assert calls[6] == 0
    assert np.array_equal(ids, np.array(fx["plain"]["ids"], dtype=np.int32))
    gap = float(np.max(np.abs(margins - np.array(fx["plain"]["margin"]))))
    print("max gap difference", gap)
    assert gap <= 2e-3
