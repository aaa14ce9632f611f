#!/usr/bin/env python3
"""Writes the greedy-stream fixtures the end-to-end parity tests hold the GPU
engine to: the reference engine itself (app_core.c, compiled into oracle/_ref
by oracle/Makefile), run on this repository's seeded synthetic checkpoint.

    python tests/golden/make_e2e_golden.py small   # 10 layers, vocab 4096
    python tests/golden/make_e2e_golden.py e2b     # config.json dimensions

For each, the checkpoint is written with igl_gemma_write (seed 0) into a
scratch folder, the prompt is drawn by igllm_amd.engine.prompt_ids, and the
reference's plain (SSE2) and tuned (AVX2+FMA) float builds each prime it and
take `gen` greedy steps with an FP8 key/value cache (--cache 8).  The fixture
keeps the prompt seed, both streams and every step's top-1/top-2 margin.
"""
import ctypes
import json
import os
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

from igllm_amd.engine import SMALL, prompt_ids, write_gemma  # noqa: E402
import oracle_lib  # noqa: E402

CASES = {
    "small": dict(shape=SMALL, prompt=600, gen=128, window=1024),
    "e2b": dict(shape={}, prompt=2048, gen=256, window=2560),
}


def ref_stream(kind, folder, prompt, gen, window, threads):
    lib = ctypes.CDLL(oracle_lib.REF_PLAIN_PATH if kind == "plain" else oracle_lib.REF_TUNED_PATH)
    fn = lib.ref_engine_greedy
    fn.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                   ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    out = np.zeros(gen, np.int32)
    margin = np.zeros(gen, np.float32)
    t0 = time.time()
    code = fn(folder.encode(), threads, 8, window, prompt.ctypes.data, prompt.size, gen,
              out.ctypes.data, margin.ctypes.data)
    if code != 0:
        raise SystemExit(f"ref_engine_greedy({kind}) returned {code}")
    return out, margin, time.time() - t0


def main():
    name = sys.argv[1] if len(sys.argv) > 1 else "small"
    case = CASES[name]
    threads = int(os.environ.get("IGL_THREADS", os.cpu_count() or 4))
    folder = os.path.join(tempfile.gettempdir(), f"igl_gemma_{name}")
    shape = write_gemma(folder, seed=0, **case["shape"])
    prompt = prompt_ids(case["prompt"], shape.vocab, seed=0)
    result = {"case": name, "seed": 0, "prompt_seed": 0, "prompt_count": case["prompt"],
              "gen": case["gen"], "window_limit": case["window"], "cache_bits": 8,
              "shape": {k: getattr(shape, k) for k, _ in shape._fields_}}
    for kind in ("plain", "tuned"):
        ids, margin, secs = ref_stream(kind, folder, prompt, case["gen"], case["window"], threads)
        result[kind] = {"ids": ids.tolist(), "margin": [float(m) for m in margin], "seconds": secs,
                        "threads": threads}
        print(kind, f"{secs:.1f}s", "min margin", float(margin.min()), flush=True)
    result["streams_agree"] = result["plain"]["ids"] == result["tuned"]["ids"]
    with open(os.path.join(HERE, f"e2e_{name}.json"), "w") as f:
        json.dump(result, f, indent=1)
    print("agree", result["streams_agree"])


if __name__ == "__main__":
    main()
