#!/usr/bin/env python3
"""Writes the greedy-stream fixtures the end-to-end parity tests hold the GPU
engine to: the reference engine itself (app_core.c, compiled into oracle/_ref
by oracle/Makefile), run on this repository's seeded synthetic checkpoint.

    python tests/golden/make_e2e_golden.py small   # 10 layers, vocab 4096
    python tests/golden/make_e2e_golden.py e2b     # config.json dimensions
    python tests/golden/make_e2e_golden.py small_guess   # --guess 4, repeating prompt
    python tests/golden/make_e2e_golden.py small_long    # 8300-id prompt, 12000-position window
    python tests/golden/make_e2e_golden.py small_kinds   # the export's plane kinds, 20 layers
    python tests/golden/make_e2e_golden.py e2b_logits    # config.json dimensions, whole logit rows
    python tests/golden/make_e2e_golden.py small_packed  # I32-packed planes with zero points
    python tests/golden/make_e2e_golden.py e2b_blocks    # config.json dimensions, fixed guess blocks

For each, the checkpoint is written with igl_gemma_write (seed 0) into a
scratch folder, the prompt is drawn by igllm_amd.engine.prompt_ids, and the
reference's plain (SSE2) and tuned (AVX2+FMA) float builds each prime it and
take `gen` greedy steps with an FP8 key/value cache (--cache 8).  The fixture
keeps the prompt seed, both streams and every step's top-1/top-2 margin.  For
the export's kinds (calibrated planes) the level build (AVX-512 VNNI, where
this host has it) is run too: its products take the integer grid.
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
    # --guess 4 on a prompt that repeats its first `repeat` ids
    "small_guess": dict(shape=SMALL, prompt=600, gen=128, window=1024, repeat=128, span=4),
    # a prompt past 8192 positions in a 12000-position window: prime batches
    # whose spans cross the attention's change of chunk length
    "small_long": dict(shape=SMALL, prompt=8300, gen=32, window=12000),
    "e2b_guess": dict(shape={}, prompt=2048, gen=256, window=2560, repeat=512, span=4),
    # config.json dimensions: the logits of whole rows at a few steps (the
    # greedy pick settles on one id; the 262144-wide rows do not)
    "e2b_logits": dict(shape={}, prompt=2048, gen=32, window=2560, probes=[0, 1, 2, 15, 31],
                       sample=512, top=64),
    # 2-bit MLPs from layer 15, I8 per-layer planes, bf16 per_layer_model_projection,
    # one scale a row, every projection but the head calibrated
    "small_kinds": dict(shape=dict(vocab=4096, hidden=512, inner=1024, layers=20, shared_layers=8, kinds=1),
                        prompt=600, gen=128, window=1024),
    # the compressed-tensors pack: weight_packed I32 + weight_shape + weight_zero_point
    # on every layer projection (4-bit, 2-bit MLPs from the middle layer, 8-bit
    # per-layer planes), zero points on all of them
    "small_packed": dict(shape=dict(SMALL, kinds=2), prompt=600, gen=128, window=1024, seed=1),
    # config.json dimensions: fixed speculative blocks of 1-5 lanes of random
    # ids (seed 2) after the prompt, each kept in part; every lane's pick and
    # gap (the greedy stream there is one id; these walk many inputs)
    "e2b_blocks": dict(shape={}, prompt=2048, gen=0, window=2560,
                       counts=[2, 3, 5, 4, 2, 5, 1, 3, 4, 2, 5, 3], keeps=[1, 2, 5, 1, 2, 3, 1, 3, 2, 1, 4, 3]),
}

PATHS = {"plain": oracle_lib.REF_PLAIN_PATH, "tuned": oracle_lib.REF_TUNED_PATH,
         "level": oracle_lib.REF_LEVEL_PATH}


def ref_stream(kind, folder, prompt, gen, window, threads):
    lib = ctypes.CDLL(PATHS[kind])
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


def ref_forced(kind, folder, prompt, forced, window, threads):
    """Each step's pick and margin with the inputs `forced` (after the prompt's
    last id) instead of the picks."""
    lib = ctypes.CDLL(PATHS[kind])
    fn = lib.ref_engine_forced
    fn.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                   ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    out = np.zeros(forced.size, np.int32)
    margin = np.zeros(forced.size, np.float32)
    code = fn(folder.encode(), threads, 8, window, prompt.ctypes.data, prompt.size, forced.ctypes.data,
              forced.size, out.ctypes.data, margin.ctypes.data)
    if code != 0:
        raise SystemExit(f"ref_engine_forced({kind}) returned {code}")
    return out, margin


def ref_probe(kind, folder, prompt, gen, window, threads, probes, vocab):
    """The greedy run's whole logit rows at the steps `probes`."""
    lib = ctypes.CDLL(PATHS[kind])
    fn = lib.ref_engine_probe
    fn.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                   ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                   ctypes.c_void_p]
    steps = np.array(probes, dtype=np.int32)
    ids = np.zeros(gen, np.int32)
    rows = np.zeros((len(probes), vocab), np.float32)
    t0 = time.time()
    code = fn(folder.encode(), threads, 8, window, prompt.ctypes.data, prompt.size, gen, steps.ctypes.data,
              steps.size, ids.ctypes.data, rows.ctypes.data)
    if code != 0:
        raise SystemExit(f"ref_engine_probe({kind}) returned {code}")
    return ids, rows, time.time() - t0


def ref_guess(kind, folder, prompt, gen, window, threads, span):
    lib = ctypes.CDLL(oracle_lib.REF_PLAIN_PATH if kind == "plain" else oracle_lib.REF_TUNED_PATH)
    fn = lib.ref_engine_guess
    fn.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                   ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    out = np.zeros(gen, np.int32)
    stats = np.zeros(3, np.int64)
    t0 = time.time()
    code = fn(folder.encode(), threads, 8, window, prompt.ctypes.data, prompt.size, gen, span,
              out.ctypes.data, stats.ctypes.data)
    if code != 0:
        raise SystemExit(f"ref_engine_guess({kind}) returned {code}")
    return out, stats, time.time() - t0


def ref_blocks(kind, folder, prompt, ids, counts, keeps, window, threads):
    lib = ctypes.CDLL(PATHS[kind])
    fn = lib.ref_engine_blocks
    fn.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                   ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                   ctypes.c_void_p]
    c = np.array(counts, np.int32)
    k = np.array(keeps, np.int32)
    picks = np.zeros(ids.size, np.int32)
    margin = np.zeros(ids.size, np.float32)
    t0 = time.time()
    code = fn(folder.encode(), threads, 8, window, prompt.ctypes.data, prompt.size, ids.ctypes.data, c.ctypes.data,
              k.ctypes.data, c.size, picks.ctypes.data, margin.ctypes.data)
    if code != 0:
        raise SystemExit(f"ref_engine_blocks({kind}) returned {code}")
    return picks, margin, time.time() - t0


def main():
    name = sys.argv[1] if len(sys.argv) > 1 else "small"
    case = CASES[name]
    threads = int(os.environ.get("IGL_THREADS", os.cpu_count() or 4))
    folder = os.path.join(tempfile.gettempdir(), f"igl_gemma_{name}")
    shape = write_gemma(folder, seed=case.get("seed", 0), **case["shape"])
    prompt = prompt_ids(case["prompt"], shape.vocab, seed=0, repeat_span=case.get("repeat", 0))
    result = {"case": name, "seed": case.get("seed", 0), "prompt_seed": 0, "prompt_count": case["prompt"],
              "gen": case["gen"], "window_limit": case["window"], "cache_bits": 8,
              "repeat_span": case.get("repeat", 0), "guess_span": case.get("span", 0),
              "shape": {k: getattr(shape, k) for k, _ in shape._fields_}}
    if case.get("counts"):
        counts, keeps = case["counts"], case["keeps"]
        ids = prompt_ids(sum(counts), shape.vocab, seed=2)
        result.update({"block_seed": 2, "counts": counts, "keeps": keeps, "block_ids": ids.tolist()})
        for kind in ("plain", "tuned"):
            picks, margin, secs = ref_blocks(kind, folder, prompt, ids, counts, keeps, case["window"], threads)
            result[kind] = {"picks": picks.tolist(), "margin": [float(m) for m in margin], "seconds": secs}
            print(kind, f"{secs:.1f}s", "distinct picks", len(set(picks.tolist())), "min margin",
                  float(margin.min()), flush=True)
        result["builds_max_margin_diff"] = float(np.max(np.abs(np.array(result["plain"]["margin"]) -
                                                              np.array(result["tuned"]["margin"]))))
        result["picks_agree"] = result["plain"]["picks"] == result["tuned"]["picks"]
        with open(os.path.join(HERE, f"e2e_{name}.json"), "w") as f:
            json.dump(result, f, indent=1)
        print("picks agree", result["picks_agree"], "builds' margin spread", result["builds_max_margin_diff"])
        return
    if case.get("probes"):
        probes = case["probes"]
        out = {}
        for kind in ("plain", "tuned"):
            ids, rows, secs = ref_probe(kind, folder, prompt, case["gen"], case["window"], threads, probes,
                                        shape.vocab)
            out[kind] = (ids, rows)
            print(kind, f"{secs:.1f}s", flush=True)
        plain_rows, tuned_rows = out["plain"][1], out["tuned"][1]
        sample = np.random.default_rng(7).choice(shape.vocab, size=case["sample"], replace=False)
        result["probes"] = []
        for i, step in enumerate(probes):
            top = np.argsort(-plain_rows[i], kind="stable")[:case["top"]]
            ids = np.concatenate([top, sample[~np.isin(sample, top)]]).astype(np.int64)
            result["probes"].append({
                "step": step, "ids": ids.tolist(),
                "plain": [float(x) for x in plain_rows[i][ids]],
                "tuned": [float(x) for x in tuned_rows[i][ids]],
                "plain_row_mean": float(plain_rows[i].astype(np.float64).mean()),
                "plain_row_rms": float(np.sqrt((plain_rows[i].astype(np.float64) ** 2).mean())),
                "builds_max_abs_diff": float(np.max(np.abs(plain_rows[i] - tuned_rows[i])))})
            print("step", step, "plain/tuned max |diff| over the row", result["probes"][-1]["builds_max_abs_diff"],
                  "row rms", result["probes"][-1]["plain_row_rms"], flush=True)
        result["plain"] = {"ids": out["plain"][0].tolist()}
        result["tuned"] = {"ids": out["tuned"][0].tolist()}
        with open(os.path.join(HERE, f"e2e_{name}.json"), "w") as f:
            json.dump(result, f, indent=1)
        return
    if case.get("span"):
        for kind in ("plain", "tuned"):
            ids, stats, secs = ref_guess(kind, folder, prompt, case["gen"], case["window"], threads,
                                         case["span"])
            result[kind] = {"ids": ids.tolist(), "rounds": int(stats[0]), "drawn": int(stats[1]),
                            "taken": int(stats[2]), "seconds": secs, "threads": threads}
            print(kind, f"{secs:.1f}s", "rounds", int(stats[0]), "drawn", int(stats[1]),
                  "taken", int(stats[2]), flush=True)
        # the same prompt without guessing: the streams must agree
        ids, margin, secs = ref_stream("plain", folder, prompt, case["gen"], case["window"], threads)
        result["greedy"] = {"ids": ids.tolist(), "margin": [float(m) for m in margin], "seconds": secs}
        result["streams_agree"] = result["plain"]["ids"] == result["tuned"]["ids"]
        result["guess_equals_greedy"] = result["plain"]["ids"] == result["greedy"]["ids"]
        with open(os.path.join(HERE, f"e2e_{name}.json"), "w") as f:
            json.dump(result, f, indent=1)
        print("agree", result["streams_agree"], "guess == greedy", result["guess_equals_greedy"])
        return
    kinds = ("plain", "tuned")
    if case["shape"].get("kinds") == 1 and oracle_lib.ref("level") is not None:
        kinds += ("level",)
    for kind in kinds:
        ids, margin, secs = ref_stream(kind, folder, prompt, case["gen"], case["window"], threads)
        result[kind] = {"ids": ids.tolist(), "margin": [float(m) for m in margin], "seconds": secs,
                        "threads": threads}
        print(kind, f"{secs:.1f}s", "min margin", float(margin.min()), flush=True)
    result["streams_agree"] = result["plain"]["ids"] == result["tuned"]["ids"]
    if case["shape"].get("kinds"):
        # a random model settles on one id; forced inputs (seed 1) walk many
        forced = prompt_ids(case["gen"], shape.vocab, seed=1)
        result["forced_seed"] = 1
        for kind in kinds:
            ids, margin = ref_forced(kind, folder, prompt, forced, case["window"], threads)
            result[kind]["forced_ids"] = ids.tolist()
            result[kind]["forced_margin"] = [float(m) for m in margin]
            print(kind, "forced: distinct picks", len(set(ids.tolist())), "min margin", float(margin.min()),
                  flush=True)
    if "level" in result:
        a, b = np.array(result["plain"]["ids"]), np.array(result["level"]["ids"])
        result["plain_level_first_difference"] = int(np.argmax(a != b)) if np.any(a != b) else None
    with open(os.path.join(HERE, f"e2e_{name}.json"), "w") as f:
        json.dump(result, f, indent=1)
    print("agree", result["streams_agree"], "plain/level first difference",
          result.get("plain_level_first_difference"))


if __name__ == "__main__":
    main()
