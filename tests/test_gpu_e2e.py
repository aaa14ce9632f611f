"""End-to-end greedy parity: the device-resident engine against the reference
engine's own greedy stream on the same seeded synthetic checkpoint
(tests/golden/e2e_small.json, written by tests/golden/make_e2e_golden.py from
the reference compiled out of app_core.c).

Bar: the greedy token stream is identical over the fixture's 128 tokens.  The
fixture records each step's top-1/top-2 margin in the reference; the smallest
is printed, since a tie closer than fp32 reassociation could flip a pick.
"""
import json
import os
import tempfile

import numpy as np
import pytest

from igllm_amd.engine import SMALL, Engine, prompt_ids, write_gemma

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def load_fixture(name):
    with open(os.path.join(HERE, "golden", f"e2e_{name}.json")) as f:
        return json.load(f)


@pytest.fixture(scope="module")
def small_model():
    fx = load_fixture("small")
    folder = os.path.join(tempfile.gettempdir(), f"igl_gemma_small_{os.getpid()}")
    write_gemma(folder, seed=fx["seed"], **SMALL)
    return folder, fx


@pytest.mark.parametrize("lane_limit", [16, 64])
def test_small_greedy_stream_matches_reference(backend, small_model, lane_limit):
    folder, fx = small_model
    prompt = prompt_ids(fx["prompt_count"], fx["shape"]["vocab"], seed=fx["prompt_seed"])
    eng = Engine(backend, folder, window_limit=fx["window_limit"], lane_limit=lane_limit, precise=True)
    try:
        ids, margins = eng.greedy(prompt, fx["gen"])
    finally:
        eng.close()
    want = np.array(fx["plain"]["ids"], dtype=np.int32)
    ref_margin = np.array(fx["plain"]["margin"])
    print("min reference margin", float(ref_margin.min()), "min engine margin", float(margins.min()))
    if not np.array_equal(ids, want):
        first = int(np.nonzero(ids != want)[0][0])
        print("first divergence at step", first, "reference margin there", ref_margin[first])
    assert np.array_equal(ids, want)
    # the top-1/top-2 gaps agree too (logits within fp32 reassociation)
    assert np.max(np.abs(margins - ref_margin)) <= 2e-3


@pytest.fixture(scope="module")
def e2b_model():
    """The config.json-dimension checkpoint (35 layers, 262144-id head, 2.6 GB),
    written once for the module."""
    import shutil

    fx = load_fixture("e2b")
    root = "/dev/shm" if os.path.isdir("/dev/shm") else tempfile.gettempdir()
    folder = os.path.join(root, f"igl_gemma_e2b_test_{os.getpid()}")
    write_gemma(folder, seed=fx["seed"])
    yield folder
    shutil.rmtree(folder, ignore_errors=True)


# (precise, lane_limit): the reference's 16-lane batches on the fp32 GEMV, and
# the fast prefill at 256 lanes a pass and at 2048 (the whole prompt in one
# pass, as the benchmark runs it)
E2B_MODES = [(True, 16), (False, 256), (False, 2048)]


@pytest.mark.parametrize("precise,lane_limit", E2B_MODES)
def test_e2b_greedy_stream_matches_reference(backend, e2b_model, precise, lane_limit):
    """Full config.json dimensions (35 layers, 262144-id head), 2048-id prompt,
    256 greedy steps, against the reference engine's stream
    (tests/golden/e2e_e2b.json, 560 s on the host).  The synthetic model's
    stream settles on one id, so the per-step top-1/top-2 gaps are compared as
    well: they carry the whole pass's arithmetic."""
    fx = load_fixture("e2b")
    prompt = prompt_ids(fx["prompt_count"], fx["shape"]["vocab"], seed=fx["prompt_seed"])
    eng = Engine(backend, e2b_model, window_limit=fx["window_limit"], lane_limit=lane_limit, precise=precise)
    try:
        ids, margins = eng.greedy(prompt, fx["gen"])
    finally:
        eng.close()
    want = np.array(fx["plain"]["ids"], dtype=np.int32)
    ref_margin = np.array(fx["plain"]["margin"])
    gap = float(np.max(np.abs(margins - ref_margin)))
    print("precise", precise, "lanes", lane_limit, "max margin difference", gap)
    assert np.array_equal(ids, want)
    assert gap <= 2e-3


@pytest.mark.parametrize("precise,lane_limit", [(True, 16), (False, 2048)])
def test_e2b_logit_rows_match_reference(backend, e2b_model, precise, lane_limit):
    """The whole pass at config.json dimensions, beyond the pick: the greedy
    stream of this checkpoint settles on one id, but its 262144-wide rows of
    logits do not.  At five steps after the 2048-id prompt the engine's row is
    compared with the reference's plain build (tests/golden/e2e_e2b_logits.json)
    at the row's top 64 ids and 512 seeded ones, and by the whole row's mean
    and rms.  The bar is set by the reference itself: three times the largest
    difference between its plain and tuned (AVX2+FMA) builds over the row, and
    at least 1e-3, for the fp32 GEMV prime and the MFMA GEMM prime alike."""
    fx = load_fixture("e2b_logits")
    prompt = prompt_ids(fx["prompt_count"], fx["shape"]["vocab"], seed=fx["prompt_seed"])
    want_ids = np.array(fx["plain"]["ids"], dtype=np.int32)
    probes = {p["step"]: p for p in fx["probes"]}
    eng = Engine(backend, e2b_model, window_limit=fx["window_limit"], lane_limit=lane_limit, precise=precise)
    worst = {}
    try:
        eng.prime(prompt)
        token = int(prompt[-1])
        for step in range(fx["gen"]):
            pick, _ = eng.step(token)
            assert pick == want_ids[step]
            if step in probes:
                p = probes[step]
                row = eng.logits(0)
                ids = np.array(p["ids"])
                diff = float(np.max(np.abs(row[ids] - np.array(p["plain"]))))
                bar = max(3 * p["builds_max_abs_diff"], 1e-3)
                row64 = row.astype(np.float64)
                mean_gap = abs(float(row64.mean()) - p["plain_row_mean"])
                rms_gap = abs(float(np.sqrt((row64 ** 2).mean())) - p["plain_row_rms"])
                worst[step] = (diff, bar, mean_gap, rms_gap)
                assert diff <= bar, (step, diff, bar)
                assert mean_gap <= bar and rms_gap <= bar, (step, mean_gap, rms_gap, bar)
            token = int(want_ids[step])
    finally:
        eng.close()
        print("step: (max |logit diff| at the sampled ids, bar, row mean gap, row rms gap)", worst)


@pytest.mark.parametrize("precise,lane_limit", [(True, 16), (False, 2048)])
def test_e2b_guess_stream_matches_reference(backend, e2b_model, precise, lane_limit):
    """--guess 4 at config.json dimensions on a 2048-id prompt that repeats its
    first 512 ids (tests/golden/e2e_e2b_guess.json: the reference's
    session_guess, app_core.c:12139-12223, under the CLI's loop,
    app_main.c:520-598): the engine's blocks give the reference's stream and
    its round, proposed and kept counts; every committed id's top-1/top-2 gap
    is the reference greedy run's gap for that id."""
    from igllm_amd.engine import Scout, guess_loop

    fx = load_fixture("e2b_guess")
    prompt = prompt_ids(fx["prompt_count"], fx["shape"]["vocab"], seed=fx["prompt_seed"],
                        repeat_span=fx["repeat_span"])
    eng = Engine(backend, e2b_model, window_limit=fx["window_limit"], lane_limit=lane_limit, precise=precise)
    gaps, held = [], {}
    try:
        eng.prime(prompt)

        def step(token):
            pick, gap = eng.step(token)
            gaps.append(gap)
            return pick

        def guess(block):
            picks, held["gaps"] = eng.guess(block)
            return picks

        def keep(count):
            gaps.extend(float(x) for x in held.pop("gaps")[:count])
            eng.keep(count)

        ids, counts = guess_loop(Scout(eng.lib), prompt, fx["gen"], fx["guess_span"], step, guess, keep)
        fill = eng.fill
    finally:
        eng.close()
    want = np.array(fx["plain"]["ids"], dtype=np.int32)
    print("counts", counts, "reference", (fx["plain"]["rounds"], fx["plain"]["drawn"], fx["plain"]["taken"]))
    assert np.array_equal(ids, want)
    assert counts == (fx["plain"]["rounds"], fx["plain"]["drawn"], fx["plain"]["taken"])
    assert fill == fx["prompt_count"] - 1 + fx["gen"]
    gap = float(np.max(np.abs(np.array(gaps) - np.array(fx["greedy"]["margin"]))))
    print("max gap difference", gap)
    assert len(gaps) == fx["gen"] and gap <= 2e-3


@pytest.mark.parametrize("precise,lane_limit", [(True, 16), (True, 64), (False, 64), (False, 2048)])
def test_small_long_prompt_matches_reference(backend, small_model, precise, lane_limit):
    """An 8300-id prompt in a 12000-position window (tests/golden/
    e2e_small_long.json): prime batches whose spans run from under to over
    8192 positions, where the attention's chunk length changes and with it the
    count of its partials (the workspace is sized for both regimes); then 32
    greedy steps against the reference's, on the fp32 GEMV (precise) and on
    the MFMA GEMM prefill (64 and 2048 lanes a pass)."""
    folder, small = small_model
    fx = load_fixture("small_long")
    assert fx["seed"] == small["seed"] and fx["shape"]["vocab"] == small["shape"]["vocab"]
    prompt = prompt_ids(fx["prompt_count"], fx["shape"]["vocab"], seed=fx["prompt_seed"])
    eng = Engine(backend, folder, window_limit=fx["window_limit"], lane_limit=lane_limit, precise=precise)
    try:
        ids, margins = eng.greedy(prompt, fx["gen"])
    finally:
        eng.close()
    want = np.array(fx["plain"]["ids"], dtype=np.int32)
    gap = float(np.max(np.abs(margins - np.array(fx["plain"]["margin"]))))
    print("max gap difference", gap)
    assert np.array_equal(ids, want)
    assert gap <= 2e-3


@pytest.mark.parametrize("graph", [True, False])
def test_small_guess_stream_matches_reference(backend, small_model, graph):
    """--guess 4 on a prompt that repeats its first 128 ids
    (tests/golden/e2e_small_guess.json): the engine's blocks (igl_engine_guess /
    igl_engine_keep) under the product's loop give the reference's stream and
    the reference's round, proposed and kept counts; every committed id's
    top-1/top-2 gap, from a block lane or an ordinary step, is the reference
    greedy run's gap for that id."""
    from igllm_amd.engine import Scout, guess_loop

    folder, small = small_model
    fx = load_fixture("small_guess")
    assert fx["seed"] == small["seed"] and fx["shape"]["vocab"] == small["shape"]["vocab"]
    prompt = prompt_ids(fx["prompt_count"], fx["shape"]["vocab"], seed=fx["prompt_seed"],
                        repeat_span=fx["repeat_span"])
    eng = Engine(backend, folder, window_limit=fx["window_limit"], lane_limit=16, precise=True)
    gaps, held = [], {}
    try:
        eng.set_graph(graph)
        eng.prime(prompt)

        def step(token):
            pick, gap = eng.step(token)
            gaps.append(gap)
            return pick

        def guess(block):
            picks, held["gaps"] = eng.guess(block)
            return picks

        def keep(count):
            gaps.extend(float(x) for x in held.pop("gaps")[:count])
            eng.keep(count)

        ids, counts = guess_loop(Scout(eng.lib), prompt, fx["gen"], fx["guess_span"], step, guess,
                                 keep)
        fill = eng.fill
    finally:
        eng.close()
    want = np.array(fx["greedy"]["ids"], dtype=np.int32)
    print("counts", counts, "reference", (fx["plain"]["rounds"], fx["plain"]["drawn"],
                                          fx["plain"]["taken"]))
    assert np.array_equal(ids, want)
    assert counts == (fx["plain"]["rounds"], fx["plain"]["drawn"], fx["plain"]["taken"])
    # the session holds the prompt and every committed id but the last
    assert fill == fx["prompt_count"] - 1 + fx["gen"]
    gap = float(np.max(np.abs(np.array(gaps) - np.array(fx["greedy"]["margin"]))))
    print("max gap difference", gap)
    assert len(gaps) == fx["gen"] and gap <= 2e-3


@pytest.mark.parametrize("precise,lane_limit,graph", [(True, 16, True), (True, 16, False), (False, 2048, True)])
def test_e2b_fixed_blocks_match_reference(backend, e2b_model, precise, lane_limit, graph):
    """config.json dimensions, the 2048-id prompt, then twelve fixed
    speculative blocks of 1-5 lanes of random ids, each kept in part
    (tests/golden/e2e_e2b_blocks.json: the reference's session_guess /
    session_guess_keep on the same blocks).  Every lane's pick equals the
    reference's and its top-1/top-2 gap is within max(2e-3, 3 x the spread
    between the reference's two builds).  The greedy stream at this size is
    one id; these blocks run multi-lane passes (graph-replayed below the GEMM
    floor, or enqueued) over inputs it never takes."""
    fx = load_fixture("e2b_blocks")
    prompt = prompt_ids(fx["prompt_count"], fx["shape"]["vocab"], seed=fx["prompt_seed"])
    ids = np.array(fx["block_ids"], dtype=np.int32)
    eng = Engine(backend, e2b_model, window_limit=fx["window_limit"], lane_limit=lane_limit, precise=precise)
    picks, gaps = [], []
    try:
        eng.set_graph(graph)
        eng.prime(prompt)
        first = 0
        for count, keep in zip(fx["counts"], fx["keeps"]):
            p, g = eng.guess(ids[first:first + count])
            picks += p.tolist()
            gaps += g.tolist()
            eng.keep(keep)
            first += count
        fill = eng.fill
    finally:
        eng.close()
    assert fill == fx["prompt_count"] - 1 + sum(fx["keeps"])
    bar = max(2e-3, 3 * fx["builds_max_margin_diff"])
    gap = float(np.max(np.abs(np.array(gaps) - np.array(fx["plain"]["margin"]))))
    print("max gap difference", gap, "bar", bar)
    assert picks == fx["plain"]["picks"]
    assert gap <= bar


def test_guess_graphs_replay_the_enqueued_blocks(backend, small_model):
    """A block replayed from its lane count's captured graph gives the picks and
    margins the same block gives enqueued, at every position it is replayed at,
    and after the desk reallocates a workspace (a 256-lane product grows the
    GEMM's) the engine captures again instead of replaying onto freed memory.
    The graph's attention grid is sized for the window's end, so its fold may
    sum the same partials in another grouping: margins to 1e-5, picks equal."""
    from igllm_amd.backend import make_plane, synth_projection

    folder, fx = small_model
    prompt = prompt_ids(600, fx["shape"]["vocab"], seed=5)
    eng = Engine(backend, folder, window_limit=2048, lane_limit=16, precise=True)
    rng = np.random.default_rng(3)
    counts = [1, 2, 3, 5, 2, 16, 3, 1, 5, 4]
    try:
        eng.prime(prompt)
        token = int(prompt[-1])
        for rnd in range(3):
            if rnd == 2:
                # a product large enough to grow the desk's GEMM workspace
                codes, gains, _ = synth_projection(512, 512, 1, seed=9)
                cp = backend.attach(make_plane(codes, gains, 512))
                act = backend.upload(rng.normal(size=256 * 512).astype(np.float32))
                out = backend.alloc(256 * 512 * 4)
                backend.mat_mat_dev(cp, act, 512, 256, out, 512)
                backend.sync()
                act.free()
                out.free()
                backend.detach(cp)
            for c in counts:
                block = np.concatenate([[token], rng.integers(3, fx["shape"]["vocab"], size=c - 1)]).astype(np.int32)
                eng.set_graph(False)
                want_picks, want_gaps = eng.guess(block)
                eng.keep(0)
                eng.set_graph(True)
                picks, gaps = eng.guess(block)
                assert np.array_equal(picks, want_picks), (rnd, c)
                assert np.allclose(gaps, want_gaps, rtol=1e-5, atol=1e-6), (rnd, c, gaps, want_gaps)
                keep = 1 + c // 2
                eng.keep(keep)
                token = int(picks[keep - 1])
    finally:
        eng.close()


# ---- the export's plane kinds ------------------------------------------------

KINDS_SHAPE = dict(vocab=4096, hidden=512, inner=1024, layers=20, shared_layers=8, kinds=1)


@pytest.fixture(scope="module")
def kinds_model():
    fx = load_fixture("small_kinds")
    folder = os.path.join(tempfile.gettempdir(), f"igl_gemma_kinds_{os.getpid()}")
    write_gemma(folder, seed=fx["seed"], **KINDS_SHAPE)
    return folder, fx


@pytest.mark.parametrize("lane_limit,precise", [(16, True), (64, False), (2048, False)])
def test_kinds_greedy_and_forced_match_reference(backend, kinds_model, lane_limit, precise):
    """A checkpoint in the export's own kinds (2-bit MLPs from layer 15 and a
    2-bit tied head, I8 per-layer planes, bf16 per_layer_model_projection, one
    scale a row, every projection but the head calibrated), against the
    reference engine (tests/golden/e2e_small_kinds.json).  Calibrated products
    take the activation grid here, exact integer sums (the reference's level
    path); the fixture's plain (SSE2 float) and level (VNNI) streams agree.

    Greedy: the stream settles on one id, so the per-step top-1/top-2 gaps are
    compared too.  Forced inputs (seed 1, so many inputs are walked): picks and
    gaps against the plain build.  The activation grids make a quantized model
    sensitive to the last bit: a product that lands near a level's edge moves a
    whole level on a different rounding, so the reference's own builds part
    too.  The bars come from that spread, recorded in the fixture: gaps within
    1.5 times the largest gap difference between the reference's float,
    tuned and level builds, and picks equal wherever the reference's gap
    exceeds 1.5 times the largest gap at which those builds pick differently.
    """
    folder, fx = kinds_model
    prompt = prompt_ids(fx["prompt_count"], fx["shape"]["vocab"], seed=fx["prompt_seed"])
    forced = prompt_ids(fx["gen"], fx["shape"]["vocab"], seed=fx["forced_seed"])
    eng = Engine(backend, folder, window_limit=fx["window_limit"], lane_limit=lane_limit, precise=precise)
    try:
        ids, margins = eng.greedy(prompt, fx["gen"])
        eng.reset()
        eng.prime(prompt)
        picks, gaps = [], []
        token = int(prompt[-1])
        for t in forced:
            pick, gap = eng.step(token)
            picks.append(pick)
            gaps.append(gap)
            token = int(t)
    finally:
        eng.close()
    want = np.array(fx["plain"]["ids"], dtype=np.int32)
    ref_margin = np.array(fx["plain"]["margin"])
    print("greedy: max gap difference", float(np.max(np.abs(margins - ref_margin))))
    assert np.array_equal(ids, want)
    assert np.max(np.abs(margins - ref_margin)) <= 2e-2
    picks = np.array(picks)
    gaps = np.array(gaps)
    fwant = np.array(fx["plain"]["forced_ids"])
    fgap = np.array(fx["plain"]["forced_margin"])
    spread, parted = 0.0, 0.0
    for kind in ("tuned", "level"):
        if kind in fx:
            other_gap = np.array(fx[kind]["forced_margin"])
            other_ids = np.array(fx[kind]["forced_ids"])
            spread = max(spread, float(np.max(np.abs(other_gap - fgap))))
            if np.any(other_ids != fwant):
                parted = max(parted, float(np.max(fgap[other_ids != fwant])))
    decided = fgap > 1.5 * parted
    print("reference builds: gap spread", spread, "largest gap where they part", parted)
    print("forced: distinct picks", len(set(picks.tolist())), "mismatches", int((picks != fwant).sum()),
          "of which decided", int(((picks != fwant) & decided).sum()), "of", int(decided.sum()),
          "max gap difference", float(np.max(np.abs(gaps - fgap))))
    assert np.array_equal(picks[decided], fwant[decided])
    assert np.max(np.abs(gaps - fgap)) <= 1.5 * spread


@pytest.fixture(scope="module")
def packed_model():
    fx = load_fixture("small_packed")
    folder = os.path.join(tempfile.gettempdir(), f"igl_gemma_packed_{os.getpid()}")
    write_gemma(folder, seed=fx["seed"], **dict(SMALL, kinds=2))
    return folder, fx


@pytest.mark.parametrize("precise,lane_limit", [(True, 16), (False, 64), (False, 600)])
def test_packed_zero_point_stream_matches_reference(backend, packed_model, precise, lane_limit):
    """A checkpoint whose layer projections are in the compressed-tensors pack
    (plane_bind_part's packed branch, app_core.c:8015-8065): weight_packed I32
    rows, weight_shape, and weight_zero_point (zero_read, 7855-7866) on every
    one of them; 4-bit attention and early MLPs, 2-bit later MLPs, 8-bit
    per-layer planes (tests/golden/e2e_small_packed.json, the reference's
    plain and tuned builds agreeing).  The engine binds them in place and
    multiplies on the zero-point GEMV and, from 64 lanes, the GEMM.  Greedy
    stream equal with gaps within 2e-3; the forced walk (seed 1): every pick
    equal, gaps within three times the largest gap difference between the
    reference's own plain and tuned builds on it (and at least 2e-3), the bar
    the logit-row test takes."""
    folder, fx = packed_model
    prompt = prompt_ids(fx["prompt_count"], fx["shape"]["vocab"], seed=fx["prompt_seed"])
    forced = prompt_ids(fx["gen"], fx["shape"]["vocab"], seed=fx["forced_seed"])
    eng = Engine(backend, folder, window_limit=fx["window_limit"], lane_limit=lane_limit, precise=precise)
    try:
        ids, margins = eng.greedy(prompt, fx["gen"])
        eng.reset()
        eng.prime(prompt)
        picks, gaps = [], []
        token = int(prompt[-1])
        for t in forced:
            pick, gap = eng.step(token)
            picks.append(pick)
            gaps.append(gap)
            token = int(t)
    finally:
        eng.close()
    want = np.array(fx["plain"]["ids"], dtype=np.int32)
    gap = float(np.max(np.abs(margins - np.array(fx["plain"]["margin"]))))
    fgap = float(np.max(np.abs(np.array(gaps) - np.array(fx["plain"]["forced_margin"]))))
    print("greedy max gap difference", gap, "forced max gap difference", fgap,
          "forced distinct picks", len(set(picks)))
    assert np.array_equal(ids, want)
    assert gap <= 2e-3
    spread = float(np.max(np.abs(np.array(fx["plain"]["forced_margin"]) - np.array(fx["tuned"]["forced_margin"]))))
    print("reference builds' forced gap spread", spread)
    assert np.array_equal(np.array(picks), np.array(fx["plain"]["forced_ids"]))
    assert fgap <= max(2e-3, 3 * spread)
