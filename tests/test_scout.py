"""CPU checks of the speculative path's host side: the prompt-lookup scout
(igl_scout_*, restating app_core.c:12311-12361) and the greedy guess loop
(igllm_amd.engine.guess_loop, restating app_main.c:520-598).

The loop is driven by a stand-in model that replays the reference's greedy
stream from tests/golden/e2e_small_guess.json: greedy verification only reads a
block's picks up to its first disagreement, and there the pick is the greedy
stream's next id, so the loop's round / proposed / kept counts must equal the
reference binary's own counts for the same prompt."""
import json
import os

import numpy as np
import pytest

from igllm_amd import native
from igllm_amd.engine import Scout, guess_loop, prompt_ids

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def lib():
    return native.load()


def draw(lib, ids, want):
    s = Scout(lib)
    try:
        s.note(np.array(ids, dtype=np.int32))
        return list(s.draw(want))
    finally:
        s.close()


def test_scout_known_answers(lib):
    # the last 3 ids (1 2 3) occurred at 0: propose what followed
    assert draw(lib, [1, 2, 3, 9, 8, 1, 2, 3], 8) == [9, 8, 1, 2, 3]
    assert draw(lib, [1, 2, 3, 9, 8, 1, 2, 3], 2) == [9, 8]
    # the latest earlier occurrence wins
    assert draw(lib, [1, 2, 3, 7, 1, 2, 3, 6, 1, 2, 3], 1) == [6]
    # reach 3 fails, reach 2 (2 3) matches
    assert draw(lib, [5, 2, 3, 4, 1, 2, 3], 3) == [4, 1, 2]
    # a single shared id is not a memory: reach 1 is never used
    assert draw(lib, [5, 6, 7, 8, 6], 3) == []
    # too short, nothing asked, nothing known
    assert draw(lib, [4, 4], 3) == []
    assert draw(lib, [1, 2, 1, 2], 0) == []
    assert draw(lib, [], 3) == []
    # a run of one id: the latest earlier match has one id after it
    assert draw(lib, [7] * 6, 5) == [7]


def test_scout_against_brute_force(lib):
    """Every suffix of random low-alphabet streams against the definition:
    the longest reach in {3, 2} with an earlier occurrence that has ids after
    it, the latest such occurrence, at most `want` of the ids after it."""
    rng = np.random.default_rng(3)
    for trial in range(40):
        ids = rng.integers(0, 4, size=int(rng.integers(1, 60))).tolist()
        want = int(rng.integers(1, 8))
        expect = []
        for reach in (3, 2):
            n = len(ids)
            if n < reach + 1:
                continue
            tail = ids[n - reach:]
            places = [p for p in range(n - reach) if ids[p:p + reach] == tail]
            if places:
                p = max(places)
                expect = ids[p + reach:p + reach + want]
                break
        assert draw(lib, ids, want) == expect, (trial, ids, want)


def test_scout_incremental_against_brute_force(lib):
    """One long stream noted a few ids at a time (the index rehashes many
    times), drawn after every note, against the definition."""
    rng = np.random.default_rng(11)
    ids = rng.integers(0, 12, size=3000).tolist()
    s = Scout(lib)
    try:
        n = 0
        while n < len(ids):
            k = int(rng.integers(1, 5))
            s.note(np.array(ids[n:n + k], dtype=np.int32))
            n = min(n + k, len(ids))
            seen = ids[:n]
            expect = []
            for reach in (3, 2):
                if n < reach + 1:
                    continue
                tail = seen[n - reach:]
                places = [p for p in range(n - reach) if seen[p:p + reach] == tail]
                if places:
                    p = max(places)
                    expect = seen[p + reach:p + reach + 3]
                    break
            assert list(s.draw(3)) == expect, n
    finally:
        s.close()


def test_scout_grows(lib):
    s = Scout(lib)
    try:
        big = np.arange(5000, dtype=np.int32) % 1000
        for chunk in np.array_split(big, 7):
            s.note(chunk)
        assert list(s.draw(4)) == [0, 1, 2, 3]
    finally:
        s.close()


def test_guess_loop_reproduces_reference_counts(lib):
    g = json.load(open(os.path.join(GOLDEN, "e2e_small_guess.json")))
    assert g["streams_agree"] and g["guess_equals_greedy"]
    greedy = np.array(g["greedy"]["ids"], dtype=np.int32)
    prompt = prompt_ids(g["prompt_count"], g["shape"]["vocab"], seed=g["prompt_seed"],
                        repeat_span=g["repeat_span"])
    made = []  # the committed stream so far, as the session holds it
    open_block = {}

    def step(token):
        pick = int(greedy[len(made)])
        made.append(pick)
        return pick

    def guess(block):
        # lane j's pick is the greedy id after block[0 .. j], valid while the
        # proposed ids so far agree with the greedy stream
        n = len(made)
        picks = np.full(block.size, -1, dtype=np.int32)
        for j in range(block.size):
            if n + j >= greedy.size:
                break
            picks[j] = greedy[n + j]
            if j + 1 < block.size and block[j + 1] != greedy[n + j]:
                break
        open_block["picks"] = picks
        return picks

    def keep(count):
        picks = open_block.pop("picks")
        made.extend(int(t) for t in picks[:count])

    ids, (rounds, drawn, taken) = guess_loop(Scout(lib), prompt, g["gen"], g["guess_span"],
                                             step, guess, keep)
    assert np.array_equal(ids, greedy)
    assert made == greedy.tolist()
    assert (rounds, drawn, taken) == (g["plain"]["rounds"], g["plain"]["drawn"],
                                      g["plain"]["taken"])
