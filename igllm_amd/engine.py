"""Python host side of the device-resident decode session (include/igl_backend.h,
igl_engine_*) and of the synthetic Gemma 4 E2B checkpoint writer."""
from __future__ import annotations

import ctypes

import numpy as np

from . import native
from .backend import Backend, BackendError


def gemma_shape(**overrides) -> native.GemmaShape:
    """config.json's dimensions (35 layers, hidden 1536, ...), with overrides."""
    lib = native.load()
    s = native.GemmaShape()
    lib.igl_gemma_shape_e2b(ctypes.byref(s))
    for k, v in overrides.items():
        setattr(s, k, v)
    return s


SMALL = dict(vocab=4096, hidden=512, inner=1024, layers=10, shared_layers=4)


def write_gemma(folder: str, seed: int = 0, **overrides) -> native.GemmaShape:
    lib = native.load()
    s = gemma_shape(**overrides)
    code = lib.igl_gemma_write(folder.encode(), ctypes.byref(s), seed)
    if code != native.IGL_OKAY:
        raise BackendError(f"igl_gemma_write: {lib.igl_code_text(code).decode()}")
    return s


def prompt_ids(count: int, vocab: int, seed: int = 0, repeat_span: int = 0) -> np.ndarray:
    """A seeded random prompt; with `repeat_span`, its first `repeat_span` ids
    repeat until `count` (the speculative-decoding prompt)."""
    rng = np.random.default_rng(seed)
    if repeat_span:
        base = rng.integers(3, vocab, size=repeat_span).astype(np.int32)
        return np.resize(base, count).astype(np.int32)
    return rng.integers(3, vocab, size=count).astype(np.int32)


class Engine:
    def __init__(self, backend: Backend, folder: str, window_limit: int = 4096, lane_limit: int = 16,
                 precise: bool = True):
        self.backend = backend
        self.lib = backend.lib
        self.lane_limit = lane_limit
        self.handle = ctypes.c_void_p()
        code = self.lib.igl_engine_open(ctypes.byref(self.handle), ctypes.byref(backend.desk),
                                        folder.encode(), window_limit, lane_limit, int(precise))
        if code != native.IGL_OKAY:
            raise BackendError(f"igl_engine_open: {self.lib.igl_code_text(code).decode()} ({code})")
        self.vocab = self.lib.igl_engine_vocab(self.handle)

    def _check(self, code, what):
        if code != native.IGL_OKAY:
            raise BackendError(f"{what}: {self.lib.igl_code_text(code).decode()} ({code})")

    def prime(self, ids: np.ndarray):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        self._check(self.lib.igl_engine_prime(self.handle, ids.ctypes.data, ids.size), "prime")

    def step(self, token: int):
        pick = ctypes.c_int32()
        margin = ctypes.c_float()
        self._check(self.lib.igl_engine_step(self.handle, int(token), ctypes.byref(pick),
                                             ctypes.byref(margin)), "step")
        return pick.value, margin.value

    def logits(self, lane: int = 0) -> np.ndarray:
        out = np.empty(self.vocab, dtype=np.float32)
        self._check(self.lib.igl_engine_logits(self.handle, out.ctypes.data, lane), "logits")
        return out

    def greedy(self, prompt: np.ndarray, count: int):
        """prime + `count` greedy steps, the CLI's answer loop without the stop id."""
        self.prime(prompt)
        token = int(prompt[-1])
        picks, margins = [], []
        for _ in range(count):
            token, margin = self.step(token)
            picks.append(token)
            margins.append(margin)
        return np.array(picks, dtype=np.int32), np.array(margins, dtype=np.float32)

    @property
    def fill(self) -> int:
        return self.lib.igl_engine_fill(self.handle)

    def reset(self):
        self._check(self.lib.igl_engine_reset(self.handle), "reset")

    def set_graph(self, on: bool):
        self._check(self.lib.igl_engine_set_graph(self.handle, int(on)), "set_graph")

    def close(self):
        if self.handle:
            self.lib.igl_engine_close(self.handle)
            self.handle = ctypes.c_void_p()

    def guess(self, ids: np.ndarray):
        """One block pass (session_guess): the greedy pick and gap of every lane."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        picks = np.empty(ids.size, dtype=np.int32)
        margins = np.empty(ids.size, dtype=np.float32)
        self._check(self.lib.igl_engine_guess(self.handle, ids.ctypes.data, ids.size,
                                              picks.ctypes.data, margins.ctypes.data), "guess")
        return picks, margins

    def keep(self, count: int):
        self._check(self.lib.igl_engine_keep(self.handle, int(count)), "keep")

    def guess_greedy(self, prompt: np.ndarray, count: int, span: int = 4):
        """The CLI's greedy --guess loop (main_answer_guess, app_main.c:520-598)
        without the stop-id check: the scout proposes up to span - 1 ids, the
        block keeps the prefix the model agrees with plus its next pick; with
        nothing proposed, an ordinary step.  Returns the ids and (rounds, ids
        proposed, ids taken)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        self.prime(prompt)
        return guess_loop(Scout(self.lib), prompt, count, min(span, self.lane_limit),
                          lambda t: self.step(t)[0], lambda b: self.guess(b)[0], self.keep)


def guess_loop(scout, prompt, count, span, step, guess, keep):
    """main_answer_guess's greedy loop over a primed session: `step(id)` is
    one ordinary step's pick, `guess(block)` the picks of a block's lanes and
    `keep(n)` session_guess_keep.  Owns and closes `scout`."""
    span = max(1, min(span, 16))
    try:
        scout.note(prompt)
        token = int(prompt[-1])
        out, rounds, drawn, taken = [], 0, 0, 0
        while len(out) < count:
            want = max(0, min(span - 1, count - len(out) - 1))
            drafts = scout.draw(want)
            rounds += 1
            if drafts.size == 0:
                token = int(step(token))
                out.append(token)
                scout.note(np.array([token], dtype=np.int32))
                continue
            block = np.concatenate([np.array([token], dtype=np.int32), drafts])
            picks = guess(block)
            drawn += drafts.size
            take = 0
            while take + 1 < block.size and picks[take] == block[take + 1]:
                take += 1
            taken += take
            made = [int(t) for t in block[1:take + 1]] + [int(picks[take])]
            out.extend(made)
            scout.note(np.array(made, dtype=np.int32))
            token = made[-1]
            keep(take + 1)
        return np.array(out, dtype=np.int32), (rounds, drawn, taken)
    finally:
        scout.close()


class Scout:
    """The prompt-lookup proposer (igl_scout_*)."""

    def __init__(self, lib):
        self.lib = lib
        self.handle = ctypes.c_void_p()
        if lib.igl_scout_open(ctypes.byref(self.handle)) != native.IGL_OKAY:
            raise BackendError("igl_scout_open")

    def note(self, ids: np.ndarray):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        if self.lib.igl_scout_note(self.handle, ids.ctypes.data, ids.size) != native.IGL_OKAY:
            raise BackendError("igl_scout_note")

    def draw(self, want: int) -> np.ndarray:
        if want < 1:
            return np.empty(0, dtype=np.int32)
        out = np.empty(want, dtype=np.int32)
        got = self.lib.igl_scout_draw(self.handle, out.ctypes.data, want)
        return out[:got].copy()

    def close(self):
        if self.handle:
            self.lib.igl_scout_close(self.handle)
            self.handle = ctypes.c_void_p()
