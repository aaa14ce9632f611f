#!/usr/bin/env python3
"""Benchmark of the gfx950 backend on the quantized projection path.

A step is one pass of the small-lane GEMV sweep (gate/up shape N=8192,K=2048
and down shape N=2048,K=8192, int4 group 32, M in {1,2,4,8} lanes of fp32
activations, seed 0): eight products, each on its own copy of the weights,
rotated through more copies than the 256 MiB Infinity Cache holds, so every
byte is read from HBM.  `value` is the step's algorithmic bytes over its time,
the K timed steps recorded once and replayed with HIP events on the desk's
stream around the replay (the GPU's time; the same steps enqueued one ctypes
call a launch are reported beside it).

Beside it, on the same run: the decode GEMV alone (M=1, 8192x2048, the
dominant kernel) against the HBM roofline, the batched prefill GEMM against
the bf16/f16 MFMA peak, the decode attention over a 16384-position byte ring,
and the reference's own CPU float path (oracle/_ref, AVX2+FMA build, the
host's cores) on a bounded sample of the same sweep.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0          # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0   # MI355X dense fp16/bf16 MFMA
MFMA_I8_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA
# Threads the CPU legs use: the GPU box's CPU share for one GPU is 16, whatever
# nproc reports there, so 16 is "all cores" of this job.
CPU_SHARE = 16
SHAPES = [(8192, 2048), (2048, 8192)]
LANES = [1, 2, 4, 8]
COPIES = 48                     # 48 x 10.5 MB per shape: past the 256 MiB MALL
ATTEND_COPIES = 40              # 40 x 8 MiB of key/value rings: past the MALL
# The roofline's profile figures come from the committed rocprofv3 summaries:
# the decode GEMV's (M=1, 8192x2048) kernel-trace duration and its FETCH_SIZE /
# WRITE_SIZE per dispatch, scaled by the factors a 256 MiB device copy gives.
GEMV_M1_PROFILE = os.path.join(ROOT, "profiles", "gemv_q4_m1_8192x2048.md")
COPY_PROFILE = os.path.join(ROOT, "profiles", "copy_256mib_calibration.md")
GEMV_M1_KERNEL = "gemv_q4_dot_kernel<1, 2, 1, 1, false>"


def profile_rows(path, kernel):
    """The table rows of a profile summary whose kernel cell names `kernel`:
    [(cells...), ...] in file order (the kernel-trace row, then the counters')."""
    rows = []
    with open(path) as f:
        for line in f:
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if line.startswith("|") and len(cells) > 1 and kernel in cells[0]:
                rows.append(cells)
    return rows


def gemv_m1_profile(algo_bytes):
    """roofline.traffic and the rocprof duration of the decode GEMV, from the
    committed profiles: traffic = FETCH_SIZE x f + WRITE_SIZE x w KiB, where
    the copy of a known 256 MiB gives f = 262144 / its FETCH_SIZE and w =
    262144 / its WRITE_SIZE."""
    try:
        copy = profile_rows(COPY_PROFILE, "__amd_rocclr_copyBuffer")
        gemv = profile_rows(GEMV_M1_PROFILE, GEMV_M1_KERNEL)
        f = 262144.0 / round(float(copy[-1][1]))
        w = 262144.0 / float(copy[-1][2])
        fetch, write = float(gemv[-1][1]), float(gemv[-1][2])
        avg_ns = float(gemv[0][2])
    except (OSError, IndexError, ValueError, ZeroDivisionError):
        return None
    traffic = int(round((fetch * f + write * w) * 1024))
    return {"traffic": traffic, "fetch_kib": fetch, "write_kib": write, "fetch_factor": round(f, 4),
            "write_factor": round(w, 4), "rocprof_avg_launch_us": round(avg_ns / 1e3, 3),
            "rocprof_frac": round(algo_bytes / (avg_ns * 1e-9) / 1e9 / HBM_PEAK_GBPS, 4),
            "source": "profiles/gemv_q4_m1_8192x2048.md (kernel trace avg ns; FETCH_SIZE, WRITE_SIZE KiB a "
                      "dispatch) scaled by profiles/copy_256mib_calibration.md"}


def gemv_bytes(N, K, M, group=32):
    return N * K // 2 + N * (K // group) * 4 + M * (K + N) * 4


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-e2e", action="store_true", help="skip the end-to-end decode leg")
    ap.add_argument("--kernel", choices=["gemv", "gemv8", "gemm", "attend", "attend_rows", "copy", "head2", "real",
                                         "calib", "readfloor", "decode", "guess"],
                    help="run one kernel's workload alone in a loop (for rocprofv3) and exit")
    ap.add_argument("--lanes", type=int, default=2048, help="--kernel gemm: the lane count M")
    ap.add_argument("--shape", type=int, default=0, choices=[0, 1],
                    help="--kernel gemm: 0 for 8192x2048, 1 for 2048x8192")
    return ap.parse_args()


def kernel_loop(be, name, reps, lanes=2048, shape=0):
    """One kernel's workload alone, for counter runs: the decode GEMV (M=1,
    8192x2048, rotated copies), the M=8 GEMV, the prefill GEMM (M lanes, either
    shape; M=2048 on 8192x2048 by default), the
    L=16384 attention, the prefill attention (2047 lanes over a 2048-position
    ring of 512-dim heads, then a 512-position window of 256-dim heads, e4m3,
    alternating), a 256 MiB device copy that calibrates FETCH_SIZE and
    WRITE_SIZE against a known byte count, the 2-bit 262144x1536 head and the
    bf16 8960x1536 real plane at M=1 (rotated copies), the calibrated
    prefill (M=2048, 8192x2048 4-bit, one gain a row), or the read floor (the
    M=1 GEMV's byte count read once, rotated buffers)."""
    import ctypes
    from igllm_amd.backend import synth_projection

    if name == "copy":
        nbytes = 256 << 20
        src, dst = be.alloc(nbytes), be.alloc(nbytes)
        lib = be.lib
        hip = ctypes.CDLL("libamdhip64.so")
        hip.hipMemcpyDtoD.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
        for _ in range(reps):
            if hip.hipMemcpyDtoD(dst.ptr, src.ptr, nbytes) != 0:
                raise RuntimeError("hipMemcpyDtoD failed")
        be.sync()
        print(json.dumps({"kernel": "copy", "bytes_each": nbytes, "reps": reps}))
        del lib
        return
    if name == "readfloor":
        N, K = SHAPES[0]
        nbytes = gemv_bytes(N, K, 1)
        bufs = [be.alloc(nbytes) for _ in range(COPIES)]
        for i in range(20):
            be.read_floor_dev(bufs[i % COPIES], nbytes)
        be.sync()
        be.mark()
        for i in range(reps):
            be.read_floor_dev(bufs[i % COPIES], nbytes)
        be.mark()
        us = be.marks_ms() * 1e3 / reps
        print(json.dumps({"kernel": "read_floor", "bytes": nbytes, "avg_us": round(us, 3),
                          "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}))
        return
    if name in ("head2", "real"):
        key = "u2_head_262144x1536" if name == "head2" else "bf16_ple_model_8960x1536"
        rot = KindRotation(be, KIND_CASES[key])
        N, K = rot.N, rot.K
        x = be.upload(np.random.default_rng(1).normal(size=(1, K)).astype(np.float32))
        y = be.alloc(N * 4)
        for i in range(3):  # first launches load the code objects
            be.gemv_dev(rot.planes[i % rot.copies], x, K, 1, y, N)
        be.sync()
        be.mark()
        for i in range(reps):
            be.gemv_dev(rot.planes[i % rot.copies], x, K, 1, y, N)
        be.mark()
        us = be.marks_ms() * 1e3 / reps
        print(json.dumps({"kernel": key, "avg_us": round(us, 3), "algorithmic_bytes": rot.algo,
                          "GBps": round(rot.algo / (us * 1e-6) / 1e9, 1)}))
        return
    if name == "calib":
        from igllm_amd.backend import make_plane
        N, K, M = 8192, 2048, 2048
        rng = np.random.default_rng(2)
        codes = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
        gains = np.abs(rng.normal(0, 0.02, size=(N, 1))).astype(np.float32)
        cp = be.attach(make_plane(codes, gains, K, group_size=K))
        cp.plane.enter_gain = 2.5 / 127
        cp.plane.leave_gain = 0.02
        a = be.upload(rng.normal(size=(M, K)).astype(np.float32))
        c = be.alloc(M * N * 4)
        for _ in range(3):  # first launches load the code objects
            be.plane_lift_dev(cp, a, K, M, c, N)
        be.sync()
        be.mark()
        for _ in range(reps):
            be.plane_lift_dev(cp, a, K, M, c, N)
        be.mark()
        us = be.marks_ms() * 1e3 / reps
        print(json.dumps({"kernel": "calib", "M": M, "N": N, "K": K, "avg_us": round(us, 2)}))
        return
    if name in ("gemv", "gemv8"):
        N, K = SHAPES[0]
        M = 1 if name == "gemv" else 8
        rot = Rotation(be, N, K)
        _, _, act = synth_projection(N, K, M, seed=0)
        a = be.upload(act)
        o = be.alloc(M * N * 4)
        for i in range(3):  # first launches load the code objects
            be.gemv_dev(rot.planes[i % COPIES], a, K, M, o, N)
        be.sync()
        be.mark()
        for i in range(reps):
            be.gemv_dev(rot.planes[i % COPIES], a, K, M, o, N)
        be.mark()
        us = be.marks_ms() * 1e3 / reps
        print(json.dumps({"kernel": name, "N": N, "K": K, "M": M, "avg_us": round(us, 3),
                          "algorithmic_bytes": gemv_bytes(N, K, M),
                          "GBps": round(gemv_bytes(N, K, M) / (us * 1e-6) / 1e9, 1)}))
        return
    if name == "gemm":
        N, K = SHAPES[shape]
        M = lanes
        rot = Rotation(be, N, K)
        a = be.alloc(M * K * 2)
        c = be.alloc(M * N * 2)
        rng = np.random.default_rng(0)
        a.put((rng.normal(size=M * K).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16))
        for i in range(3):  # first launches load the code objects
            be.gemm_bf16_dev(rot.planes[i % COPIES], a, K, M, c, N)
        be.sync()
        be.mark()
        for i in range(reps):
            be.gemm_bf16_dev(rot.planes[i % COPIES], a, K, M, c, N)
        be.mark()
        us = be.marks_ms() * 1e3 / reps
        print(json.dumps({"kernel": "gemm", "M": M, "N": N, "K": K, "avg_us": round(us, 2),
                          "TFLOPs": round(2.0 * M * N * K / (us * 1e-6) / 1e12, 1)}))
        return
    if name == "attend":
        # int8 rings of 16384 positions, 40 copies (320 MB, past the MALL)
        L, head, copies = 16384, 256, ATTEND_COPIES
        rng = np.random.default_rng(1)
        rings = [(be.upload(rng.integers(0, 256, size=(L, head), dtype=np.uint8)),
                  be.upload(rng.integers(0, 256, size=(L, head), dtype=np.uint8))) for _ in range(copies)]
        q = be.upload(rng.normal(size=(8, head)).astype(np.float32))
        o = be.alloc(8 * head * 4)
        for i in range(3):  # first launches load the code objects
            be.attend_dev(rings[i][0], rings[i][1], 1, 4.0 / 127, 4.0 / 127, L, 1, 8, head, q, 0, L, 1.0 / 16, o)
        be.sync()
        be.mark()
        for i in range(reps):
            kb, vb = rings[i % copies]
            be.attend_dev(kb, vb, 1, 4.0 / 127, 4.0 / 127, L, 1, 8, head, q, 0, L, 1.0 / 16, o)
        be.mark()
        us = be.marks_ms() * 1e3 / reps
        print(json.dumps({"kernel": "attend", "L": L, "copies": copies, "avg_us": round(us, 2)}))
        return
    if name == "attend_rows":
        lanes, rng = 2047, np.random.default_rng(2)
        cases = []
        for window, head in ((0, 512), (512, 256)):
            span = window + lanes if window else lanes + 1
            kb = be.upload(rng.integers(0, 120, size=(span, head), dtype=np.uint8))
            vb = be.upload(rng.integers(0, 120, size=(span, head), dtype=np.uint8))
            q = be.upload(rng.normal(size=(lanes, 8 * head)).astype(np.float32))
            o = be.alloc(lanes * 8 * head * 4)
            cases.append((window, head, span, kb, vb, q, o))

        def launch(c):
            window, head, span, kb, vb, q, o = c
            code = be.lib.igl_attend_lanes_dev(ctypes.byref(be.desk), kb.ptr, vb.ptr, 0, 0.02, 0.02, span, 1, 8,
                                               head, q.ptr, 8 * head, 1, window, lanes, 1.0 / 16, o.ptr)
            if code != 0:
                raise RuntimeError("igl_attend_lanes_dev failed: %d" % code)
        for c in cases:
            launch(c)
        be.sync()
        be.mark()
        for i in range(reps):
            launch(cases[i % 2])
        be.mark()
        us = be.marks_ms() * 1e3 / reps
        print(json.dumps({"kernel": "attend_rows", "lanes": lanes, "avg_us_per_launch": round(us, 2)}))
        return
    if name == "decode":
        decode_loop(be, reps)
        return
    if name == "guess":
        guess_loop_blocks(be, reps)


def decode_loop(be, steps):
    """Decode steps alone, for kernel traces: the synthetic E2B checkpoint, a
    2048-id prompt primed, then `steps` greedy steps launched eagerly (the e2e
    leg's decode without its timers or its step graph)."""
    import tempfile
    from igllm_amd.engine import Engine, prompt_ids, write_gemma

    root = "/dev/shm" if os.path.isdir("/dev/shm") else tempfile.gettempdir()
    folder = os.path.join(root, f"igl_gemma_e2b_{os.getpid()}")
    try:
        shape = write_gemma(folder, seed=0)
        prompt = prompt_ids(2048, shape.vocab, seed=0)
        eng = Engine(be, folder, window_limit=2048 + steps + 64, lane_limit=16, precise=True)
        try:
            # eager: the step's launches one by one, not its captured graph
            # (rocprofv3's kernel trace of the graph launch has aborted in the
            # profiler's interception)
            eng.set_graph(False)
            eng.prime(prompt)
            token = int(prompt[-1])
            for _ in range(steps):
                token, _ = eng.step(token)
            be.sync()
        finally:
            eng.close()
    finally:
        import shutil
        shutil.rmtree(folder, ignore_errors=True)
    print(json.dumps({"kernel": "decode", "prompt": 2048, "steps": steps}))


def guess_loop_blocks(be, blocks, lanes=2):
    """Speculative blocks alone, for kernel traces: the synthetic E2B
    checkpoint, a 2048-id prompt primed, then `blocks` blocks of `lanes` ids
    (the next input and a proposal) launched eagerly and not kept: the
    --guess leg's 2-lane round without its step graph."""
    import tempfile
    from igllm_amd.engine import Engine, prompt_ids, write_gemma

    root = "/dev/shm" if os.path.isdir("/dev/shm") else tempfile.gettempdir()
    folder = os.path.join(root, f"igl_gemma_e2b_{os.getpid()}")
    try:
        shape = write_gemma(folder, seed=0)
        prompt = prompt_ids(2048, shape.vocab, seed=0)
        eng = Engine(be, folder, window_limit=2048 + 64, lane_limit=16, precise=True)
        try:
            eng.set_graph(False)
            eng.prime(prompt)
            block = np.full(lanes, int(prompt[-1]), np.int32)
            for _ in range(blocks):
                eng.guess(block)
                eng.keep(0)
            be.sync()
        finally:
            eng.close()
    finally:
        import shutil
        shutil.rmtree(folder, ignore_errors=True)
    print(json.dumps({"kernel": "guess", "prompt": 2048, "blocks": blocks, "lanes": lanes}))


def cpu_e2e(folder, prompt, gen=8, prime=2048):
    """The reference engine itself (oracle/_ref, AVX2+FMA build) on the same
    checkpoint, on this host's cores: the GPU leg's whole 2048-id prompt, so the
    decode steps run at the same context, then `gen` greedy steps (a bounded
    sample of the GPU leg's 256), each phase timed by the reference."""
    import ctypes
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as ol

    if ol.ref("tuned") is None:
        return None
    lib = ctypes.CDLL(ol.REF_TUNED_PATH)
    fn = lib.ref_engine_clock
    fn.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                   ctypes.c_int, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]
    cores = min(CPU_SHARE, os.cpu_count() or 1)
    ids = np.ascontiguousarray(prompt[:prime], dtype=np.int32)
    prime_s, step_s = ctypes.c_double(), ctypes.c_double()
    code = fn(folder.encode(), cores, 8, prime + gen + 16, ids.ctypes.data, ids.size, gen,
              ctypes.byref(prime_s), ctypes.byref(step_s))
    if code != 0:
        return {"error": f"ref_engine_clock returned {code}"}
    return {"decode_tok_s": round(gen / step_s.value, 2), "prefill_tok_s": round((prime - 1) / prime_s.value, 1),
            "cores": cores, "kind": "reference",
            "sample": f"reference engine (app_core.c, AVX2+FMA build), {prime}-id prompt then {gen} greedy "
                      f"steps (the GPU leg's context) on the same checkpoint, {cores} threads"}


# Lanes a fast-mode prefill pass carries: the whole 2048-id prompt at once.  The
# prefill products are then M = 2047 GEMMs that fill the GPU; at 256 lanes a
# pass the 2048-row projections were 8 tiles (15.5k against 38.7k tok/s).
FAST_LANES = 2048


def decode_bytes(shape, place):
    """HBM bytes one decode step at `place` reads at config dimensions with
    int4 group-32 planes: every plane's codes and scales once (the projections
    of each layer, the per-layer-input gate and projection, the model's
    per-layer projection and the tied head), the embedding rows it gathers, and
    the FP8 key/value bytes each layer's attention reads (a sliding layer the
    last `window` positions, a full one all of them; a layer that shares
    another's cache reads that cache again)."""
    def plane(n, k):
        return n * k // 2 + n * (k // 32) * 4

    from igllm_amd.native import load
    import ctypes
    lib = load()
    H, P, L = shape.hidden, shape.ple_size, shape.layers
    total = plane(shape.vocab, H) + plane(P * L, H)  # head and the model's per-layer projection
    total += H // 2 + H // 32 * 4 + P * L // 2 + P * L // 32 * 4  # one embedding row of each table
    first_share = L - shape.shared_layers
    for i in range(L):
        full = lib.igl_gemma_full_layer(ctypes.byref(shape), i)
        hd = shape.full_head_dim if full else shape.head_dim
        inner = shape.inner * (2 if shape.double_wide and i >= first_share else 1)
        q = shape.heads * hd
        total += plane(q, H) + plane(H, q)  # q and o
        if i < first_share:
            total += 2 * plane(shape.kv_heads * hd, H)  # k and v
        total += 2 * plane(inner, H) + plane(H, inner)  # gate, up, down
        total += plane(P, H) + plane(H, P)  # per-layer-input gate and projection
        span = place + 1 if full else min(place + 1, shape.window)
        total += 2 * span * shape.kv_heads * hd
    return total


def e2e_decode(be, prompt_count=2048, gen=256, cpu=True):
    """Synthetic Gemma-4-E2B-shaped decode (model/config.json dimensions, every
    plane int4 group 32, FP8 key/value cache): write the seeded checkpoint,
    prime a 2048-id seeded prompt, then 256 greedy steps."""
    import tempfile
    from igllm_amd.engine import Engine, prompt_ids, write_gemma

    root = "/dev/shm" if os.path.isdir("/dev/shm") else tempfile.gettempdir()
    folder = os.path.join(root, f"igl_gemma_e2b_{os.getpid()}")
    t0 = time.perf_counter()
    shape = write_gemma(folder, seed=0)
    write_s = time.perf_counter() - t0
    prompt = prompt_ids(prompt_count, shape.vocab, seed=0)
    out = {"model": "synthetic Gemma-4-E2B text stack (model/config.json dims), int4 g32, "
                    "FP8 KV cache", "prompt": prompt_count, "gen": gen,
           "checkpoint_write_s": round(write_s, 1)}
    try:
        for precise in (False, True):
            t0 = time.perf_counter()
            eng = Engine(be, folder, window_limit=prompt_count + gen + 64,
                         lane_limit=16 if precise else FAST_LANES, precise=precise)
            load_s = time.perf_counter() - t0
            try:
                t0 = time.perf_counter()
                eng.prime(prompt)
                be.sync()
                prime_s = time.perf_counter() - t0
                token = int(prompt[-1])
                picks, margins = [], []
                t0 = time.perf_counter()
                for _ in range(gen):
                    token, margin = eng.step(token)
                    picks.append(token)
                    margins.append(margin)
                decode_s = time.perf_counter() - t0
            finally:
                eng.close()
            key = "precise" if precise else "fast_prefill"
            step_bytes = decode_bytes(shape, prompt_count - 1 + gen // 2)
            out[key] = {"load_s": round(load_s, 2),
                        "prefill_tok_s": round((prompt_count - 1) / prime_s, 1),
                        "decode_tok_s": round(gen / decode_s, 1),
                        "decode_ms_per_token": round(decode_s * 1e3 / gen, 3),
                        "bytes_per_token": step_bytes,
                        "hbm_frac": round(step_bytes / (decode_s / gen) / 1e9 / HBM_PEAK_GBPS, 4),
                        "min_margin": round(float(min(margins)), 5),
                        "first_ids": picks[:16],
                        "lane_limit": 16 if precise else FAST_LANES}
            out.setdefault("streams", []).append(picks)
        out["prefill_modes_agree"] = out["streams"][0] == out["streams"][1]
        out.pop("streams")
        out["guess"] = e2e_guess(be, folder, shape, prompt_count, gen)
        if cpu:
            out["cpu_baseline"] = cpu_e2e(folder, prompt)
    finally:
        import shutil
        shutil.rmtree(folder, ignore_errors=True)
    out["export_kinds"] = e2e_kinds(be, prompt_count, gen)
    return out


def e2e_kinds(be, prompt_count, gen):
    """The same dimensions in the export's own kinds: 2-bit MLPs from layer 15
    and a 2-bit tied head, I8 per-layer planes, bf16 per_layer_model_projection,
    one scale a row, every projection but the head calibrated (activation
    grids, the product on integer levels)."""
    import shutil
    import tempfile
    from igllm_amd.engine import Engine, prompt_ids, write_gemma

    root = "/dev/shm" if os.path.isdir("/dev/shm") else tempfile.gettempdir()
    folder = os.path.join(root, f"igl_gemma_e2b_kinds_{os.getpid()}")
    try:
        shape = write_gemma(folder, seed=0, kinds=1)
        prompt = prompt_ids(prompt_count, shape.vocab, seed=0)
        eng = Engine(be, folder, window_limit=prompt_count + gen + 64, lane_limit=FAST_LANES, precise=False)
        try:
            t0 = time.perf_counter()
            eng.prime(prompt)
            be.sync()
            prime_s = time.perf_counter() - t0
            token = int(prompt[-1])
            margins = []
            t0 = time.perf_counter()
            for _ in range(gen):
                token, margin = eng.step(token)
                margins.append(margin)
            decode_s = time.perf_counter() - t0
        finally:
            eng.close()
        return {"prefill_tok_s": round((prompt_count - 1) / prime_s, 1),
                "decode_tok_s": round(gen / decode_s, 1),
                "decode_ms_per_token": round(decode_s * 1e3 / gen, 3),
                "min_margin": round(float(min(margins)), 5), "lane_limit": FAST_LANES}
    finally:
        shutil.rmtree(folder, ignore_errors=True)


def e2e_guess(be, folder, shape, prompt_count, gen, span=4, repeat=512):
    """--guess 4 against plain greedy decode on a prompt that repeats its first
    512 ids, on one engine: plain decode, then the same prompt again under the
    prompt-lookup loop.  The two streams must agree."""
    from igllm_amd.engine import Engine, Scout, guess_loop, prompt_ids

    prompt = prompt_ids(prompt_count, shape.vocab, seed=0, repeat_span=repeat)
    eng = Engine(be, folder, window_limit=prompt_count + gen + 64, lane_limit=16, precise=True)
    try:
        eng.prime(prompt)
        be.sync()
        token, plain = int(prompt[-1]), []
        t0 = time.perf_counter()
        for _ in range(gen):
            token, _ = eng.step(token)
            plain.append(token)
        plain_s = time.perf_counter() - t0
        eng.reset()
        eng.prime(prompt)
        be.sync()
        t0 = time.perf_counter()
        ids, (rounds, drawn, taken) = guess_loop(
            Scout(eng.lib), prompt, gen, span, lambda t: eng.step(t)[0],
            lambda b: eng.guess(b)[0], eng.keep)
        guess_s = time.perf_counter() - t0
    finally:
        eng.close()
    return {"prompt": f"{prompt_count} ids repeating the first {repeat}", "span": span,
            "gen": gen, "decode_tok_s": round(gen / guess_s, 1),
            "plain_decode_tok_s": round(gen / plain_s, 1),
            "rounds": rounds, "drawn": drawn, "taken": taken,
            "streams_agree": bool(np.array_equal(ids, plain)), "first_ids": ids[:16].tolist()}


# The shipped export's other decode products (model/config.json
# module_quant_configs; one gain a row): name -> (N, K, bits, flip) for code
# planes, (N, K, "bf16") for the real plane.
KIND_CASES = {
    "u2_mlp_gate_6144x1536": (6144, 1536, 2, 0),
    "u2_mlp_down_1536x6144": (1536, 6144, 2, 0),
    "u2_head_262144x1536": (262144, 1536, 2, 0),
    "i8_ple_gate_256x1536": (256, 1536, 8, 128),
    "i8_ple_proj_1536x256": (1536, 256, 8, 128),
    "u4_q_proj_2048x1536": (2048, 1536, 4, 0),
    "bf16_ple_model_8960x1536": (8960, 1536, "bf16"),
    # calibrated (enter_gain): the product on the activation grid, igl_plane_lift_dev
    "u4_calibrated_8192x2048": (8192, 2048, 4, 0, 2.5 / 127),
    "u2_calibrated_mlp_gate_6144x1536": (6144, 1536, 2, 0, 2.5 / 127),
}


class KindRotation:
    """Device copies of one plane of another kind (enough to pass the 256 MiB
    MALL), each bound as its own plane; `algo` is one M=1 product's
    algorithmic bytes."""

    def __init__(self, backend, case, seed=0):
        import ctypes
        from igllm_amd import native
        from igllm_amd.backend import make_plane, make_real_plane

        rng = np.random.default_rng(seed)
        N, K = case[0], case[1]
        if case[2] == "bf16":
            w = rng.normal(0, 0.05, size=(N, K)).astype(np.float32)
            rows = (w.view(np.uint32) >> 16).astype(np.uint16)
            payload, gains = rows, None
            maker = lambda: make_real_plane(rows, native.IGL_STORE_BF16)  # noqa: E731
            self.lift = False
            self.algo = N * K * 2 + (K + N) * 4
        else:
            bits, flip = case[2], case[3]
            stride = ((K * bits + 7) // 8 + 15) // 16 * 16
            codes = rng.integers(0, 256, size=(N, stride), dtype=np.uint8)
            gains = np.abs(rng.normal(0, 0.02, size=(N, 1))).astype(np.float32)
            payload = codes
            step = case[4] if len(case) > 4 else 0.0

            def maker():
                cp = make_plane(codes, gains, K, group_size=K, bits=bits, code_flip=flip)
                cp.plane.enter_gain = step
                return cp
            self.lift = step > 0
            self.algo = N * stride + N * 4 + (K + N) * 4
        pstride = (payload.nbytes + 255) // 256 * 256
        self.copies = max(2, -(-(320 << 20) // pstride))
        self.payload = backend.alloc(pstride * self.copies)
        self.gains = backend.upload(gains) if gains is not None else None
        self.planes = []
        for c in range(self.copies):
            self.payload.put(payload, c * pstride)
            cp = maker()
            code = backend.lib.igl_plane_bind_dev(
                ctypes.byref(backend.desk), ctypes.byref(cp.plane), self.payload.ptr + c * pstride,
                self.gains.ptr if self.gains is not None else None)
            if code != native.IGL_OKAY:
                raise RuntimeError(f"bind_dev: {code}")
            self.planes.append(cp)
        self.N, self.K = N, K


def kinds_leg(be, reps=100):
    """M=1 GEMV of each KIND_CASES plane, rotated copies, HIP events."""
    out = {}
    for name, case in KIND_CASES.items():
        rot = KindRotation(be, case)
        N, K = rot.N, rot.K
        x = be.upload(np.random.default_rng(1).normal(size=(1, K)).astype(np.float32))
        y = be.alloc(N * 4)
        run = be.plane_lift_dev if rot.lift else be.gemv_dev
        for i in range(10):
            run(rot.planes[i % rot.copies], x, K, 1, y, N)
        be.sync()
        be.mark()
        for i in range(reps):
            run(rot.planes[i % rot.copies], x, K, 1, y, N)
        be.mark()
        us = be.marks_ms() * 1e3 / reps
        gbps = rot.algo / (us * 1e-6) / 1e9
        out[name] = {"us": round(us, 3), "algorithmic_bytes": rot.algo, "GBps": round(gbps, 1),
                     "frac_of_hbm_peak": round(gbps / HBM_PEAK_GBPS, 4), "copies": rot.copies}
        for cp in rot.planes:
            be.detach(cp)
        rot.payload.free()
        if rot.gains is not None:
            rot.gains.free()
        x.free()
        y.free()
    return out


class Rotation:
    """COPIES device copies of one weight set, each bound as its own plane."""

    def __init__(self, backend, N, K, seed=0):
        from igllm_amd.backend import make_plane, synth_projection

        codes, gains, _ = synth_projection(N, K, 1, seed=seed)
        self.host = (codes, gains)
        self.N, self.K = N, K
        cbytes, gbytes = codes.nbytes, gains.nbytes
        self.cstride = (cbytes + 255) // 256 * 256
        self.gstride = (gbytes + 255) // 256 * 256
        self.codes = backend.alloc(self.cstride * COPIES)
        self.gains = backend.alloc(self.gstride * COPIES)
        self.planes = []
        for c in range(COPIES):
            self.codes.put(codes, c * self.cstride)
            self.gains.put(gains, c * self.gstride)
            cp = make_plane(codes, gains, K)
            backend.bind_dev(cp, self.codes, self.gains, c * self.cstride, c * self.gstride)
            self.planes.append(cp)


def cpu_baseline(budget_s=10.0):
    """The reference's float back_mat_mat over the same sweep, on this host:
    the job's whole CPU share (16 threads), then one thread."""
    allc = cpu_sweep(min(CPU_SHARE, os.cpu_count() or 1), budget_s)
    one = cpu_sweep(1, budget_s)
    allc["one_thread"] = {k: one[k] for k in ("value", "unit", "cores", "kind", "sample")}
    return allc


def ref_tuned():
    """The reference's AVX2+FMA build (oracle/_ref) when this host can run it,
    else None."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as ol

    flags = ""
    try:
        flags = open("/proc/cpuinfo").read()
    except OSError:
        pass
    lib = ol.ref("tuned")
    return lib if lib is not None and " avx2" in flags and " fma" in flags else None


def cpu_attention(budget_s=3.0):
    """The reference's own decode attention (ref_attend: attend_score_band and
    attend_blend_band forked over its pool, AVX2+FMA build) on the bench's case:
    one lane, 8 query heads on one key/value head of 256 dims, int8 rings of
    16384 positions; the job's CPU share of threads, then one, each for about
    `budget_s` seconds."""
    import ctypes

    lib = ref_tuned()
    if lib is None:
        return None
    import oracle_lib as ol

    L, head, scale = 16384, 256, 4.0 / 127
    rng = np.random.default_rng(1)
    kb = rng.integers(0, 256, size=(L, head), dtype=np.uint8)
    vb = rng.integers(0, 256, size=(L, head), dtype=np.uint8)
    q = rng.normal(size=(8, head)).astype(np.float32)
    grid = np.arange(256, dtype=np.uint32).astype(np.uint8).view(np.int8).astype(np.float32) * np.float32(scale)
    out = np.zeros((8, head), dtype=np.float32)
    res = {}
    for cores in (min(CPU_SHARE, os.cpu_count() or 1), 1):
        desk = lib.ref_desk_open(cores, 64, 2048)
        try:
            calls, t0 = 0, time.perf_counter()
            while True:
                lib.ref_attend(desk, ol.p(kb), ol.p(vb), ol.p(grid), ol.p(grid), L, head, 0, ol.p(q), 0, 8,
                               head, 0, L, ol.p(out))
                calls += 1
                if time.perf_counter() - t0 > budget_s:
                    break
            us = (time.perf_counter() - t0) * 1e6 / calls
        finally:
            lib.ref_desk_close(desk)
        res[cores] = (us, calls)
    cores = max(res)
    return {"us": round(res[cores][0], 1), "GBps": round(2 * L * head / (res[cores][0] * 1e-6) / 1e9, 2),
            "cores": cores, "one_thread_us": round(res[1][0], 1), "kind": "reference",
            "sample": f"{res[cores][1]} and {res[1][1]} calls of ref_attend (app_core.c's score and blend "
                      f"bands, AVX2+FMA build) at L={L}, int8 rings, {cores} threads and 1"}


def cpu_prefill(budget_s=5.0):
    """The reference's back_mat_mat (AVX2+FMA float path, its pool) on a
    256-lane prefill of the 8192x2048 int4 plane: the job's CPU share of threads
    and one, each for about `budget_s` seconds.  256 lanes, not 2048: the
    reference takes the same 16-lane chunks either way, and 2048 lanes would
    run past the bench's few minutes on one thread."""
    import ctypes
    from igllm_amd.backend import synth_projection

    lib = ref_tuned()
    if lib is None:
        return None
    import oracle_lib as ol

    (N, K), M = SHAPES[0], 256
    codes, gains, act = synth_projection(N, K, M, seed=0)
    d = ol.plane_desc(codes, gains, K)
    out = np.empty((M, N), dtype=np.float32)
    res = {}
    for cores in (min(CPU_SHARE, os.cpu_count() or 1), 1):
        desk = lib.ref_desk_open(cores, 256, 8192)
        try:
            calls, t0 = 0, time.perf_counter()
            while True:
                lib.ref_desk_mat_mat(desk, ctypes.byref(d), ol.p(act), K, M, ol.p(out), N)
                calls += 1
                if time.perf_counter() - t0 > budget_s:
                    break
            s_each = (time.perf_counter() - t0) / calls
        finally:
            lib.ref_desk_close(desk)
        res[cores] = (s_each, calls)
    cores = max(res)
    flops = 2.0 * M * N * K
    return {"TFLOPs": round(flops / res[cores][0] / 1e12, 4), "lanes_per_s": round(M / res[cores][0], 1),
            "cores": cores, "one_thread_TFLOPs": round(flops / res[1][0] / 1e12, 5), "kind": "reference",
            "sample": f"{res[cores][1]} and {res[1][1]} calls of back_mat_mat (AVX2+FMA float build), "
                      f"M={M} lanes of the {N}x{K} int4 plane, {cores} threads and 1"}


def cpu_sweep(cores, budget_s):
    """`cores` threads of the reference's float back_mat_mat over the sweep for
    about `budget_s` seconds."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import ctypes
    import oracle_lib as ol
    from igllm_amd.backend import synth_projection

    lib = ol.ref("tuned")
    kind = "reference"
    flags = ""
    try:
        flags = open("/proc/cpuinfo").read()
    except OSError:
        pass
    if lib is None or " avx2" not in flags or " fma" not in flags:
        lib, kind = None, "port"
    cases = []
    for (N, K) in SHAPES:
        for M in LANES:
            codes, gains, act = synth_projection(N, K, M, seed=0)
            cases.append((N, K, M, codes, gains, act))
    total_bytes = 0
    t0 = time.perf_counter()
    passes = 0
    if kind == "reference":
        desk = lib.ref_desk_open(cores, 256, 8192)
        try:
            while True:
                for (N, K, M, codes, gains, act) in cases:
                    d = ol.plane_desc(codes, gains, K)
                    out = np.empty((M, N), dtype=np.float32)
                    lib.ref_desk_mat_mat(desk, ctypes.byref(d), ol.p(act), K, M, ol.p(out), N)
                    total_bytes += gemv_bytes(N, K, M)
                passes += 1
                if time.perf_counter() - t0 > budget_s:
                    break
        finally:
            lib.ref_desk_close(desk)
    else:
        while True:
            for (N, K, M, codes, gains, act) in cases:
                ol.oracle_mat_mat(codes, gains, act, K, threads=cores)
                total_bytes += gemv_bytes(N, K, M)
            passes += 1
            if time.perf_counter() - t0 > budget_s:
                break
    secs = time.perf_counter() - t0
    model = ""
    for line in flags.splitlines():
        if line.startswith("model name"):
            model = line.split(":", 1)[1].strip()
            break
    return {
        "value": round(total_bytes / secs / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": kind,
        "sample": f"{passes} passes of the 8-product sweep (both shapes, M=1,2,4,8), "
                  f"{secs:.1f} s, {'ref back_mat_mat AVX2+FMA float path, pool' if kind == 'reference' else 'C restatement'}"
                  f" of {cores} threads on {model}",
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this backend runs on one GPU; multi-GPU sharding is "
                                   "not built (rows of a plane would be split across GPUs, one all-gather "
                                   "of the outputs a product)"}))
        sys.exit(2)
    from igllm_amd.backend import Backend, make_plane, synth_projection

    be = Backend(device=0, sum_limit=256, col_limit=8192, lane_limit=16)
    if args.kernel:
        kernel_loop(be, args.kernel, args.steps, args.lanes, args.shape)
        be.close()
        return
    rot = {shape: Rotation(be, *shape) for shape in SHAPES}
    acts = {}
    outs = {}
    for (N, K) in SHAPES:
        for M in LANES:
            _, _, act = synth_projection(N, K, M, seed=0)
            acts[(N, K, M)] = be.upload(act)
            outs[(N, K, M)] = be.alloc(M * N * 4)
    step_bytes = sum(gemv_bytes(N, K, M) for (N, K) in SHAPES for M in LANES)

    counter = [0]

    # Launches enqueued one ctypes call each carry ~4 us of host time; the same
    # launches recorded once and replayed (igl_record_*: no host launch each)
    # time the kernels themselves.
    def replayed(enqueue, count=2 * COPIES):
        be.record_begin()
        for i in range(count):
            enqueue(i)
        handle = be.record_end()
        try:
            be.replay_run(handle)
            be.sync()
            be.mark()
            be.replay_run(handle)
            be.mark()
            return be.marks_ms() * 1e3 / count
        finally:
            be.replay_free(handle)


    def step():
        for (N, K) in SHAPES:
            r = rot[(N, K)]
            for M in LANES:
                cp = r.planes[counter[0] % COPIES]
                counter[0] += 1
                be.gemv_dev(cp, acts[(N, K, M)], K, M, outs[(N, K, M)], N)

    for _ in range(args.warmup):
        step()
    be.sync()
    # The timed region: the K steps enqueued one ctypes call a launch (the
    # host's ~4 us a call bounds the short products), and the same K steps
    # recorded once and replayed (the GPU's own time; `value`).
    be.mark()
    for _ in range(args.steps):
        step()
    be.mark()
    enqueued_ms_per_step = be.marks_ms() / args.steps
    be.record_begin()
    for _ in range(args.steps):
        step()
    steps_replay = be.record_end()
    try:
        be.replay_run(steps_replay)  # untimed: every copy's first read of this pass
        be.sync()
        be.mark()
        be.replay_run(steps_replay)
        be.mark()
        ms_total = be.marks_ms()
    finally:
        be.replay_free(steps_replay)
    ms_per_step = ms_total / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    # ---- dominant kernel: decode GEMV M=1, 8192 x 2048, on rotating copies.
    N, K = SHAPES[0]
    r = rot[(N, K)]
    launches = 400
    for i in range(20):
        be.gemv_dev(r.planes[i % COPIES], acts[(N, K, 1)], K, 1, outs[(N, K, 1)], N)
    be.sync()
    be.mark()
    for i in range(launches):
        be.gemv_dev(r.planes[i % COPIES], acts[(N, K, 1)], K, 1, outs[(N, K, 1)], N)
    be.mark()
    gemv_enq_us = be.marks_ms() * 1e3 / launches
    gemv_algo = gemv_bytes(N, K, 1)
    prof = gemv_m1_profile(gemv_algo)

    # ---- the read floor: a kernel that only reads the same bytes once (16-byte
    # loads, two a thread), over as many rotated buffers, launched the same way.
    floor_bufs = [be.alloc(gemv_algo) for _ in range(COPIES)]
    for i in range(20):
        be.read_floor_dev(floor_bufs[i % COPIES], gemv_algo)
    be.sync()
    be.mark()
    for i in range(launches):
        be.read_floor_dev(floor_bufs[i % COPIES], gemv_algo)
    be.mark()
    floor_us = be.marks_ms() * 1e3 / launches

    gemv_replayed_us = replayed(lambda i: be.gemv_dev(r.planes[i % COPIES], acts[(N, K, 1)], K, 1,
                                                      outs[(N, K, 1)], N), launches)
    gemv_us = gemv_replayed_us
    gemv_gbps = gemv_algo / (gemv_us * 1e-6) / 1e9
    floor_replayed_us = replayed(lambda i: be.read_floor_dev(floor_bufs[i % COPIES], gemv_algo))
    for b in floor_bufs:
        b.free()
    read_floor = {"enqueued_us": round(floor_us, 3), "replayed_us": round(floor_replayed_us, 3),
                  "replayed_GBps": round(gemv_algo / (floor_replayed_us * 1e-6) / 1e9, 1),
                  "replayed_frac_of_peak": round(gemv_algo / (floor_replayed_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                  "gemv_replayed_us": round(gemv_replayed_us, 3),
                  "gemv_replayed_frac_of_peak": round(gemv_algo / (gemv_replayed_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                  "gemv_frac_of_floor": round(floor_replayed_us / gemv_replayed_us, 4),
                  "note": "read_floor_kernel: the same byte count read once and nothing else (16-byte "
                          f"loads, two a thread), rotated over {COPIES} buffers; 'replayed' = "
                          f"{2 * COPIES} launches recorded once and replayed, no host launch each"}

    # ---- per-config GEMV rates (same rotation), for the record.
    sweep = {}
    for (N, K) in SHAPES:
        for M in LANES:
            rr = rot[(N, K)]
            for i in range(10):
                be.gemv_dev(rr.planes[i % COPIES], acts[(N, K, M)], K, M, outs[(N, K, M)], N)
            be.sync()
            be.mark()
            for i in range(100):
                be.gemv_dev(rr.planes[i % COPIES], acts[(N, K, M)], K, M, outs[(N, K, M)], N)
            be.mark()
            enq_us = be.marks_ms() * 1e3 / 100
            us = replayed(lambda i: be.gemv_dev(rr.planes[i % COPIES], acts[(N, K, M)], K, M, outs[(N, K, M)], N))
            sweep[f"{N}x{K}_M{M}"] = {"us": round(us, 3),
                                      "GBps": round(gemv_bytes(N, K, M) / (us * 1e-6) / 1e9, 1),
                                      "enqueued_us": round(enq_us, 3)}

    # ---- prefill GEMM, bf16 in/out, M in {64, 256, 1024, 2048} lanes (both
    # shapes; BASELINE's prefill config), timed replayed (the GEMM launches
    # recorded once: no host launch each).  From 256 lanes the bound is the
    # MFMA peak; at 64 lanes the product is below the ridge (182 FLOP a byte
    # against ~312 for bf16), so it is also quoted against the HBM roof.
    prefill = {}
    for (N, K) in SHAPES:
        for M in (64, 256, 1024, 2048):
            a = be.alloc(M * K * 2)
            c = be.alloc(M * N * 2)
            rng = np.random.default_rng(0)
            a.put((rng.normal(size=M * K).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16))
            planes = rot[(N, K)].planes
            for i in range(3):
                be.gemm_bf16_dev(planes[i % COPIES], a, K, M, c, N)
            be.sync()
            reps = 20 if M >= 1024 else 2 * COPIES
            us = replayed(lambda i: be.gemm_bf16_dev(planes[i % COPIES], a, K, M, c, N), reps)
            tflops = 2.0 * M * N * K / (us * 1e-6) / 1e12
            nbytes = N * K // 2 + N * (K // 32) * 4 + 2 * M * (K + N)
            entry = {"us": round(us, 2), "TFLOPs": round(tflops, 1),
                     "frac_of_mfma_peak": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)}
            if M == 64:
                entry["GBps"] = round(nbytes / (us * 1e-6) / 1e9, 1)
                entry["frac_of_hbm_peak"] = round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)
            prefill[f"{N}x{K}_M{M}"] = entry
            a.free()
            c.free()

    # ---- calibrated prefill (enter_gain, one gain a row): fp32 lanes through
    # plane_lift_dev, the MFMA GEMM on levels and unit gains plus the row close.
    from igllm_amd.backend import make_plane as _make_plane
    for name, (N, K, bits) in {"calibrated_u4_8192x2048_M2048": (8192, 2048, 4),
                               "calibrated_u2_6144x1536_M2048": (6144, 1536, 2)}.items():
        M = 2048
        rng = np.random.default_rng(2)
        codes = rng.integers(0, 256, size=(N, K * bits // 8), dtype=np.uint8)
        gains = np.abs(rng.normal(0, 0.02, size=(N, 1))).astype(np.float32)
        cp = be.attach(_make_plane(codes, gains, K, group_size=K, bits=bits))
        cp.plane.enter_gain = 2.5 / 127
        cp.plane.leave_gain = 0.02
        a = be.upload(rng.normal(size=(M, K)).astype(np.float32))
        c = be.alloc(M * N * 4)
        for _ in range(3):
            be.plane_lift_dev(cp, a, K, M, c, N)
        be.sync()
        be.mark()
        reps = 20
        for _ in range(reps):
            be.plane_lift_dev(cp, a, K, M, c, N)
        be.mark()
        us = be.marks_ms() * 1e3 / reps
        tops = 2.0 * M * N * K / (us * 1e-6) / 1e12
        prefill[name] = {"us": round(us, 2), "TOPs": round(tops, 1),
                         "frac_of_i8_mfma_peak": round(tops / MFMA_I8_PEAK_TOPS, 4),
                         "note": "fp32 in/out; the level pass (act_level_kernel) and the int8 MFMA GEMM with "
                                 "the row close and leave grid (gemm_level_kernel), against the int8 "
                                 "peak (5.0 POP/s)"}
        a.free()
        c.free()
        be.detach(cp)

    # ---- decode attention, 8 q heads / 1 KV head / d=256, L=16384, int8 bytes.
    L, head, rings = 16384, 256, ATTEND_COPIES
    rng = np.random.default_rng(1)
    ring_bytes = L * head
    kb = be.alloc(ring_bytes * rings)
    vb = be.alloc(ring_bytes * rings)
    block = rng.integers(0, 256, size=ring_bytes, dtype=np.uint8)
    for i in range(rings):
        kb.put(block, i * ring_bytes)
        vb.put(block[::-1].copy(), i * ring_bytes)
    q = be.upload(rng.normal(size=(8, head)).astype(np.float32))
    o = be.alloc(8 * head * 4)
    lib, desk = be.lib, be.desk
    import ctypes

    def attend(i):
        code = lib.igl_attend_dev(ctypes.byref(desk), kb.ptr + (i % rings) * ring_bytes,
                                  vb.ptr + (i % rings) * ring_bytes, 1, 4.0 / 127, 4.0 / 127, L, 1,
                                  8, head, q.ptr, 0, L, 1.0 / 16, o.ptr)
        if code != 0:
            raise RuntimeError(f"attend: {code}")

    for i in range(5):
        attend(i)
    be.sync()
    be.mark()
    reps = 100
    for i in range(reps):
        attend(i)
    be.mark()
    att_enq_us = be.marks_ms() * 1e3 / reps
    att_us = replayed(attend, 2 * rings)
    att_bytes = 2 * L * head + 2 * 8 * head * 4
    attention = {"L": L, "us": round(att_us, 2),
                 "GBps": round(att_bytes / (att_us * 1e-6) / 1e9, 1),
                 "frac_of_hbm_peak": round(att_bytes / (att_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                 "enqueued_us": round(att_enq_us, 2),
                 "note": f"int8 K/V rings rotated over {rings} copies (past the MALL); the chunk kernel and "
                         "the fold, recorded once and replayed (enqueued_us: one ctypes call each)"}
    kb.free()
    vb.free()
    # the decode step's sliding-window call: 512 positions of 256 dims, e4m3,
    # at position 2300 of a 2560-slot ring (rotated past the MALL)
    Ls, win, srings = 2560, 512, 200
    ring_s = Ls * head
    ks = be.alloc(ring_s * srings)
    vs = be.alloc(ring_s * srings)
    blk = rng.integers(0, 256, size=ring_s, dtype=np.uint8) & 0xBF  # no 0x7F / 0xFF codes
    for i in range(srings):
        ks.put(blk, i * ring_s)
        vs.put(blk[::-1].copy(), i * ring_s)

    def slide(i):
        code = lib.igl_attend_lanes_dev(ctypes.byref(desk), ks.ptr + (i % srings) * ring_s,
                                        vs.ptr + (i % srings) * ring_s, 0, 0.02, 0.02, Ls, 1, 8, head,
                                        q.ptr, 8 * head, 2300, win, 1, 1.0, o.ptr)
        if code != 0:
            raise RuntimeError(f"attend sliding: {code}")

    for i in range(5):
        slide(i)
    be.sync()
    sl_us = replayed(slide, srings)
    attention["sliding_512"] = {"us": round(sl_us, 2),
                                "note": "one lane at position 2300, window 512, head 256, e4m3 rings rotated "
                                        f"over {srings} copies; chunk kernel and fold, replayed"}
    ks.free()
    vs.free()

    kinds = kinds_leg(be)
    e2e = None if args.no_e2e else e2e_decode(be, cpu=not args.no_cpu)
    cpu = None if args.no_cpu else cpu_baseline()
    if not args.no_cpu:
        attention["cpu_baseline"] = cpu_attention()
        prefill["cpu_baseline"] = cpu_prefill()

    line = {
        "metric": "decode tok/s + int4 GEMV HBM GB/s (% of peak) + prefill GEMM % MFMA, 1 GPU",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "enqueued_ms_per_step": round(enqueued_ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xfp32",
        "data": "synthetic (seeded splitmix64/xoshiro256**, int4 uniform -8..7, |N(0,0.02)| gains, "
                "N(0,1) activations)",
        "config": {"workload": "small-lane int4 g32 GEMV sweep: N=8192,K=2048 and N=2048,K=8192, "
                               "M in {1,2,4,8}, fp32 activations, weights rotated over "
                               f"{COPIES} copies per shape",
                   "step_bytes": step_bytes},
        "roofline": {"bound": "hbm", "kernel": "gemv_q4_dot_kernel<1, 2, 1, 1, false> 8192x2048 M=1",
                     "achieved": round(gemv_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gemv_gbps / HBM_PEAK_GBPS, 4),
                     "traffic": prof["traffic"] if prof else None,
                     "profile": prof,
                     "algorithmic_bytes": gemv_algo, "avg_launch_us": round(gemv_us, 3),
                     "avg_launch_us_enqueued": round(gemv_enq_us, 3),
                     "timing": f"{launches} launches on rotated copies recorded once and replayed, HIP events "
                               "on the desk's stream; enqueued: the same launches one ctypes call each",
                     "read_floor": read_floor},
        "cpu_baseline": cpu,
        "gemv_sweep": sweep,
        "prefill_gemm": prefill,
        "decode_attention": attention,
        "other_plane_kinds_m1": kinds,
        "decode_tok_s": None if not e2e else e2e["precise"]["decode_tok_s"],
        "e2e": e2e,
    }
    print(json.dumps(line))
    be.close()


if __name__ == "__main__":
    main()
