"""The host code's launches, audited on the CPU (tests/audit).

The backend's own host code (back_hip.c, igl_engine.c and the host side of
every .hip file, built with --cuda-host-only) runs against a stand-in HIP
runtime that records every allocation and checks every launch: each grid and
block against gfx950's limits, and each buffer handed to a launcher, at the
extent the launcher's arguments imply, against the allocation it lies in
(tests/audit/audit_stub.c).  No kernel runs and no value is computed; what is
proven is that the engine never hands a kernel a pointer, stride, lane count or
workspace that reaches past what it allocated.

Cases:
  * e2b-decode: the synthetic E2B checkpoint at lane limit 16 on the precise
    GEMV path, the 2048-id prime in 128 passes of 16 lanes, then eager and
    graph-captured steps (bench.py's decode trace workload);
  * e2b-fast: the same prime as one 2048-lane pass on the GEMM path;
  * small-guess: guess blocks of every lane count up to the limit, kept in part;
  * packed: zero-point planes in the compressed-tensors pack, both paths;
  * planted: a buffer one float short, a pointer past its allocation and a
    workspace below the launcher's need must each be reported.
"""
import os
import shutil
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
AUDIT_DIR = os.path.join(HERE, "audit")
AUDIT = os.path.join(AUDIT_DIR, "_build", "audit")


@pytest.fixture(scope="module")
def audit_bin():
    if shutil.which("make") is None or not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc or make absent")
    r = subprocess.run(["make", "-s", "-j8", "-C", AUDIT_DIR], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    return AUDIT


def run_case(audit_bin, case):
    root = "/dev/shm" if os.path.isdir("/dev/shm") else tempfile.gettempdir()
    folder = tempfile.mkdtemp(prefix=f"igl_audit_{case}_", dir=root)
    try:
        r = subprocess.run([audit_bin, case, folder], capture_output=True, text=True, timeout=900)
    finally:
        shutil.rmtree(folder, ignore_errors=True)
    print(r.stdout.strip())
    print(r.stderr[-3000:])
    return r


@pytest.mark.parametrize("case", ["planted", "small-guess", "packed", "e2b-decode", "e2b-fast"])
def test_launches_stay_inside_their_allocations(audit_bin, case):
    r = run_case(audit_bin, case)
    assert r.returncode == 0, r.stdout + r.stderr[-3000:]
    last = r.stdout.strip().splitlines()[-1]
    launches = int(last.split("launches ")[1].split(",")[0])
    if case == "planted":
        assert "violations 3" in last
        assert r.stderr.count("AUDIT VIOLATION") == 3
    else:
        assert "violations 0" in last
        assert launches > 1000
