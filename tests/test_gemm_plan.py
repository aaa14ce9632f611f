"""CPU check of the prefill GEMM's launch plan: the tile form, the K slices
across workgroups and the workspace the callers allocate for them.

The launcher picks one of six tile forms and, on long rows (K >= 4096) at a
few hundred lanes or less, splits K across workgroups into 2, 4 or 8 slices
whose fp32 partial tiles live in the workspace.  This replays a grid of
(M, N, K) shapes through igl_gemm_form / igl_gemm_slices /
igl_gemm_work_bytes and checks what the kernels assume of them: every K split
(inside the workgroup and across workgroups) divides K, the slice count is a
power of two that keeps the split's workgroups within one round of the 256
CUs, and the workspace holds the binary16 activation copy, the row scales and
every slice's partial tile.  Pure host arithmetic: no device is touched.
"""
import ctypes

import pytest

# (K split inside the workgroup, tile rows n, tile lanes m) of forms 0-5, one-
# and two-term activations (the two-term 16 x 64 form splits K in four).
FORMS = {1: [(1, 256, 256), (2, 128, 128), (4, 64, 64), (4, 32, 64), (8, 16, 64), (2, 64, 64)],
         2: [(1, 256, 256), (2, 128, 128), (4, 64, 64), (4, 32, 64), (4, 16, 64), (2, 64, 64)]}
STEP_K = 64


@pytest.fixture(scope="module")
def lib():
    from igllm_amd import native

    lib = native.load()
    for name in ("igl_gemm_form", "igl_gemm_slices", "igl_gemm_fits"):
        getattr(lib, name).restype = ctypes.c_int
        getattr(lib, name).argtypes = [ctypes.c_int] * (3 if name == "igl_gemm_fits" else 4)
    lib.igl_gemm_work_bytes.restype = ctypes.c_size_t
    lib.igl_gemm_work_bytes.argtypes = [ctypes.c_int] * 4
    return lib


def tiles(N, M, n, m):
    return ((N + n - 1) // n) * ((M + m - 1) // m)


SHAPES = [(N, K) for N in (16, 300, 1536, 2048, 6144, 8192, 262144)
          for K in (32, 96, 640, 1056, 1536, 2048, 4096, 4224, 6144, 8192, 12288, 16384)]
LANES = (64, 65, 100, 128, 192, 256, 300, 512, 1024, 2047)


@pytest.mark.parametrize("terms", [1, 2])
def test_plan_divides_k_and_sizes_the_work(lib, terms):
    split_seen = set()
    for N, K in SHAPES:
        for M in LANES:
            assert lib.igl_gemm_fits(M, N, K)
            form = lib.igl_gemm_form(M, N, K, terms)
            slices = lib.igl_gemm_slices(M, N, K, terms)
            ks, n, m = FORMS[terms][form]
            assert 0 <= form <= 5
            assert slices in (1, 2, 4, 8), (M, N, K, slices)
            kp = (K + STEP_K - 1) // STEP_K * STEP_K
            if ks > 1:
                assert K % (STEP_K * ks) == 0, (M, N, K, form)
            if slices > 1:
                split_seen.add(slices)
                # slices only on long rows, on the 64 x 64 eight-wave form, each
                # slice a whole number of stages, one round of 256 workgroups
                assert K >= 4096 and form == 2
                assert K % (slices * STEP_K * ks) == 0
                assert tiles(N, M, n, m) * slices <= 256
            need = kp * M * 2 * terms + M * 4 + (slices * M * N * 4 if slices > 1 else 0)
            have = lib.igl_gemm_work_bytes(M, N, K, terms)
            assert have >= need, (M, N, K, have, need)
    assert split_seen == {2, 4, 8}


def test_two_a_cu_form_only_past_one_round(lib):
    """Form 5 (64 x 64 tiles, two four-wave workgroups a CU) where the 64 x 64
    tiles pass one round of 256 and the wide forms do not fill the CUs, or
    where K is a multiple of 128 but not of 256; never on long rows."""
    for N, K in SHAPES:
        for M in LANES:
            form = lib.igl_gemm_form(M, N, K, 1)
            if form != 5:
                continue
            assert K < 4096 or K % 256
            assert tiles(N, M, 64, 64) > 256 or K % 256
            assert K % 128 == 0


def test_bench_shapes(lib):
    """The bench's prefill shapes keep the plans their measured figures were
    taken on."""
    want = {(64, 8192, 2048): (3, 1), (256, 8192, 2048): (5, 1), (1024, 8192, 2048): (1, 1),
            (2048, 8192, 2048): (0, 1), (64, 2048, 8192): (2, 8), (256, 2048, 8192): (2, 2),
            (1024, 2048, 8192): (2, 1), (2048, 2048, 8192): (1, 1)}
    for (M, N, K), plan in want.items():
        assert (lib.igl_gemm_form(M, N, K, 1), lib.igl_gemm_slices(M, N, K, 1)) == plan, (M, N, K)
