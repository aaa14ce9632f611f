"""GPU parity of the shipped export's other plane kinds against the oracle:
2-bit planes (value + 2, four codes a byte), signed I8 planes (code_flip 128,
code_bias 128), unsigned 8-bit planes, 4-bit planes with a flip, and one gain
a row (per-channel scales, G = 1), at the widths the export has them
(model/config.json module_quant_configs: MLP of layers 15-34, lm_head and
embed_tokens 2-bit; per_layer_input_gate and per_layer_projection 8-bit),
and real planes of bf16, binary16 or fp32 rows (per_layer_model_projection).

Bar: every output within relative error 1e-3 of the oracle, relative to
max(|y_ref|, rms(y_ref)), as for the 4-bit GEMV.
"""
import numpy as np
import pytest

import oracle_lib as ol
from igllm_amd.backend import BackendError, make_plane

pytestmark = pytest.mark.gpu


def rel_err(got, want):
    want = want.astype(np.float64)
    floor = np.sqrt(np.mean(want ** 2))
    return float(np.max(np.abs(got.astype(np.float64) - want) / np.maximum(np.abs(want), floor)))


def print_case(**kw):
    print("case", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def synth_kind(N, K, bits, group, lanes, seed, stride=None):
    """Uniform codes of any width (uniform bytes), |N(0, 0.02)| gains, N(0,1) x."""
    rng = np.random.default_rng(seed)
    stride = stride or ((K * bits + 7) // 8 + 15) // 16 * 16
    codes = rng.integers(0, 256, size=(N, stride), dtype=np.uint8)
    G = (K + group - 1) // group
    gains = np.abs(rng.normal(0, 0.02, size=(N, G))).astype(np.float32)
    act = rng.normal(size=(lanes, K)).astype(np.float32)
    return codes, gains, act


def run_dev(backend, cp, act, lanes, path="gemv"):
    K, N = cp.K, cp.N
    dev_act = backend.upload(act)
    dev_out = backend.alloc(lanes * N * 4)
    fn = backend.gemv_dev if path == "gemv" else backend.mat_mat_dev
    fn(cp, dev_act, K, lanes, dev_out, N)
    backend.sync()
    out = dev_out.get(np.float32, lanes * N).reshape(lanes, N)
    dev_act.free()
    dev_out.free()
    return out


KINDS = {
    "u2": dict(bits=2, code_flip=0),
    "i8": dict(bits=8, code_flip=128),
    "u8": dict(bits=8, code_flip=0),
    "u4flip": dict(bits=4, code_flip=5),
}


@pytest.mark.parametrize("kind", list(KINDS))
@pytest.mark.parametrize("N,K,group,lanes", [
    (6144, 1536, 1536, 1),   # gate/up of a 2-bit MLP layer, per-channel
    (1536, 6144, 6144, 1),   # its down projection
    (256, 1536, 1536, 1),    # per_layer_input_gate
    (1536, 256, 256, 1),     # per_layer_projection
    (1536, 256, 256, 3),
    (2048, 1536, 32, 2),     # group-32 scales
    (1000, 2048, 128, 4),
    (300, 1536, 1536, 5),
    (129, 6144, 6144, 8),
    (70, 96, 96, 1),         # K not a multiple of 64
    (33, 20480, 20480, 2),   # two K-chunks
    (64, 4096, 32, 16),
])
def test_kind_gemv(backend, kind, N, K, group, lanes):
    kw = KINDS[kind]
    print_case(test="kind_gemv", kind=kind, N=N, K=K, group=group, lanes=lanes)
    codes, gains, act = synth_kind(N, K, kw["bits"], group, lanes, seed=N + K + lanes)
    cp = backend.attach(make_plane(codes, gains, K, group_size=group, **kw))
    got = run_dev(backend, cp, act, lanes)
    want = ol.oracle_mat_mat(codes, gains, act, K, group, threads=8, bits=kw["bits"],
                             code_bias=1 << (kw["bits"] - 1), code_flip=kw["code_flip"])
    err = rel_err(got, want)
    print("rel_err", err)
    assert err <= 1e-3
    backend.detach(cp)


@pytest.mark.parametrize("kind", ["u2", "i8"])
def test_kind_table_entries(backend, kind):
    """mat_vec / mat_mat through the table (host pointers), 70 lanes."""
    kw = KINDS[kind]
    N, K, lanes = 512, 1536, 70
    print_case(test="kind_table", kind=kind, N=N, K=K, lanes=lanes)
    codes, gains, act = synth_kind(N, K, kw["bits"], K, lanes, seed=7)
    cp = backend.attach(make_plane(codes, gains, K, group_size=K, **kw))
    want = ol.oracle_mat_mat(codes, gains, act, K, K, threads=8, bits=kw["bits"],
                             code_bias=1 << (kw["bits"] - 1), code_flip=kw["code_flip"])
    got = backend.mat_mat(cp, act)
    assert rel_err(got, want) <= 1e-3
    one = backend.mat_vec(cp, act[0])
    assert np.array_equal(one, got[0])
    backend.detach(cp)


@pytest.mark.parametrize("kind", ["u2", "i8"])
@pytest.mark.parametrize("fill", ["zeros", "tiny", "subnormal", "huge", "mixed"])
def test_kind_activation_range(backend, kind, fill):
    """The digit form over units of zeros, 1e-30, subnormal and 1e30 activations."""
    kw = KINDS[kind]
    N, K = 512, 1536
    print_case(test="kind_range", kind=kind, fill=fill)
    codes, gains, act = synth_kind(N, K, kw["bits"], 32, 1, seed=11)
    if fill == "zeros":
        act[:] = 0.0
        act[0, 64:96] = np.linspace(-1, 1, 32)
    elif fill == "tiny":
        act *= 1e-30
    elif fill == "subnormal":
        act = (act * 1e-39).astype(np.float32)
    elif fill == "huge":
        act *= 1e30
    else:
        act[0, ::3] *= 1e20
        act[0, 1::7] = 0.0
    cp = backend.attach(make_plane(codes, gains, K, group_size=32, **kw))
    got = run_dev(backend, cp, act, 1)
    want = ol.oracle_mat_mat(codes, gains, act, K, 32, threads=8, bits=kw["bits"],
                             code_bias=1 << (kw["bits"] - 1), code_flip=kw["code_flip"])
    assert np.all(np.isfinite(got))
    bar = 1e-3 if fill == "subnormal" else 1e-5
    err = rel_err(got, want)
    print("rel_err", err)
    assert err <= bar
    backend.detach(cp)


def test_kind_refusals(backend):
    """Kinds the kernels do not compute are refused at attach, not emulated."""
    codes, gains, act = synth_kind(64, 96, 3, 32, 1, seed=1)
    with pytest.raises(BackendError):
        backend.attach(make_plane(codes, gains, 96, bits=3))
    codes, gains, act = synth_kind(64, 96, 8, 48, 1, seed=1)
    with pytest.raises(BackendError):
        backend.attach(make_plane(codes, gains, 96, group_size=48, bits=8))
    codes, gains, act = synth_kind(64, 96, 8, 96, 1, seed=1)
    with pytest.raises(BackendError):
        backend.attach(make_plane(codes, gains, 96, group_size=96, bits=8, code_bias=0))
    with pytest.raises(BackendError):
        backend.attach(make_plane(codes, gains, 96, group_size=96, bits=8, code_flip=256))


# ---- real planes (per_layer_model_projection: 8960 x 1536 bf16) --------------

def real_rows(N, K, real_type, seed):
    rng = np.random.default_rng(seed)
    w = rng.normal(0, 0.05, size=(N, K)).astype(np.float32)
    if real_type == ol.REAL_F32:
        return w
    if real_type == ol.REAL_F16:
        return w.astype(np.float16).view(np.uint16)
    return (w.view(np.uint32) >> 16).astype(np.uint16)


@pytest.mark.parametrize("real_type", [ol.REAL_BF16, ol.REAL_F16, ol.REAL_F32])
@pytest.mark.parametrize("N,K,lanes", [
    (8960, 1536, 1), (8960, 1536, 2), (8960, 1536, 5), (1000, 1536, 8), (300, 1536, 16),
    (3, 8, 1), (70, 72, 3), (100, 12288, 8), (77, 20000, 1),
])
def test_real_gemv(backend, real_type, N, K, lanes):
    from igllm_amd.backend import make_real_plane

    print_case(test="real_gemv", real_type=real_type, N=N, K=K, lanes=lanes)
    rows = real_rows(N, K, real_type, seed=N + K)
    act = np.random.default_rng(lanes).normal(size=(lanes, K)).astype(np.float32)
    cp = backend.attach(make_real_plane(rows, real_type))
    got = run_dev(backend, cp, act, lanes)
    want = ol.oracle_mat_mat_real(rows, real_type, act)
    err = rel_err(got, want)
    print("rel_err", err)
    assert err <= 1e-3
    backend.detach(cp)


def test_real_table_entries(backend):
    from igllm_amd.backend import make_real_plane

    N, K, lanes = 8960, 1536, 70
    print_case(test="real_table", N=N, K=K, lanes=lanes)
    rows = real_rows(N, K, ol.REAL_BF16, seed=3)
    act = np.random.default_rng(3).normal(size=(lanes, K)).astype(np.float32)
    cp = backend.attach(make_real_plane(rows, ol.REAL_BF16))
    want = ol.oracle_mat_mat_real(rows, ol.REAL_BF16, act)
    got = backend.mat_mat(cp, act)
    assert rel_err(got, want) <= 1e-3
    # one lane takes the whole row in one K-chunk, eight lanes two: not bit-equal
    assert rel_err(backend.mat_vec(cp, act[0])[None], want[:1]) <= 1e-3
    backend.detach(cp)


# ---- zero points (the compressed-tensors pack's weight_zero_point) ----------

@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("N,K,group,lanes", [
    (1536, 512, 32, 1), (2048, 512, 32, 3), (512, 2048, 128, 8), (300, 1536, 1536, 2),
    (1024, 512, 32, 16), (512, 1024, 32, 64), (1536, 512, 32, 300), (70, 96, 32, 65),
])
def test_zero_point_planes(backend, bits, N, K, group, lanes):
    """Planes with a zero point a row and group, every value of the code
    range's signed half, against the oracle (kern_row_code's
    gain (dot - (bias + zero) sum), pinned to the reference's plain build):
    below 64 lanes the zero-point GEMV, from 64 lanes 4-bit planes take the
    MFMA GEMM with the zero folded into the weight operand's subtrahend and
    2/8-bit planes the GEMV; both routes through igl_mat_mat_dev and, for
    the GEMV, igl_gemv_dev."""
    print_case(test="zero_points", bits=bits, N=N, K=K, group=group, lanes=lanes)
    r = np.random.default_rng(bits * 1000 + N + lanes)
    codes, gains, act = synth_kind(N, K, bits, group, lanes, seed=bits + N + lanes)
    half = 1 << (bits - 1)
    zeros = r.integers(-half, half, size=gains.shape).astype(np.int8)
    cp = backend.attach(make_plane(codes, gains, K, group_size=group, bits=bits, zeros=zeros))
    want = ol.oracle_mat_mat(codes, gains, act, K, group, threads=8, bits=bits, code_bias=half,
                             zeros=zeros)
    got = run_dev(backend, cp, act, lanes, path="mat_mat")
    err = rel_err(got, want)
    print("rel_err mat_mat", err)
    assert err <= 1e-3
    got = run_dev(backend, cp, act, lanes, path="gemv")
    err = rel_err(got, want)
    print("rel_err gemv", err)
    assert err <= 1e-3
    backend.detach(cp)


def test_zero_point_bf16_gemm(backend):
    """bf16 prefill on a 4-bit zero-point plane: the GEMM's bf16 output within
    its rounding of the float64 closed form."""
    N, K, M = 1024, 2048, 256
    r = np.random.default_rng(77)
    codes, gains, act = synth_kind(N, K, 4, 32, M, seed=77)
    zeros = r.integers(-8, 8, size=gains.shape).astype(np.int8)
    cp = backend.attach(make_plane(codes, gains, K, bits=4, zeros=zeros))
    u = act.view(np.uint32).astype(np.uint64)
    a16 = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    a32 = (a16.astype(np.uint32) << 16).view(np.float32)
    dev_a = backend.upload(a16)
    dev_c = backend.alloc(M * N * 2)
    backend.gemm_bf16_dev(cp, dev_a, K, M, dev_c, N)
    backend.sync()
    got = (dev_c.get(np.uint16, M * N).astype(np.uint32) << 16).view(np.float32).reshape(M, N).astype(np.float64)
    nib = np.stack([codes[:, :K // 2] & 15, codes[:, :K // 2] >> 4], axis=-1).reshape(N, K).astype(np.float64)
    w = (nib - 8 - np.repeat(zeros.astype(np.float64), 32, axis=1)) * np.repeat(gains.astype(np.float64), 32, axis=1)
    want = a32.astype(np.float64) @ w.T
    rms = float(np.sqrt(np.mean(want ** 2)))
    assert float((np.abs(got - want) - (2.0 ** -8 * np.abs(want) + 1e-4 * rms)).max()) <= 0.0
    dev_a.free()
    dev_c.free()
    backend.detach(cp)
