"""ctypes access to the checker: oracle/liboracle.so (the C restatement) and,
where it was built, oracle/_ref (the reference's own app_core.c).

Test infrastructure only.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_PATH = os.path.join(ROOT, "oracle", "liboracle.so")
REF_PLAIN_PATH = os.path.join(ROOT, "oracle", "_ref", "libigl_ref_plain.so")
REF_TUNED_PATH = os.path.join(ROOT, "oracle", "_ref", "libigl_ref_tuned.so")
REF_LEVEL_PATH = os.path.join(ROOT, "oracle", "_ref", "libigl_ref_level.so")
REF_DROPIN_PATH = os.path.join(ROOT, "oracle", "_ref", "libigl_ref_dropin.so")

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_Z = ctypes.c_size_t


class PlaneDesc(ctypes.Structure):
    """oracle_plane / ref_plane_desc (same layout)."""

    _fields_ = [
        ("row_count", _I),
        ("col_count", _I),
        ("code_data", _P),
        ("row_stride", _Z),
        ("gain_data", _P),
        ("bias_data", _P),
        ("bit_count", _I),
        ("code_bias", _I),
        ("code_flip", _I),
        ("group_size", _I),
        ("group_count", _I),
    ]


ORACLE_SIGS = {
    "oracle_pack_read": (ctypes.c_uint32, [_P, _Z, _I]),
    "oracle_plane_row": (None, [ctypes.POINTER(PlaneDesc), _I, _P]),
    "oracle_quant_step": (_F, [_F, _F]),
    "oracle_group_sum": (None, [ctypes.POINTER(PlaneDesc), _P, _P]),
    "oracle_dot_code": (_F, [_P, _I, _I, _P, _I, _I]),
    "oracle_row_code": (_F, [ctypes.POINTER(PlaneDesc), _I, _P, _P]),
    "oracle_mat_mat": (_I, [ctypes.POINTER(PlaneDesc), _P, _I, _I, _P, _I, _I]),
    "oracle_mat_mat_real": (_I, [_P, _I, _I, _I, _P, _I, _I, _P, _I]),
    "oracle_mat_mat_level": (_I, [ctypes.POINTER(PlaneDesc), _P, _I, _I, _F, _P, _I]),
    "oracle_pack8": (_F, [_F]),
    "oracle_code8": (ctypes.c_uint8, [_F]),
    "oracle_real8": (_F, [ctypes.c_uint8]),
    "oracle_grid_fill8": (None, [_P, _F]),
    "oracle_code_i8": (ctypes.c_uint8, [_F, _F]),
    "oracle_grid_fill_i8": (None, [_P, _F]),
    "oracle_exp_near": (_F, [_F]),
    "oracle_soft_max": (None, [_P, _I]),
    "oracle_attend": (None, [_P, _P, _P, _P, _I, _I, _I, _P, _I, _I, _I, _I, _I, _F, _P, _P]),
    "oracle_encode8_many": (None, [_P, _Z, _F, _P]),
    "oracle_encode_i8_many": (None, [_P, _Z, _F, _P]),
    "oracle_norm_rms": (None, [_P, _P, _I, _F, _P]),
    "oracle_gelu_gate": (None, [_P, _P, _I]),
    "oracle_rope_turn": (None, [_P, _I, _P, _P]),
    "oracle_clock": (ctypes.c_double, []),
}

REF_SIGS = {
    "ref_flavor": (ctypes.c_char_p, []),
    "ref_pack_read": (ctypes.c_uint32, [_P, _Z, _I]),
    "ref_zero_read": (_I, [_P, _I, _I, _I, _I]),
    "ref_plane_row": (None, [ctypes.POINTER(PlaneDesc), _I, _P]),
    "ref_desk_open": (_P, [_I, _I, _I]),
    "ref_desk_close": (None, [_P]),
    "ref_desk_mat_mat": (None, [_P, ctypes.POINTER(PlaneDesc), _P, _I, _I, _P, _I]),
    "ref_desk_mat_mat_real": (None, [_P, _P, _I, _I, _I, _P, _I, _I, _P, _I]),
    "ref_desk_mat_mat_step": (None, [_P, ctypes.POINTER(PlaneDesc), _F, _P, _I, _I, _P, _I]),
    "ref_level_live": (_I, [_P]),
    "ref_cache_pack8": (_F, [_F]),
    "ref_cache_code8": (ctypes.c_uint8, [_F]),
    "ref_cache_real8": (_F, [ctypes.c_uint8]),
    "ref_cache_grid_fill": (None, [_P, _F]),
    "ref_exp_near": (_F, [_F]),
    "ref_soft_max": (None, [_P, _I]),
    "ref_quant_step": (_F, [_F, _F]),
    "ref_attend": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _P, _I, _I, _I, _I, _I, _P]),
}


def _load(path, sigs):
    lib = ctypes.CDLL(path)
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_cache = {}


def oracle():
    if "oracle" not in _cache:
        _cache["oracle"] = _load(ORACLE_PATH, ORACLE_SIGS)
    return _cache["oracle"]


def host_has_vnni() -> bool:
    try:
        flags = open("/proc/cpuinfo").read()
    except OSError:
        return False
    return all(f" {f}" in flags for f in ("avx512f", "avx512bw", "avx512dq", "avx512vl", "avx512_vnni",
                                          "gfni"))


def ref(kind: str = "plain"):
    """The compiled reference harness (plain, tuned or level), or None where it
    was not built, or for the level build, where this host lacks AVX-512 VNNI."""
    path = {"plain": REF_PLAIN_PATH, "tuned": REF_TUNED_PATH, "level": REF_LEVEL_PATH}[kind]
    if not os.path.exists(path) or (kind == "level" and not host_has_vnni()):
        return None
    key = "ref_" + kind
    if key not in _cache:
        _cache[key] = _load(path, REF_SIGS)
    return _cache[key]


def p(a: np.ndarray) -> int:
    return a.ctypes.data


def plane_desc(codes: np.ndarray, gains: np.ndarray, K: int, group_size: int = 32, bits: int = 4,
               code_bias: int = 8, code_flip: int = 0, zeros: np.ndarray | None = None) -> PlaneDesc:
    d = PlaneDesc()
    d.row_count = codes.shape[0]
    d.col_count = K
    d.code_data = p(codes)
    d.row_stride = codes.shape[1]
    d.gain_data = p(gains)
    d.bias_data = None if zeros is None else p(zeros)
    d.bit_count = bits
    d.code_bias = code_bias
    d.code_flip = code_flip
    d.group_size = group_size
    d.group_count = gains.shape[1]
    return d


def oracle_mat_mat(codes, gains, act, K, group_size=32, threads=1, **kw) -> np.ndarray:
    codes = np.ascontiguousarray(codes)
    gains = np.ascontiguousarray(gains, dtype=np.float32)
    act = np.ascontiguousarray(act, dtype=np.float32)
    lanes = act.shape[0]
    out = np.empty((lanes, codes.shape[0]), dtype=np.float32)
    d = plane_desc(codes, gains, K, group_size, **kw)
    rc = oracle().oracle_mat_mat(ctypes.byref(d), p(act), act.shape[1], lanes, p(out), codes.shape[0],
                                 threads)
    assert rc == 0
    return out


def ref_mat_mat(lib, codes, gains, act, K, group_size=32, threads=1, **kw) -> np.ndarray:
    codes = np.ascontiguousarray(codes)
    gains = np.ascontiguousarray(gains, dtype=np.float32)
    act = np.ascontiguousarray(act, dtype=np.float32)
    lanes = act.shape[0]
    out = np.empty((lanes, codes.shape[0]), dtype=np.float32)
    d = plane_desc(codes, gains, K, group_size, **kw)
    desk = lib.ref_desk_open(threads, gains.shape[1], K)
    assert desk
    try:
        lib.ref_desk_mat_mat(desk, ctypes.byref(d), p(act), act.shape[1], lanes, p(out), codes.shape[0])
    finally:
        lib.ref_desk_close(desk)
    return out


REAL_F32, REAL_F16, REAL_BF16 = 1, 2, 3  # the reference's store_type values


def quant_step(x, step):
    """quant_step (app_core.c:1930-1940) through the oracle, element by element."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    f = oracle().oracle_quant_step
    return np.array([f(float(v), step) for v in x.ravel()], dtype=np.float32).reshape(x.shape)


def oracle_mat_mat_level(codes, gains, act, K, group_size, step, **kw) -> np.ndarray:
    codes = np.ascontiguousarray(codes)
    gains = np.ascontiguousarray(gains, dtype=np.float32)
    act = np.ascontiguousarray(act, dtype=np.float32)
    out = np.empty((act.shape[0], codes.shape[0]), dtype=np.float32)
    d = plane_desc(codes, gains, K, group_size, **kw)
    rc = oracle().oracle_mat_mat_level(ctypes.byref(d), p(act), act.shape[1], act.shape[0], step, p(out),
                                       codes.shape[0])
    assert rc == 0
    return out


def ref_mat_mat_step(lib, codes, gains, act, K, group_size, step, threads=1, **kw) -> np.ndarray:
    codes = np.ascontiguousarray(codes)
    gains = np.ascontiguousarray(gains, dtype=np.float32)
    act = np.ascontiguousarray(act, dtype=np.float32)
    out = np.empty((act.shape[0], codes.shape[0]), dtype=np.float32)
    d = plane_desc(codes, gains, K, group_size, **kw)
    desk = lib.ref_desk_open(threads, gains.shape[1], K)
    assert desk
    try:
        assert lib.ref_level_live(desk) == 1
        lib.ref_desk_mat_mat_step(desk, ctypes.byref(d), step, p(act), act.shape[1], act.shape[0], p(out),
                                  codes.shape[0])
    finally:
        lib.ref_desk_close(desk)
    return out


def oracle_mat_mat_real(real, real_type, act) -> np.ndarray:
    """A real plane [N, K] (float32, or uint16 bits of binary16 / bf16) times lanes of x."""
    real = np.ascontiguousarray(real)
    act = np.ascontiguousarray(act, dtype=np.float32)
    N, K = real.shape
    out = np.empty((act.shape[0], N), dtype=np.float32)
    rc = oracle().oracle_mat_mat_real(p(real), real_type, N, K, p(act), K, act.shape[0], p(out), N)
    assert rc == 0
    return out


def ref_mat_mat_real(lib, real, real_type, act, threads=1) -> np.ndarray:
    real = np.ascontiguousarray(real)
    act = np.ascontiguousarray(act, dtype=np.float32)
    N, K = real.shape
    out = np.empty((act.shape[0], N), dtype=np.float32)
    desk = lib.ref_desk_open(threads, 1, K)
    assert desk
    try:
        lib.ref_desk_mat_mat_real(desk, p(real), real_type, N, K, p(act), K, act.shape[0], p(out), N)
    finally:
        lib.ref_desk_close(desk)
    return out


def oracle_attend(key_store, value_store, key_grid, value_grid, cache_span, kv_width, kv_index,
                  query, head_first, group_share, head_size, place_start, span_count,
                  score_scale=1.0):
    heads = query.shape[0]
    out = np.zeros((heads, head_size), dtype=np.float32)
    room = np.empty(group_share * span_count, dtype=np.float32)
    oracle().oracle_attend(p(key_store), p(value_store), p(key_grid), p(value_grid), cache_span,
                           kv_width, kv_index, p(query), head_first, group_share, head_size,
                           place_start, span_count, score_scale, p(out), p(room))
    return out


def grid8(scale: float) -> np.ndarray:
    g = np.empty(256, dtype=np.float32)
    oracle().oracle_grid_fill8(p(g), scale)
    return g


def grid_i8(scale: float) -> np.ndarray:
    g = np.empty(256, dtype=np.float32)
    oracle().oracle_grid_fill_i8(p(g), scale)
    return g


def encode(values: np.ndarray, scale: float, fmt: int) -> np.ndarray:
    """cache_lay's bytes for `values` at `scale`: fmt 0 = e4m3 (code8 of v / scale),
    1 = int8 (rint(v / scale) clamped to +-127)."""
    flat = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(flat.shape, dtype=np.uint8)
    fn = oracle().oracle_encode8_many if fmt == 0 else oracle().oracle_encode_i8_many
    fn(p(flat), flat.size, scale, p(out))
    return out
