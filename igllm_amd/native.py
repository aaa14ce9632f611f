"""ctypes binding of libigl_hip.so, the gfx950 backend's C ABI
(include/igl_backend.h).

The library is built in-tree (igllm_amd/libigl_hip.so) by
``make -C igllm_amd/csrc``.  Loading fails loudly when it is missing: there is
no CPU path behind these names.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libigl_hip.so")

IGL_OKAY = 0
IGL_FAIL_ARGUMENT = -1
IGL_FAIL_MEMORY = -2
IGL_FAIL_SUPPORT = -6
IGL_FAIL_STATE = -7
IGL_FAIL_DEVICE = -8

IGL_PLANE_CODE = 2
IGL_STORE_F32 = 1
IGL_STORE_F16 = 2
IGL_STORE_BF16 = 3
IGL_PLANE_REAL = 1
IGL_CACHE_E4M3 = 0
IGL_CACHE_INT8 = 1

c_float_p = ctypes.POINTER(ctypes.c_float)
c_u8_p = ctypes.POINTER(ctypes.c_uint8)


class Plane(ctypes.Structure):
    """`igl_plane`: the reference's `plane` (app_core.c:1775-1795) plus a device handle."""

    _fields_ = [
        ("form", ctypes.c_int),
        ("row_count", ctypes.c_int),
        ("col_count", ctypes.c_int),
        ("real_data", ctypes.c_void_p),
        ("real_type", ctypes.c_int),
        ("code_data", ctypes.c_void_p),
        ("row_stride", ctypes.c_size_t),
        ("gain_data", ctypes.c_void_p),
        ("gain_type", ctypes.c_int),
        ("bias_data", ctypes.c_void_p),
        ("bit_count", ctypes.c_int),
        ("code_bias", ctypes.c_int),
        ("code_flip", ctypes.c_int),
        ("group_size", ctypes.c_int),
        ("group_count", ctypes.c_int),
        ("enter_gain", ctypes.c_float),
        ("leave_gain", ctypes.c_float),
        ("own_block", ctypes.c_void_p),
        ("device", ctypes.c_void_p),
    ]


class Desk(ctypes.Structure):
    """`igl_desk`: the six entries of the reference's `back_desk`."""

    _fields_ = [
        ("name_text", ctypes.c_char_p),
        ("state", ctypes.c_void_p),
        ("mat_vec", ctypes.c_void_p),
        ("mat_mat", ctypes.c_void_p),
        ("norm_rms", ctypes.c_void_p),
        ("soft_max", ctypes.c_void_p),
        ("gelu_gate", ctypes.c_void_p),
        ("rope_turn", ctypes.c_void_p),
    ]


class Rng(ctypes.Structure):
    _fields_ = [("s", ctypes.c_uint64 * 4)]


class GemmaShape(ctypes.Structure):
    """`igl_gemma_shape`: the synthetic checkpoint's text-stack dimensions."""

    _fields_ = [(n, ctypes.c_int) for n in (
        "vocab", "hidden", "inner", "layers", "heads", "kv_heads", "head_dim", "full_head_dim",
        "window", "ple_size", "shared_layers", "double_wide", "full_every", "max_positions",
        "cache_scales", "kinds")] + [(n, ctypes.c_float) for n in (
            "norm_eps", "logit_cap", "rope_local", "rope_global", "partial_rotary")]


MAT_VEC_FN = ctypes.CFUNCTYPE(None, ctypes.POINTER(Desk), ctypes.POINTER(Plane), c_float_p, c_float_p)
MAT_MAT_FN = ctypes.CFUNCTYPE(None, ctypes.POINTER(Desk), ctypes.POINTER(Plane), c_float_p,
                              ctypes.c_int, ctypes.c_int, c_float_p, ctypes.c_int)
NORM_RMS_FN = ctypes.CFUNCTYPE(None, ctypes.POINTER(Desk), c_float_p, c_float_p, ctypes.c_int,
                               ctypes.c_float, c_float_p)
SOFT_MAX_FN = ctypes.CFUNCTYPE(None, ctypes.POINTER(Desk), c_float_p, ctypes.c_int)
GELU_GATE_FN = ctypes.CFUNCTYPE(None, ctypes.POINTER(Desk), c_float_p, c_float_p, ctypes.c_int)
ROPE_TURN_FN = ctypes.CFUNCTYPE(None, ctypes.POINTER(Desk), c_float_p, ctypes.c_int, c_float_p,
                                c_float_p)

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_Z = ctypes.c_size_t

# name -> (restype, argtypes); every function include/igl_backend.h declares.
SIGNATURES = {
    "igl_back_open": (_I, [ctypes.POINTER(Desk), _I, _I, _I, _I]),
    "igl_back_close": (None, [ctypes.POINTER(Desk)]),
    "igl_desk_error_take": (_I, [ctypes.POINTER(Desk)]),
    "igl_code_text": (ctypes.c_char_p, [_I]),
    "igl_plane_attach": (_I, [ctypes.POINTER(Desk), ctypes.POINTER(Plane)]),
    "igl_plane_bind_dev": (_I, [ctypes.POINTER(Desk), ctypes.POINTER(Plane), _P, _P]),
    "igl_plane_detach": (None, [ctypes.POINTER(Desk), ctypes.POINTER(Plane)]),
    "igl_mat_mat_dev": (_I, [ctypes.POINTER(Desk), ctypes.POINTER(Plane), _P, _I, _I, _P, _I]),
    "igl_gemv_dev": (_I, [ctypes.POINTER(Desk), ctypes.POINTER(Plane), _P, _I, _I, _P, _I]),
    "igl_gemm_bf16_dev": (_I, [ctypes.POINTER(Desk), ctypes.POINTER(Plane), _P, _I, _I, _P, _I]),
    "igl_gemm_lane_floor": (_I, []),
    "igl_quant_step_dev": (_I, [ctypes.POINTER(Desk), _P, _I, _P, _I, _I, _I, _F]),
    "igl_plane_lift_dev": (_I, [ctypes.POINTER(Desk), ctypes.POINTER(Plane), _P, _I, _I, _P, _I]),
    "igl_attend_dev": (_I, [ctypes.POINTER(Desk), _P, _P, _I, _F, _F, _I, _I, _I, _I, _P, _I, _I,
                            _F, _P]),
    "igl_attend_lanes_dev": (_I, [ctypes.POINTER(Desk), _P, _P, _I, _F, _F, _I, _I, _I, _I, _P,
                                  _I, _I, _I, _I, _F, _P]),
    "igl_attend_lanes_fixed_dev": (_I, [ctypes.POINTER(Desk), _P, _P, _I, _F, _F, _I, _I, _I, _I,
                                        _P, _I, _I, _I, _I, _F, _P]),
    "igl_gemma_shape_e2b": (None, [ctypes.POINTER(GemmaShape)]),
    "igl_gemma_full_layer": (_I, [ctypes.POINTER(GemmaShape), _I]),
    "igl_gemma_write": (_I, [ctypes.c_char_p, ctypes.POINTER(GemmaShape), ctypes.c_uint64]),
    "igl_zero_unpack": (None, [_P, _I, _I, _I, _P]),
    "igl_engine_open": (_I, [ctypes.POINTER(_P), ctypes.POINTER(Desk), ctypes.c_char_p, _I, _I, _I]),
    "igl_engine_close": (None, [_P]),
    "igl_engine_prime": (_I, [_P, _P, _I]),
    "igl_engine_step": (_I, [_P, ctypes.c_int32, ctypes.POINTER(ctypes.c_int32),
                             ctypes.POINTER(ctypes.c_float)]),
    "igl_engine_logits": (_I, [_P, _P, _I]),
    "igl_engine_fill": (_I, [_P]),
    "igl_engine_vocab": (_I, [_P]),
    "igl_engine_reset": (_I, [_P]),
    "igl_engine_set_graph": (_I, [_P, _I]),
    "igl_engine_guess": (_I, [_P, _P, _I, _P, _P]),
    "igl_engine_keep": (_I, [_P, _I]),
    "igl_scout_open": (_I, [ctypes.POINTER(_P)]),
    "igl_scout_close": (None, [_P]),
    "igl_scout_note": (_I, [_P, _P, _I]),
    "igl_scout_draw": (_I, [_P, _P, _I]),
    "igl_cache_lay_dev": (_I, [ctypes.POINTER(Desk), _P, _I, _F, _I, _P, _Z]),
    "igl_norm_rms_dev": (_I, [ctypes.POINTER(Desk), _P, _P, _I, _I, _I, _F, _P]),
    "igl_soft_max_dev": (_I, [ctypes.POINTER(Desk), _P, _I, _I, _I]),
    "igl_gelu_gate_dev": (_I, [ctypes.POINTER(Desk), _P, _P, _I]),
    "igl_rope_turn_dev": (_I, [ctypes.POINTER(Desk), _P, _I, _I, _P, _P]),
    "igl_dev_alloc": (_P, [ctypes.POINTER(Desk), _Z]),
    "igl_dev_free": (None, [ctypes.POINTER(Desk), _P]),
    "igl_copy_to_dev": (_I, [ctypes.POINTER(Desk), _P, _P, _Z]),
    "igl_copy_to_host": (_I, [ctypes.POINTER(Desk), _P, _P, _Z]),
    "igl_fill_dev": (_I, [ctypes.POINTER(Desk), _P, _I, _Z]),
    "igl_sync": (_I, [ctypes.POINTER(Desk)]),
    "igl_mark": (_I, [ctypes.POINTER(Desk)]),
    "igl_marks_ms": (_F, [ctypes.POINTER(Desk)]),
    "igl_read_floor_dev": (_I, [ctypes.POINTER(Desk), _P, _Z]),
    "igl_record_begin": (_I, [ctypes.POINTER(Desk)]),
    "igl_record_end": (_I, [ctypes.POINTER(Desk), ctypes.POINTER(_P)]),
    "igl_replay_run": (_I, [ctypes.POINTER(Desk), _P]),
    "igl_replay_free": (None, [ctypes.POINTER(Desk), _P]),
    "igl_rng_seed": (None, [ctypes.POINTER(Rng), ctypes.c_uint64]),
    "igl_rng_next": (ctypes.c_uint64, [ctypes.POINTER(Rng)]),
    "igl_rng_normal": (None, [ctypes.POINTER(Rng), _P, _Z, _F, _F]),
    "igl_rng_codes4": (None, [ctypes.POINTER(Rng), _P, _I, _I, _Z]),
    "igl_rng_gains": (None, [ctypes.POINTER(Rng), _P, _Z, _F]),
}

_lib = None


class BackendMissing(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """The backend library, with every declared signature applied."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise BackendMissing(
            f"{LIB_PATH} is not built; run `make -C igllm_amd/csrc` (the gfx950 backend has no "
            "CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib
