"""Python host side of the gfx950 backend, over the C ABI in include/igl_backend.h.

`Backend` opens a desk (igl_back_open, the drop-in for the reference's
back_open, app_core.c:5415-5443) and exposes its table entries with the
reference's argument meanings, plus the device-resident entries.  Arrays are
numpy; device memory is the library's own (no torch).  Every call checks the
desk's sticky error and raises `BackendError` on failure.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import native
from .native import Desk, Plane, Rng


class BackendError(RuntimeError):
    pass


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


class DevBuf:
    """A block of device memory owned by a Backend."""

    def __init__(self, backend: "Backend", nbytes: int):
        self.backend = backend
        self.nbytes = int(nbytes)
        self.ptr = backend.lib.igl_dev_alloc(ctypes.byref(backend.desk), self.nbytes)
        if not self.ptr:
            raise BackendError(f"igl_dev_alloc({self.nbytes}) failed")

    def put(self, host: np.ndarray, offset: int = 0) -> "DevBuf":
        host = np.ascontiguousarray(host)
        if offset + host.nbytes > self.nbytes:
            raise BackendError("copy past the end of a device buffer")
        self.backend._check(self.backend.lib.igl_copy_to_dev(
            ctypes.byref(self.backend.desk), self.ptr + offset, _ptr(host), host.nbytes), "copy_to_dev")
        return self

    def get(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        if offset + out.nbytes > self.nbytes:
            raise BackendError("copy past the end of a device buffer")
        self.backend._check(self.backend.lib.igl_copy_to_host(
            ctypes.byref(self.backend.desk), _ptr(out), self.ptr + offset, out.nbytes), "copy_to_host")
        return out

    def free(self):
        if self.ptr:
            self.backend.lib.igl_dev_free(ctypes.byref(self.backend.desk), self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


@dataclass
class CodePlane:
    """A plane (code or real): the numpy arrays it points into and its igl_plane."""

    plane: Plane
    codes: np.ndarray  # uint8 [N, row_stride]
    gains: np.ndarray  # float32 [N, G]
    zeros: np.ndarray | None = None  # int8 [N, G] zero points, kept alive with the plane

    @property
    def N(self) -> int:
        return self.plane.row_count

    @property
    def K(self) -> int:
        return self.plane.col_count


def make_plane(codes: np.ndarray, gains: np.ndarray, K: int, group_size: int = 32,
               code_bias: int | None = None, bits: int = 4, code_flip: int = 0,
               zeros: np.ndarray | None = None) -> CodePlane:
    """A code plane over `codes` [N, row_stride] (bits-wide fields, low bits
    first) and F32 `gains` [N, groups]; code_bias defaults to 2^(bits-1), the
    export's offset (plane_bind_gemma, app_core.c:7931-7935).  `zeros`: int8
    zero points [N, groups] (plane_bind_part's bias_data, app_core.c:8053-8063),
    or None for a symmetric plane."""
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    gains = np.ascontiguousarray(gains, dtype=np.float32)
    if zeros is not None:
        zeros = np.ascontiguousarray(zeros, dtype=np.int8)
        assert zeros.shape == gains.shape
    N = codes.shape[0]
    p = Plane()
    p.form = native.IGL_PLANE_CODE
    p.row_count = N
    p.col_count = K
    p.code_data = _ptr(codes)
    p.row_stride = codes.shape[1]
    p.gain_data = _ptr(gains)
    p.gain_type = native.IGL_STORE_F32
    p.bias_data = None if zeros is None else _ptr(zeros)
    p.bit_count = bits
    p.code_bias = (1 << (bits - 1)) if code_bias is None else code_bias
    p.code_flip = code_flip
    p.group_size = group_size
    p.group_count = gains.shape[1]
    return CodePlane(p, codes, gains, zeros)


def make_real_plane(rows: np.ndarray, real_type: int) -> CodePlane:
    """A real plane over `rows` [N, K]: float32, or the uint16 bits of binary16
    (IGL_STORE_F16) or bf16 (IGL_STORE_BF16) values."""
    rows = np.ascontiguousarray(rows)
    want = np.float32 if real_type == native.IGL_STORE_F32 else np.uint16
    if rows.dtype != want:
        raise ValueError(f"real_type {real_type} takes {want.__name__} rows")
    p = Plane()
    p.form = native.IGL_PLANE_REAL
    p.row_count = rows.shape[0]
    p.col_count = rows.shape[1]
    p.real_data = _ptr(rows)
    p.real_type = real_type
    return CodePlane(p, rows, np.zeros((0,), dtype=np.float32))


class Backend:
    def __init__(self, device: int = 0, sum_limit: int = 1024, col_limit: int = 16384,
                 lane_limit: int = 16):
        self.lib = native.load()
        self.desk = Desk()
        code = self.lib.igl_back_open(ctypes.byref(self.desk), device, sum_limit, col_limit, lane_limit)
        if code != native.IGL_OKAY:
            raise BackendError(f"igl_back_open: {self.lib.igl_code_text(code).decode()}")
        self._mat_vec = native.MAT_VEC_FN(self.desk.mat_vec)
        self._mat_mat = native.MAT_MAT_FN(self.desk.mat_mat)
        self._norm_rms = native.NORM_RMS_FN(self.desk.norm_rms)
        self._soft_max = native.SOFT_MAX_FN(self.desk.soft_max)
        self._gelu_gate = native.GELU_GATE_FN(self.desk.gelu_gate)
        self._rope_turn = native.ROPE_TURN_FN(self.desk.rope_turn)
        self.name = self.desk.name_text.decode()

    # -- errors ---------------------------------------------------------------
    def error_take(self) -> int:
        return self.lib.igl_desk_error_take(ctypes.byref(self.desk))

    def _check(self, code: int, what: str):
        sticky = self.error_take()
        code = code if code != native.IGL_OKAY else sticky
        if code != native.IGL_OKAY:
            raise BackendError(f"{what}: {self.lib.igl_code_text(code).decode()} ({code})")

    def _after_table(self, what: str):
        self._check(native.IGL_OKAY, what)

    def close(self):
        if self.desk.state:
            self.lib.igl_back_close(ctypes.byref(self.desk))

    # -- planes ---------------------------------------------------------------
    def attach(self, cp: CodePlane) -> CodePlane:
        self._check(self.lib.igl_plane_attach(ctypes.byref(self.desk), ctypes.byref(cp.plane)), "attach")
        return cp

    def bind_dev(self, cp: CodePlane, codes: DevBuf, gains: DevBuf, code_offset: int = 0,
                 gain_offset: int = 0) -> CodePlane:
        self._check(self.lib.igl_plane_bind_dev(ctypes.byref(self.desk), ctypes.byref(cp.plane),
                                                codes.ptr + code_offset, gains.ptr + gain_offset),
                    "bind_dev")
        return cp

    def detach(self, cp: CodePlane):
        self.lib.igl_plane_detach(ctypes.byref(self.desk), ctypes.byref(cp.plane))

    # -- the table (host pointers) --------------------------------------------
    def mat_vec(self, cp: CodePlane, act: np.ndarray) -> np.ndarray:
        act = np.ascontiguousarray(act, dtype=np.float32)
        out = np.empty(cp.N, dtype=np.float32)
        self._mat_vec(ctypes.byref(self.desk), ctypes.byref(cp.plane),
                      act.ctypes.data_as(native.c_float_p), out.ctypes.data_as(native.c_float_p))
        self._after_table("mat_vec")
        return out

    def mat_mat(self, cp: CodePlane, act: np.ndarray) -> np.ndarray:
        act = np.ascontiguousarray(act, dtype=np.float32)
        lanes = act.shape[0]
        out = np.empty((lanes, cp.N), dtype=np.float32)
        self._mat_mat(ctypes.byref(self.desk), ctypes.byref(cp.plane),
                      act.ctypes.data_as(native.c_float_p), act.shape[1], lanes,
                      out.ctypes.data_as(native.c_float_p), cp.N)
        self._after_table("mat_mat")
        return out

    def norm_rms(self, values: np.ndarray, gain, eps: float) -> np.ndarray:
        values = np.ascontiguousarray(values, dtype=np.float32)
        out = np.empty_like(values)
        g = None if gain is None else np.ascontiguousarray(gain, dtype=np.float32)
        self._norm_rms(ctypes.byref(self.desk), values.ctypes.data_as(native.c_float_p),
                       None if g is None else g.ctypes.data_as(native.c_float_p), values.size,
                       eps, out.ctypes.data_as(native.c_float_p))
        self._after_table("norm_rms")
        return out

    def soft_max(self, values: np.ndarray) -> np.ndarray:
        v = np.array(values, dtype=np.float32, copy=True)
        self._soft_max(ctypes.byref(self.desk), v.ctypes.data_as(native.c_float_p), v.size)
        self._after_table("soft_max")
        return v

    def gelu_gate(self, gate: np.ndarray, rise: np.ndarray) -> np.ndarray:
        g = np.array(gate, dtype=np.float32, copy=True)
        r = np.ascontiguousarray(rise, dtype=np.float32)
        self._gelu_gate(ctypes.byref(self.desk), g.ctypes.data_as(native.c_float_p),
                        r.ctypes.data_as(native.c_float_p), g.size)
        self._after_table("gelu_gate")
        return g

    def rope_turn(self, values: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
        v = np.array(values, dtype=np.float32, copy=True)
        c = np.ascontiguousarray(cos, dtype=np.float32)
        s = np.ascontiguousarray(sin, dtype=np.float32)
        self._rope_turn(ctypes.byref(self.desk), v.ctypes.data_as(native.c_float_p), v.size,
                        c.ctypes.data_as(native.c_float_p), s.ctypes.data_as(native.c_float_p))
        self._after_table("rope_turn")
        return v

    # -- device-resident entries ------------------------------------------------
    def alloc(self, nbytes: int) -> DevBuf:
        return DevBuf(self, nbytes)

    def upload(self, host: np.ndarray) -> DevBuf:
        host = np.ascontiguousarray(host)
        return DevBuf(self, max(host.nbytes, 1)).put(host)

    def mat_mat_dev(self, cp, act: DevBuf, act_stride, lanes, out: DevBuf, out_stride, act_off=0, out_off=0):
        self._check(self.lib.igl_mat_mat_dev(ctypes.byref(self.desk), ctypes.byref(cp.plane),
                                             act.ptr + act_off, act_stride, lanes, out.ptr + out_off,
                                             out_stride), "mat_mat_dev")

    def gemv_dev(self, cp, act: DevBuf, act_stride, lanes, out: DevBuf, out_stride, act_off=0, out_off=0):
        self._check(self.lib.igl_gemv_dev(ctypes.byref(self.desk), ctypes.byref(cp.plane),
                                          act.ptr + act_off, act_stride, lanes, out.ptr + out_off,
                                          out_stride), "gemv_dev")

    def plane_lift_dev(self, cp, act: DevBuf, act_stride, lanes, out: DevBuf, out_stride):
        """plane_lift_many on device: enter_gain grid, product, leave_gain grid."""
        self._check(self.lib.igl_plane_lift_dev(ctypes.byref(self.desk), ctypes.byref(cp.plane),
                                                act.ptr, act_stride, lanes, out.ptr, out_stride),
                    "plane_lift_dev")

    def quant_step_dev(self, src: DevBuf, src_stride, dst: DevBuf, dst_stride, n, lanes, step):
        self._check(self.lib.igl_quant_step_dev(ctypes.byref(self.desk), src.ptr, src_stride, dst.ptr,
                                                dst_stride, n, lanes, float(step)), "quant_step_dev")

    def gemm_bf16_dev(self, cp, act: DevBuf, act_stride, lanes, out: DevBuf, out_stride):
        self._check(self.lib.igl_gemm_bf16_dev(ctypes.byref(self.desk), ctypes.byref(cp.plane),
                                               act.ptr, act_stride, lanes, out.ptr, out_stride),
                    "gemm_bf16_dev")

    def attend_dev(self, key_store: DevBuf, value_store: DevBuf, fmt: int, key_scale: float,
                   value_scale: float, cache_span: int, kv_count: int, group_share: int,
                   head_size: int, query: DevBuf, place_start: int, span_count: int,
                   score_scale: float, blend_out: DevBuf):
        self._check(self.lib.igl_attend_dev(ctypes.byref(self.desk), key_store.ptr, value_store.ptr,
                                            fmt, key_scale, value_scale, cache_span, kv_count,
                                            group_share, head_size, query.ptr, place_start,
                                            span_count, score_scale, blend_out.ptr), "attend_dev")

    def cache_lay_dev(self, row: DevBuf, width: int, scale: float, fmt: int, store: DevBuf,
                      slot_first: int, row_off: int = 0):
        self._check(self.lib.igl_cache_lay_dev(ctypes.byref(self.desk), row.ptr + row_off, width,
                                               scale, fmt, store.ptr, slot_first), "cache_lay_dev")

    def sync(self):
        self._check(self.lib.igl_sync(ctypes.byref(self.desk)), "sync")

    def mark(self):
        self._check(self.lib.igl_mark(ctypes.byref(self.desk)), "mark")

    def marks_ms(self) -> float:
        ms = self.lib.igl_marks_ms(ctypes.byref(self.desk))
        self._check(native.IGL_OKAY, "marks_ms")
        return ms

    def record_begin(self):
        """Starts recording the device entries called next (igl_record_begin)."""
        self._check(self.lib.igl_record_begin(ctypes.byref(self.desk)), "record_begin")

    def record_end(self) -> int:
        """Ends the recording; returns the replay handle (igl_record_end)."""
        handle = ctypes.c_void_p()
        code = self.lib.igl_record_end(ctypes.byref(self.desk), ctypes.byref(handle))
        if code != native.IGL_OKAY:
            raise BackendError(f"record_end: {self.lib.igl_code_text(code).decode()} ({code})")
        return handle.value

    def replay_run(self, handle: int):
        self._check(self.lib.igl_replay_run(ctypes.byref(self.desk), handle), "replay_run")

    def replay_free(self, handle: int):
        self.lib.igl_replay_free(ctypes.byref(self.desk), handle)

    def read_floor_dev(self, src: DevBuf, nbytes: int):
        """Reads nbytes of a device buffer once and keeps nothing (the HBM read
        floor the GEMV's rate is judged against)."""
        self._check(self.lib.igl_read_floor_dev(ctypes.byref(self.desk), src.ptr, nbytes), "read_floor_dev")


# -- synthetic inputs -----------------------------------------------------------

class Synth:
    """The seeded generator (splitmix64 -> xoshiro256**, Box-Muller) in the library."""

    def __init__(self, seed: int = 0):
        self.lib = native.load()
        self.rng = Rng()
        self.lib.igl_rng_seed(ctypes.byref(self.rng), seed)

    def next(self) -> int:
        return self.lib.igl_rng_next(ctypes.byref(self.rng))

    def normal(self, count: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
        out = np.empty(count, dtype=np.float32)
        self.lib.igl_rng_normal(ctypes.byref(self.rng), _ptr(out), count, mean, std)
        return out

    def codes4(self, N: int, K: int, row_stride: int | None = None) -> np.ndarray:
        row_stride = row_stride or K // 2
        out = np.empty((N, row_stride), dtype=np.uint8)
        self.lib.igl_rng_codes4(ctypes.byref(self.rng), _ptr(out), N, K, row_stride)
        return out

    def gains(self, count: int, std: float = 0.02) -> np.ndarray:
        out = np.empty(count, dtype=np.float32)
        self.lib.igl_rng_gains(ctypes.byref(self.rng), _ptr(out), count, std)
        return out


def synth_projection(N: int, K: int, lanes: int, seed: int = 0, group_size: int = 32):
    """The projection configs' inputs: codes, then gains, then activations, from one stream."""
    s = Synth(seed)
    codes = s.codes4(N, K)
    gains = s.gains(N * (K // group_size)).reshape(N, K // group_size)
    act = s.normal(lanes * K).reshape(lanes, K)
    return codes, gains, act
