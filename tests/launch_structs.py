"""ctypes mirrors of the internal launch structs (igllm_amd/csrc/igl_launch.h)
that GPU tests pass to the launchers directly; test_struct_layout.py pins
each to the C layout."""
import ctypes


class CodeView(ctypes.Structure):
    """igl_code_view, field for field."""
    _fields_ = [("codes", ctypes.c_void_p), ("row_stride", ctypes.c_longlong), ("gains", ctypes.c_void_p),
                ("gain_stride", ctypes.c_int), ("group_shift", ctypes.c_int), ("bit_count", ctypes.c_int),
                ("code_bias", ctypes.c_int), ("code_flip", ctypes.c_int)]


class Prologue(ctypes.Structure):
    """igl_gemv_prologue, field for field; lane_stride is read by the grouped
    launch with several lanes only."""
    _fields_ = [("state_in", ctypes.c_void_p), ("state_out", ctypes.c_void_p), ("lift", ctypes.c_void_p),
                ("lift_gain", ctypes.c_void_p), ("scale", ctypes.c_float), ("apply_scale", ctypes.c_int),
                ("norm_gain", ctypes.c_void_p), ("eps", ctypes.c_float), ("lane_stride", ctypes.c_int)]
