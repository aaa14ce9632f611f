"""igllm_amd: a gfx950 (MI355X) backend for igllm's quantized projection path.

The product is libigl_hip.so (hand-written HIP kernels behind a C11 shim that
fills the reference engine's backend table, include/igl_backend.h).  This
package is its Python host side: `native` binds the C ABI, `backend` wraps it.
"""
from .native import load, LIB_PATH, BackendMissing  # noqa: F401
