"""MI355X (gfx950) quantized DiT-block hot path, behind the reference's op API.

Import name: ``x_minimaxh3_amd`` (the directory name carries a hyphen, so it is
loaded by path: ``__graft_entry__.load_package()``).

Ops (reference names and signatures): ``quantize_int8_rowwise``,
``int8_linear``, ``w4a8_int8_linear``, ``rms_adaln``,
``apply_rope_split_half(_)``, ``rms_rope_split_half(_)`` and the interleaved
``apply_rope(_)``, ``rms_rope(_)``; fused hot-path ops:
``norm_rope``, ``w8a8_mlp``, ``w4a8_mlp``. H3 call-site adapters live in
``h3``; the token-chunked / streamed MLP driver in ``driver``.
"""

from . import _lib
from .exceptions import BackendError, BackendNotFoundError, BackendNotImplementedError, NoCapableBackendError
from .ops import (
    DTYPE_CODE_TO_DTYPE,
    DTYPE_TO_CODE,
    apply_rope,
    apply_rope1,
    apply_rope1_,
    apply_rope_,
    apply_rope_split_half,
    apply_rope_split_half1,
    apply_rope_split_half1_,
    apply_rope_split_half_,
    disable_backend,
    enable_backend,
    int8_linear,
    list_backends,
    mm_int8,
    norm_rope,
    quantize_int8_rowwise,
    rms_adaln,
    rms_rope,
    rms_rope1,
    rms_rope1_,
    rms_rope_,
    rms_rope_split_half,
    rms_rope_split_half1,
    rms_rope_split_half1_,
    rms_rope_split_half_,
    set_backend_priority,
    use_backend,
    w4a8_int8_linear,
    w4a8_mlp,
    w8a8_mlp,
)
from .registry import registry

__all__ = [
    "apply_rope", "apply_rope1", "apply_rope1_", "apply_rope_", "rms_rope", "rms_rope1", "rms_rope1_", "rms_rope_",
    "apply_rope_split_half", "apply_rope_split_half1", "apply_rope_split_half1_", "apply_rope_split_half_",
    "disable_backend", "enable_backend", "int8_linear", "list_backends", "mm_int8", "norm_rope",
    "quantize_int8_rowwise", "rms_adaln", "rms_rope_split_half", "rms_rope_split_half1",
    "rms_rope_split_half1_", "rms_rope_split_half_", "set_backend_priority", "use_backend",
    "w4a8_int8_linear", "w4a8_mlp", "w8a8_mlp", "registry", "BackendError", "BackendNotFoundError",
    "BackendNotImplementedError", "NoCapableBackendError", "DTYPE_CODE_TO_DTYPE", "DTYPE_TO_CODE",
]


def library_loaded() -> bool:
    return _lib._LIB is not None


def ensure_library():
    """Load the HIP library (raises ImportError with the build command if it is missing)."""
    return _lib.load()
