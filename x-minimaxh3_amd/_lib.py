"""ctypes binding of ``libxmh3_hip.so`` (the C ABI declared in include/xmh3.h).

torch is imported first so that the library's ``libamdhip64.so.7`` dependency
binds to the HIP runtime torch already loaded (same SONAME): kernels then run
on torch's streams and memory.

There is no fallback: if the library is missing, importing the package's ops
raises with the build command.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

LIB_PATH = Path(__file__).resolve().parent / "libxmh3_hip.so"

c_void_p = ctypes.c_void_p
c_int = ctypes.c_int
c_i64 = ctypes.c_int64
c_size = ctypes.c_size_t
c_float = ctypes.c_float
P_I64 = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); the order of every argtypes list is the
# prototype in include/xmh3.h
SIGNATURES: dict[str, tuple] = {
    "xmh3_last_error": (ctypes.c_char_p, []),
    "xmh3_abi_version": (c_int, []),
    "xmh3_quantize_int8_rowwise": (c_int, [c_void_p, c_int, c_int, c_i64, c_i64, c_i64, c_void_p, c_void_p, c_void_p]),
    "xmh3_quantize_int8_rowwise_sr": (c_int, [c_void_p, c_int, c_i64, c_i64, c_i64, c_void_p, c_void_p, c_int,
                                              ctypes.c_uint64, c_void_p]),
    "xmh3_quantize_int8_rowwise_ex": (c_int, [c_void_p, c_int, c_int, c_i64, c_i64, c_i64, c_void_p, c_void_p,
                                              c_void_p, c_void_p]),
    "xmh3_quantize_int8_rowwise_convrot": (c_int, [c_void_p, c_int, c_int, c_i64, c_i64, c_i64, c_int, c_void_p,
                                                   c_void_p, c_void_p]),
    "xmh3_quantize_int8_rowwise_convrot_sr": (c_int, [c_void_p, c_int, c_int, c_i64, c_i64, c_i64, c_int, c_void_p,
                                                      c_void_p, c_int, ctypes.c_uint64, c_void_p]),
    "xmh3_requant_int8_rows": (c_int, [c_void_p, c_int, c_i64, c_i64, c_i64, c_void_p, c_void_p, c_void_p, c_void_p]),
    "xmh3_int8_gemm": (c_int, [c_void_p, c_i64, c_void_p, c_i64, c_i64, c_i64, c_i64, c_void_p, c_void_p, c_int,
                               c_void_p, c_void_p, c_int, c_i64, c_int, c_void_p, c_void_p]),
    "xmh3_int8_gemm_gated_residual": (c_int, [c_void_p, c_i64, c_void_p, c_i64, c_i64, c_i64, c_i64, c_void_p,
                                              c_void_p, c_int, c_void_p, c_void_p, c_int, c_i64, c_void_p, c_int,
                                              c_i64, c_i64, c_void_p, c_void_p]),
    "xmh3_int8_group_sums": (c_int, [c_void_p, c_i64, c_void_p, c_i64, c_i64, c_i64, c_void_p, c_int, c_i64,
                                     c_void_p]),
    "xmh3_w4_decode_int8": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_i64, c_i64, c_i64, c_void_p, c_void_p]),
    "xmh3_w8a8_mlp_workspace_bytes": (c_size, [c_i64, c_i64, c_i64]),
    "xmh3_w8a8_mlp": (c_int, [c_void_p, c_int, c_i64, c_i64, c_i64, c_i64, c_void_p, c_void_p, c_int, c_void_p,
                              c_void_p, c_int, c_void_p, c_i64, c_void_p, c_size, c_void_p]),
    "xmh3_w8a8_mlp_noalloc": (c_int, [c_void_p, c_int, c_i64, c_i64, c_i64, c_i64, c_void_p, c_void_p, c_int,
                                      c_void_p, c_void_p, c_int, c_void_p, c_i64, c_void_p]),
    "xmh3_w4a8_mlp_workspace_bytes": (c_size, [c_i64, c_i64, c_i64, c_i64]),
    "xmh3_w4a8_gemm": (c_int, [c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_int, c_i64, c_i64, c_i64, c_i64, c_i64,
                               c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_i64, c_void_p]),
    "xmh3_w4a8_mlp": (c_int, [c_void_p, c_int, c_i64, c_i64, c_i64, c_i64, c_void_p, c_void_p, c_void_p,
                              c_void_p, c_void_p, c_void_p, c_int, c_i64, c_void_p, c_i64, c_void_p, c_size,
                              c_void_p]),
    "xmh3_norm_rope": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_i64, c_i64, c_i64, c_i64,
                               c_void_p, c_void_p, c_int, c_i64, c_i64, c_void_p, c_int, c_i64, c_int, c_float,
                               c_void_p]),
    "xmh3_rms_adaln": (c_int, [c_void_p, c_void_p, c_int, c_i64, c_i64, c_i64, c_i64, c_void_p, c_void_p,
                               c_void_p, c_int, c_i64, c_void_p, c_i64, c_float, c_void_p]),
    "launch_rms_rope_kernel": (None, [c_void_p] * 7 + [c_i64] * 32 + [c_float] + [c_int] * 3 + [ctypes.c_bool] * 2
                               + [c_void_p]),
    "xmh3_rope_split_half": (c_int, [c_void_p, c_void_p, c_int, c_i64, c_i64, c_i64, c_i64, P_I64, P_I64,
                                     c_void_p, c_int, c_void_p, c_int, P_I64, c_int, c_float, c_int, c_void_p]),
    "xmh3_rope_heads": (c_int, [c_void_p, c_void_p, c_int, c_i64, c_i64, c_i64, c_i64, P_I64, P_I64,
                                c_void_p, c_int, c_void_p, c_int, P_I64, c_int, c_float, c_int, c_int, c_void_p]),
    "xmh3_rope_heads_qk": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_i64, c_i64, c_i64, c_i64,
                                   P_I64, P_I64, P_I64, P_I64, c_void_p, c_void_p, c_int, c_void_p, c_int, P_I64,
                                   c_int, c_float, c_int, c_int, c_void_p]),
}

_LIB: ctypes.CDLL | None = None


class KernelError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise ImportError(
            f"HIP library {p} is missing: build it with "
            "`python x-minimaxh3_amd/build.py` (or __graft_entry__.build())")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


def call(name: str, *args) -> None:
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.xmh3_last_error().decode(errors="replace")
        if rc in (1, 3):
            raise ValueError(f"{name}: {msg}")
        raise KernelError(f"{name} failed ({rc}): {msg}")


def query(name: str, *args):
    return getattr(load(), name)(*args)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def i64array(vals) -> ctypes.Array:
    arr = (ctypes.c_int64 * len(vals))(*[int(v) for v in vals])
    return arr


DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
