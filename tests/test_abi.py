"""The C-ABI library loads and exports every symbol include/xmh3.h declares
(no compute calls: runs without a GPU)."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "xmh3.h"
LIB = ROOT / "x-minimaxh3_amd" / "libxmh3_hip.so"


def declared_symbols() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b((?:xmh3_|launch_)[a-z0-9_]+)\s*\(", text))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for s in ("xmh3_quantize_int8_rowwise", "xmh3_int8_gemm", "xmh3_w8a8_mlp", "xmh3_w4a8_mlp",
              "xmh3_norm_rope", "xmh3_rms_adaln", "xmh3_rope_split_half", "xmh3_w4_decode_int8",
              "xmh3_last_error"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    if not LIB.exists():
        pytest.fail(f"{LIB} missing: run __graft_entry__.build()")
    lib = ctypes.CDLL(str(LIB))
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    lib.xmh3_abi_version.restype = ctypes.c_int
    assert lib.xmh3_abi_version() == 1


def test_binding_table_matches_header(pkg):
    from x_minimaxh3_amd import _lib

    assert set(_lib.SIGNATURES) == declared_symbols()


def test_workspace_queries_without_gpu(pkg):
    from x_minimaxh3_amd import _lib

    lib = _lib.load()
    n = lib.xmh3_w8a8_mlp_workspace_bytes(25200, 5120, 13824)
    # q1 + sx + g(bf16) + amax + q2 + sg, each 256-byte aligned
    expect = 0
    for b in (25200 * 5120, 25200 * 4, 25200 * 13824 * 2, 25200 * 4, 25200 * 13824, 25200 * 4):
        expect += (b + 255) // 256 * 256
    assert n == expect
    # W4A8 decodes W1 into q2's region (needs M >= d) and W2 into h's (2M >= d)
    assert lib.xmh3_w4a8_mlp_workspace_bytes(25200, 5120, 13824, 128) == n
    w8 = lib.xmh3_w8a8_mlp_workspace_bytes
    assert lib.xmh3_w4a8_mlp_workspace_bytes(64, 256, 512, 128) == w8(64, 256, 512) + 2 * 512 * 256
    assert lib.xmh3_w4a8_mlp_workspace_bytes(200, 256, 512, 64) == w8(200, 256, 512) + 512 * 256
    assert lib.xmh3_w4a8_mlp_workspace_bytes(256, 256, 512, 16) == w8(256, 256, 512)


def test_argument_errors_need_no_gpu(pkg):
    """Shape validation happens before any launch: bad arguments return status 1
    with a message, and nothing crosses the ABI as an exception."""
    from x_minimaxh3_amd import _lib

    lib = _lib.load()
    rc = lib.xmh3_int8_gemm(None, 16, None, 16, 4, 4, 17, None, None, 0, None, None, 2, 4, 0, None, None)
    assert rc == 1
    assert b"K must be a multiple of 16" in lib.xmh3_last_error() or b"null" in lib.xmh3_last_error()
    rc = lib.xmh3_quantize_int8_rowwise(None, 2, 2, 4, 16, 16, None, None, None)
    assert rc == 1 and b"input_act" in lib.xmh3_last_error()
    rc = lib.xmh3_w8a8_mlp(None, 2, 8, 100, 64, 100, None, None, 1, None, None, 1, None, 100, None, 0, None)
    assert rc == 1 and b"multiples of 16" in lib.xmh3_last_error()


def test_argument_errors_of_the_h3_entry_points(pkg):
    """The ConvRot quantizer, the gated-residual GEMM and the W4A8 group sums
    reject bad shapes before any launch (the pointers below are never
    dereferenced: every case fails validation first)."""
    from x_minimaxh3_amd import _lib

    lib = _lib.load()
    fake = 4096   # aligned, never used
    err = lambda: lib.xmh3_last_error()
    # ConvRot quantizer: group, width, activation
    for bad_group in (32, 2048, 4096, 3):
        assert lib.xmh3_quantize_int8_rowwise_convrot(fake, 2, 0, 4, 4096, 4096, bad_group, fake, fake, None) == 1
        assert b"convrot_groupsize" in err()
    assert lib.xmh3_quantize_int8_rowwise_convrot(fake, 2, 0, 4, 768, 768, 1024, fake, fake, None) == 1
    assert b"multiple of convrot_groupsize" in err()
    assert lib.xmh3_quantize_int8_rowwise_convrot(fake, 2, 0, 4, 100, 128, 256, fake, fake, None) == 1
    assert b"multiple of 256" in err()
    assert lib.xmh3_quantize_int8_rowwise_convrot(fake, 2, 0, 4, 16640, 16640, 256, fake, fake, None) == 1
    assert b"16384" in err()
    assert lib.xmh3_quantize_int8_rowwise_convrot(fake, 2, 5, 4, 256, 256, 256, fake, fake, None) == 1
    assert b"activation" in err()
    assert lib.xmh3_quantize_int8_rowwise_convrot(fake, 2, 1, 4, 256, 256, 0, fake, fake, None) == 3
    assert b"only swiglu" in err()
    assert lib.xmh3_quantize_int8_rowwise_convrot(fake, 0, 0, 4, 256, 256, 256, fake, fake, None) == 3
    assert b"bf16 or fp16" in err()
    # gated residual: width multiple of 4, residual dtype, gate dtype, gate rows
    args = lambda n, rdt, gdt, nrows: (fake, 512, fake, 512, 8, n, 512, fake, fake, 1, None, fake, rdt, n + 2,
                                       fake, gdt, n + 2, nrows, fake, None)
    assert lib.xmh3_int8_gemm_gated_residual(*args(6, 2, 0, 1)) == 1 and b"multiples of 4" in err()
    assert lib.xmh3_int8_gemm_gated_residual(*args(8, 0, 0, 1)) == 1 and b"bf16 or fp16" in err()
    assert lib.xmh3_int8_gemm_gated_residual(*args(8, 2, 1, 1)) == 1 and b"gate must be" in err()
    assert lib.xmh3_int8_gemm_gated_residual(*args(8, 2, 0, 0)) == 1 and b"gate table" in err()
    # W4A8 correction group sums
    assert lib.xmh3_int8_group_sums(fake, 64, fake, 4, 60, 16, fake, 2, 4, None) == 1
    assert b"multiple of group_size" in err()
    assert lib.xmh3_int8_group_sums(fake, 64, fake, 4, 64, 16, fake, 7, 4, None) == 3
    assert b"out dtype" in err()


def test_reference_rope_launcher_signature(pkg):
    """launch_rms_rope_kernel keeps the reference's 46-argument list (the
    argtypes single_qknorm_rope.py pins) and rejects arguments outside its
    rules without launching anything."""
    from x_minimaxh3_amd import _lib

    res, args = _lib.SIGNATURES["launch_rms_rope_kernel"]
    assert res is None and len(args) == 46
    assert args == [ctypes.c_void_p] * 7 + [ctypes.c_int64] * 32 + [ctypes.c_float] + [ctypes.c_int] * 3 + \
        [ctypes.c_bool] * 2 + [ctypes.c_void_p]
    lib = _lib.load()
    fake = 4096
    base = [fake, None, fake, fake, None, fake, None, 1, 8, 4, 128, 128, 1, 8, 1,
            4096, 512, 128, 1, 0, 0, 0, 0, 4096, 512, 128, 1, 0, 0, 0, 0,
            0, 256, 0, 4, 2, 1, 1, 0, 1e-6, 2, 0, 2, False, True, None]
    assert len(base) == 46
    interleaved = list(base)       # split_half = false runs, with its own rot_dim rule
    interleaved[44] = False
    interleaved[11] = 12           # rot_dim
    lib.launch_rms_rope_kernel(*interleaved)
    assert b"interleaved rot_dim" in lib.xmh3_last_error()
    interleaved[44] = True         # split-half needs rot_dim % 16
    lib.launch_rms_rope_kernel(*interleaved)
    assert b"multiple of 16" in lib.xmh3_last_error()
    strided = list(base)
    strided[18] = 2            # q_s3
    lib.launch_rms_rope_kernel(*strided)
    assert b"contiguous" in lib.xmh3_last_error()
