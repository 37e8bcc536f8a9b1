import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


def pytest_collection_modifyitems(config, items):
    gpu_items = [it for it in items if "gpu" in it.keywords]
    if not gpu_items:
        return
    import torch

    if not torch.cuda.is_available():
        skip = pytest.mark.skip(reason="no GPU visible")
        for it in gpu_items:
            it.add_marker(skip)


@pytest.fixture(scope="session")
def pkg():
    import __graft_entry__

    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def dev(pkg):
    import torch

    pkg.ensure_library()
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def corc():
    """The plain-C oracle (ctypes), built by `make -C oracle`."""
    import ctypes
    import subprocess

    so = ROOT / "oracle" / "_build" / "liboracle.so"
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)   # rebuilds if oracle.c changed
    lib = ctypes.CDLL(str(so))
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.orc_quant_rows_bf16.argtypes = [vp, i64, i64, vp, vp]
    lib.orc_int_mm.argtypes = [vp, vp, i64, i64, i64, vp]
    lib.orc_dequant_bf16.argtypes = [vp, vp, vp, ctypes.c_int, i64, i64, vp]
    lib.orc_w4_decode.argtypes = [vp, vp, i64, i64, i64, vp]
    lib.orc_pcg_hash.argtypes = [vp, i64, vp]
    lib.orc_quant_rows_sr_bf16.argtypes = [vp, i64, i64, ctypes.c_uint64, vp, vp]
    for f in (lib.orc_quant_rows_bf16, lib.orc_int_mm, lib.orc_dequant_bf16, lib.orc_w4_decode, lib.orc_pcg_hash,
              lib.orc_quant_rows_sr_bf16):
        f.restype = None
    return lib
