"""The allocation-free MLP entry point (static device scratch) against the
workspace entry point, through the C ABI: two calls in a row, the second
smaller, both bit-equal to xmh3_w8a8_mlp on the same inputs."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(m, d, f, seed):
    from x_minimaxh3_amd import workloads

    return workloads.mlp_inputs(M=m, d=d, ffn=f, n_outlier=8, seed=seed)


def _run(lib, name, inp, dev, workspace=None):
    from x_minimaxh3_amd import _lib

    x, w1, s1, w2, s2 = (inp[k].to(dev) for k in ("x", "w1", "s1", "w2", "s2"))
    m, d = x.shape
    f = w1.shape[0]
    y = torch.full((m, d), float("nan"), dtype=torch.bfloat16, device=dev)
    st = _lib.stream_of(x)
    common = (x.data_ptr(), 2, m, d, f, d, w1.data_ptr(), s1.data_ptr(), 1, w2.data_ptr(), s2.data_ptr(), 1,
              y.data_ptr(), d)
    if workspace is None:
        rc = lib.xmh3_w8a8_mlp_noalloc(*common, st)
    else:
        rc = lib.xmh3_w8a8_mlp(*common, workspace.data_ptr(), workspace.numel(), st)
    assert rc == 0, lib.xmh3_last_error()
    torch.cuda.synchronize()
    return y


def test_mlp_noalloc_matches_workspace_entry(pkg, dev):
    from x_minimaxh3_amd import _lib

    lib = _lib.load()
    d, f = 1536, 6144
    for m, seed in ((1000, 0), (257, 1)):          # the second call is smaller
        print(f"noalloc mlp m={m} d={d} ffn={f}", flush=True)
        inp = _inputs(m, d, f, seed)
        ws = torch.empty(lib.xmh3_w8a8_mlp_workspace_bytes(m, d, f), dtype=torch.uint8, device=dev)
        want = _run(lib, "ws", inp, dev, workspace=ws)
        got = _run(lib, "noalloc", inp, dev)
        assert torch.equal(got, want), m


def test_mlp_noalloc_rejects_sizes_beyond_the_scratch(pkg, dev):
    from x_minimaxh3_amd import _lib

    lib = _lib.load()
    rc = lib.xmh3_w8a8_mlp_noalloc(None, 2, 1440, 5120, 13824, 5120, None, None, 1, None, None, 1, None, 5120, None)
    assert rc == 1 and b"static scratch" in lib.xmh3_last_error()
