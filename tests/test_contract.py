"""Host-side contract of the op boundary (CPU only): dispatch errors, argument
validation with the reference's error types, in-place guards, modulation
broadcast grouping and the workload generators."""

import pytest
import torch

from oracle import cpu_ref


def test_cpu_tensors_fail_loudly(pkg):
    x = torch.randn(4, 64).bfloat16()
    with pytest.raises(pkg.NoCapableBackendError, match="device cpu"):
        pkg.int8_linear(x, torch.zeros(8, 64, dtype=torch.int8), torch.ones(8))
    with pytest.raises(pkg.NoCapableBackendError):
        pkg.quantize_int8_rowwise(x)
    with pytest.raises(pkg.NoCapableBackendError):
        pkg.rms_adaln(x, x[:1], x[:1])


def test_registry_surface(pkg):
    backs = pkg.list_backends()
    assert backs["mi355x"]["available"]
    assert "int8_linear" in backs["mi355x"]["capabilities"]
    with pytest.raises(pkg.BackendNotFoundError):
        with pkg.use_backend("cuda"):
            pass
    pkg.disable_backend("mi355x")
    try:
        with pytest.raises(pkg.NoCapableBackendError):
            pkg.registry.get_capable_backend("int8_linear", {})
        with pytest.raises(pkg.BackendNotFoundError, match="disabled"):
            pkg.registry.get_implementation("int8_linear", backend="mi355x")
    finally:
        pkg.enable_backend("mi355x")
    with pytest.raises(pkg.BackendNotImplementedError):
        pkg.registry.get_implementation("scaled_mm_nvfp4", backend="mi355x")


def test_unimplemented_reference_features_raise(pkg):
    from x_minimaxh3_amd import backend

    x = torch.randn(2, 256).bfloat16()
    w = torch.zeros(8, 256, dtype=torch.int8)
    with pytest.raises(NotImplementedError, match="ConvRot group size 4096"):
        backend.int8_linear(x, w, torch.ones(8), convrot=True, convrot_groupsize=4096)
    with pytest.raises(NotImplementedError, match="multiple of the ConvRot group size 1024"):
        backend.int8_linear(x, w, torch.ones(8), convrot=True, convrot_groupsize=1024)
    with pytest.raises(NotImplementedError, match="activated width 128"):
        backend.int8_linear(x, w[:, :128].contiguous(), torch.ones(8), input_act="swiglu")
    with pytest.raises(NotImplementedError, match="dtype"):
        backend.int8_linear(x.float(), w, torch.ones(8), convrot=True)
    with pytest.raises(ValueError, match="inner dimensions"):
        backend.int8_linear(torch.randn(2, 512).bfloat16(), w, torch.ones(8), input_act="gelu_tanh")
    with pytest.raises(ValueError, match="unsupported input_act"):
        backend.int8_linear(x, w, torch.ones(8), input_act="relu")
    with pytest.raises(ValueError, match="inner dimensions"):
        backend.int8_linear(x, torch.zeros(8, 128, dtype=torch.int8), torch.ones(8))
    with pytest.raises(ValueError, match="per-output-channel"):
        backend.int8_linear(x, w, torch.ones(3))
    with pytest.raises(ValueError, match="64 bits"):
        backend.quantize_int8_rowwise_convrot64(x, 256, stochastic_rounding=1 << 64)
    with pytest.raises(ValueError, match="64 bits"):
        backend.quantize_int8_rowwise(x, stochastic_rounding=1 << 64)


def test_w4a8_operand_validation(pkg):
    from x_minimaxh3_amd import backend

    q = torch.zeros(16, 128, dtype=torch.int8)  # K = 256
    ok = dict(s_rel=torch.zeros(16, 2), s_channel=torch.zeros(16), codebook=None, correction=None,
              group_size=128, convrot_groupsize=128)
    backend.validate_w4a8_operands(q, **ok)
    with pytest.raises(ValueError, match="s_rel must have shape"):
        backend.validate_w4a8_operands(q, **{**ok, "s_rel": torch.zeros(16, 3)})
    with pytest.raises(ValueError, match="s_channel must have shape"):
        backend.validate_w4a8_operands(q, **{**ok, "s_channel": torch.zeros(15)})
    with pytest.raises(ValueError, match="divisible by 16"):
        backend.validate_w4a8_operands(q, **{**ok, "group_size": 24})
    with pytest.raises(ValueError, match="codebook must have shape"):
        backend.validate_w4a8_operands(q, **{**ok, "codebook": torch.zeros(8)})
    with pytest.raises(ValueError, match="2D int8"):
        backend.validate_w4a8_operands(q.float(), **ok)


def test_rope_inplace_guards(pkg):
    from x_minimaxh3_amd import backend

    qkv = torch.randn(1, 6, 3, 4, 128)
    q, k = qkv[:, :, 0], qkv[:, :, 1]
    backend.check_rope_inplace(q, k)              # packed QKV slices interleave, no overlap
    with pytest.raises(ValueError, match="non-overlapping"):
        backend.check_rope_inplace(q, q)
    base = torch.randn(64, 128)
    with pytest.raises(ValueError, match="internal overlap"):
        backend.check_rope_inplace(base.as_strided((4, 128), (1, 1)))
    freqs = torch.randn(1, 6, 1, 64, 2, 2)
    with pytest.raises(ValueError, match="frequencies or scales"):
        backend.check_rope_inplace(freqs.view(1, 6, 1, 256)[..., :128], readonly=(freqs,))
    with pytest.raises(RuntimeError, match="autograd"):
        backend.check_rope_inplace(torch.randn(2, 8, requires_grad=True))


def test_modulation_grouping(pkg):
    from x_minimaxh3_amd import backend

    x = torch.randn(2, 10, 64)
    s = torch.randn(2, 1, 64)
    rows, g = backend._modulation_rows(s, x)
    assert rows.shape == (2, 64) and g == 10
    rows, g = backend._modulation_rows(torch.randn(64), x)
    assert rows.shape == (1, 64) and g == 20
    rows, g = backend._modulation_rows(torch.randn(1, 10, 64), x)   # broadcast over the outer dim
    assert rows.shape == (20, 64) and g == 1


def test_workloads_deterministic_and_match_oracle_generators(pkg):
    from x_minimaxh3_amd import workloads

    a = workloads.mlp_inputs(64, 256, 512, n_outlier=4, seed=0, weights="both")
    b = workloads.mlp_inputs(64, 256, 512, n_outlier=4, seed=0, weights="both")
    for k in a:
        assert torch.equal(a[k], b[k]), k
    assert (a["x"][:, a["outliers"]].float().abs().mean() > 5 * a["x"].float().abs().mean())
    g = torch.Generator().manual_seed(0)
    torch.randn(64, 256, generator=g)
    torch.randperm(256, generator=g)
    w1f = torch.randn(512, 256, generator=g) * 0.02
    packed, srel, sch = cpu_ref.quantize_w4_weight(w1f, 128)
    assert torch.equal(a["w1_packed"], packed)
    assert torch.equal(a["w1_srel"], srel.to(torch.bfloat16))
    assert torch.equal(a["w1_schannel"], sch)
    q, s = a["w1"], a["s1"]
    assert q.dtype == torch.int8 and torch.equal(q, (w1f / s.view(-1, 1)).round().clamp(-128, 127).to(torch.int8))


def test_h3_w4a8_spec_and_loader(pkg, tmp_path):
    """The H3 W4A8 checkpoint layout: spec validation as the reference's
    W4A8QuantSpec, and loading the five tensor names from a safetensors file
    (no compute: the tensors stay on the CPU)."""
    from safetensors import safe_open
    from safetensors.torch import save_file

    from x_minimaxh3_amd import h3

    h3.W4A8QuantSpec().validate_supported()
    for bad in ({"format": "w4a8"}, {"format": "asym_w4a8_int8", "group_size": 12},
                {"format": "asym_w4a8_int8", "convrot": False},
                {"format": "asym_w4a8_int8", "convrot_groupsize": 128}):
        with pytest.raises(ValueError):
            h3.W4A8QuantSpec.from_mapping(bad).validate_supported()
    n, k, gs = 64, 512, 16
    g = torch.Generator().manual_seed(0)
    tensors = {
        "blk.fc.weight": torch.randint(-128, 128, (n, k // 2), generator=g, dtype=torch.int8),
        "blk.fc.weight_s_rel": (torch.rand(n, k // gs, generator=g) * 100 + 20).to(torch.float8_e4m3fn),
        "blk.fc.weight_s_channel": torch.rand(n, generator=g) * 1e-3,
        "blk.fc.weight_codebook": torch.linspace(-1, 1, 16),
        "blk.fc.weight_correction": torch.randn(k // gs, n, generator=g) * 1e-3,
        "blk.fc.bias": torch.randn(n, generator=g),
    }
    path = tmp_path / "w4a8.safetensors"
    save_file(tensors, str(path))
    with safe_open(str(path), framework="pt") as f:
        loaded = {key: f.get_tensor(key) for key in f.keys()}
    lin = h3.load_w4a8_linear(loaded, "blk.fc")
    assert lin.in_features == k and lin.out_features == n and lin.spec.group_size == 16
    assert lin.s_rel.dtype == torch.float8_e4m3fn and lin.correction.shape == (k // gs, n)
    with pytest.raises(KeyError):
        h3.load_w4a8_linear(loaded, "blk.other")
    bad = dict(loaded)
    bad["blk.fc.weight_correction"] = torch.zeros(n, k // gs)
    with pytest.raises(ValueError, match="correction"):
        h3.load_w4a8_linear(bad, "blk.fc")
    with pytest.raises(ValueError):
        h3.load_w4a8_linear(loaded, "blk.fc", spec={"format": "asym_w4a8_int8", "group_size": 12})


def test_constraints_carry_the_reference_validation_surface(pkg):
    """Every capability entry exposes what CK/constraints.py:127-255 reads, so
    the table registers in the reference registry unchanged, and the
    reference's validation steps give the expected verdicts on it."""
    import importlib

    from x_minimaxh3_amd import backend
    reg = importlib.import_module("x_minimaxh3_amd.registry")   # the package re-exports the instance as `registry`

    caps = backend._capabilities()
    assert caps
    for name, c in caps.items():
        assert hasattr(c, "min_compute_capability") and c.min_compute_capability is None
        assert isinstance(c.default_devices, frozenset) and isinstance(c.call_rules, tuple)
        for pname, pc in c.params.items():
            for attr in ("dtypes", "devices", "shape_rules", "check_dtype", "check_device", "check_shape"):
                assert hasattr(pc, attr), (name, pname, attr)
            for rule in pc.shape_rules:
                assert isinstance(rule, reg.ShapeRule) and rule.describe()
    c = caps["int8_linear"]
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    assert c.params["x"].check_dtype(x) and not c.params["x"].check_dtype(torch.zeros(4, dtype=torch.int8))
    assert not c.params["x"].check_device(x, c.default_devices)          # the input must be on the GPU
    assert c.params["weight_scale"].check_device(x.float(), c.default_devices)   # small operands may not be
    assert c.params["weight"].check_shape(torch.zeros(8, 64, dtype=torch.int8))
    assert not c.params["weight"].check_shape(torch.zeros(8, dtype=torch.int8))
    r = reg.validate_function_call(c, {"x": x}, (9, 5))
    assert not r.success and r.failed_param == "x" and "device cpu" in r.failure_reason
    need = reg.FunctionConstraints(params={}, min_compute_capability=(9, 5))
    assert reg.validate_function_call(need, {}, (9, 5)).success
    assert reg.validate_function_call(need, {}, (9, 4)).failed_param == "__hardware__"
    assert reg.validate_function_call(need, {}, None).failed_param == "__hardware__"


def test_host_tensors_raise_before_any_kernel_call(pkg, monkeypatch):
    """A host tensor in a data, output or workspace slot raises ValueError
    before the C ABI is reached (a host pointer handed to a kernel would fault
    the GPU)."""
    from x_minimaxh3_amd import backend

    def no_call(*a, **k):
        raise AssertionError("the C ABI was reached")

    monkeypatch.setattr(backend, "call", no_call)
    x = torch.randn(4, 256).bfloat16()
    w8 = torch.zeros(8, 256, dtype=torch.int8)
    tab = torch.zeros(1, 4, 1, 64, 2, 2)
    q4 = torch.randn(1, 4, 2, 128).bfloat16()
    cases = [
        lambda: backend.quantize_int8_rowwise(x),
        lambda: backend.int8_linear(x, w8, torch.ones(8)),
        lambda: backend.w8a8_mlp(x, torch.zeros(512, 256, dtype=torch.int8), torch.ones(512),
                                 torch.zeros(256, 512, dtype=torch.int8), torch.ones(256)),
        lambda: backend.rms_adaln(x, x[:1], x[:1]),
        lambda: backend.rms_adaln_rows(x, None, x[:2], x[:2], torch.zeros(4, dtype=torch.int32), 1e-5),
        lambda: backend.norm_rope(x.reshape(4, 256), x.reshape(4, 256), x[:1], x[:1], tab, 1e-6, 128),
        lambda: backend.apply_rope_split_half1_(q4, tab),
        lambda: backend.rms_rope_split_half_(q4, q4.clone(), tab, torch.ones(128).bfloat16()),
        lambda: backend.dequant_int4_grouped_to_int8(torch.zeros(8, 128, dtype=torch.int8),
                                                     torch.ones(8, 2), None, 128),
        lambda: backend.int8_linear_gated_residual_(x, w8, torch.ones(8), None, torch.zeros(4, 8).bfloat16(),
                                                    torch.ones(1, 8), torch.zeros(4, dtype=torch.int32),
                                                    convrot=False, input_act=None),
    ]
    for i, f in enumerate(cases):
        with pytest.raises(ValueError, match="runs on the GPU"):
            f()
    # an output or workspace on another device than the input
    meta = torch.empty(4, 256, dtype=torch.bfloat16, device="meta")
    with pytest.raises(ValueError, match="out is on cpu"):
        backend._same_device(meta.device, out=torch.empty(4, 256))


def test_segment_rows_resolve_like_tensor_indexing(pkg):
    """h3.segment_row_map with the table's row count resolves rows as the
    reference's scale[row] does: negative rows count from the end, rows out
    of range raise IndexError (never a read past the table)."""
    from x_minimaxh3_amd import h3

    m = h3.segment_row_map(10, ((0, 4, -1), (4, 10, 0)), "cpu", n_rows=3)
    assert m.tolist() == [2] * 4 + [0] * 6
    with pytest.raises(IndexError, match="out of bounds"):
        h3.segment_row_map(10, ((0, 4, 3), (4, 10, 0)), "cpu", n_rows=3)
    with pytest.raises(IndexError):
        h3.segment_row_map(10, ((0, 4, -4), (4, 10, 0)), "cpu", n_rows=3)
    with pytest.raises(ValueError, match="ordered partition"):
        h3.segment_row_map(10, ((0, 4, 0), (5, 10, 0)), "cpu", n_rows=3)


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus 2 exits with a message and a
    non-zero status before any device work (no JSON line is printed)."""
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=root)
    assert r.returncode != 0
    assert "one GPU" in r.stdout + r.stderr
    assert not any(line.startswith("{") for line in r.stdout.splitlines())
