"""GPU parity of the HIP path (through the C ABI) against the CPU oracle.

Bars: int8 codes and int32 accumulators bit-exact; deterministic elementwise
epilogues (dequant, rotation) bit-exact given identical inputs; bf16 outputs
that pass through a reduction or a transcendental within max-abs 2e-2 and
cosine >= 0.9999 (the tolerance the hot path is specified with), with the
GELU-stage mismatch rate reported.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import cpu_ref

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MIN_COS = 0.9999


def say(msg):
    print(msg, flush=True)


def cos_sim(a, b):
    a, b = a.double().flatten(), b.double().flatten()
    return (a @ b / (a.norm() * b.norm())).item()


def close(got, want, what):
    got = got.cpu()
    d = (got.float() - want.float()).abs().max().item() if want.numel() else 0.0
    c = cos_sim(got, want) if want.numel() and want.float().abs().max() > 0 else 1.0
    exact = (got == want).float().mean().item() if want.numel() else 1.0
    say(f"  {what}: max|d|={d:.3e} cos={c:.7f} exact={exact:.5f}")
    assert d <= MAX_ABS and c >= MIN_COS, (what, d, c)


def same(got, want, what=""):
    """Bit-exact check that prints a few mismatching elements on failure."""
    got = got.cpu()
    eq = torch.equal(got, want)
    if not eq:
        idx = (got != want).nonzero()[:6]
        say(f"  {what} mismatches: {(got != want).sum().item()} of {want.numel()}")
        for i in idx.tolist():
            say(f"    at {i}: got {got[tuple(i)].item()!r} want {want[tuple(i)].item()!r}")
    return eq


def outlier_acts(m, k, seed=0, n_out=8, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g)
    x[:, torch.randperm(k, generator=g)[:n_out]] *= 20
    return x.to(dtype)


# --------------------------------------------------------------------------- quantizer

@pytest.mark.parametrize("m,k,dtype", [
    (25200, 5120, torch.bfloat16),   # fc1 input of the 720p MLP
    (999, 13824, torch.bfloat16),    # fc2 width (four waves per row)
    (7, 9000, torch.float16),        # four waves per row, uneven quarters
    (3, 8704, torch.float32),        # four waves per row, fp32 rows
    (513, 3072, torch.bfloat16),     # four waves per row, two steps each
    (65, 7680, torch.float16),       # four waves per row, four steps each
    (9, 11264, torch.bfloat16),      # four waves per row, six steps each
    (37, 1536, torch.float16),
    (33, 520, torch.float32),
    (7, 20000, torch.bfloat16),      # wider than the register path
    (5, 100, torch.bfloat16),        # K not a multiple of 8
])
def test_quantize_bit_exact(pkg, dev, m, k, dtype):
    say(f"quantize m={m} k={k} {dtype}")
    x = outlier_acts(m, k, seed=m, dtype=dtype)
    x[0] = 0                                  # zero row -> scale 1e-30, codes 0
    q, s = pkg.quantize_int8_rowwise(x.to(dev))
    torch.cuda.synchronize()
    qr, sr = cpu_ref.quantize_int8_rowwise(x)
    assert torch.equal(s.cpu(), sr)
    assert torch.equal(q.cpu(), qr), (q.cpu() != qr).sum().item()


@pytest.mark.parametrize("shape,dtype,seed,strided", [
    ((300, 1536), torch.bfloat16, 1, False),
    ((2, 150, 777), torch.bfloat16, (9 << 32) + 12345, False),   # 3-D, ragged K, seed past 2^32
    ((64, 5120), torch.float16, 42, False),
    ((33, 520), torch.float32, 7, False),
    ((40, 1000), torch.bfloat16, 3, True),                       # row stride 1024
    ((1, 13824), torch.bfloat16, 2 ** 64 - 5, False),           # the index + seed wraps
])
def test_quantize_stochastic_bit_exact(pkg, dev, shape, dtype, seed, strided):
    """stochastic_rounding=seed: codes and scales equal the oracle's (the
    reference CUDA quantizer's hash noise, one rounding of the sum to the row
    dtype, floor), including 3-D inputs, a strided view and seeds whose
    64-bit key wraps or folds its high word."""
    say(f"quantize stochastic {shape} {dtype} seed={seed} strided={strided}")
    g = torch.Generator().manual_seed(len(shape) * 1000 + shape[-1])
    x = torch.randn(*shape, generator=g)
    x[..., : max(1, shape[-1] // 100)] *= 20
    x = x.to(dtype)
    xd = x.to(dev)
    if strided:
        wide = torch.zeros(shape[0], 1024, dtype=dtype, device=dev)
        wide[:, : shape[-1]] = xd
        xd = wide[:, : shape[-1]]
    q, s = pkg.quantize_int8_rowwise(xd, stochastic_rounding=seed)
    torch.cuda.synchronize()
    qr, sr = cpu_ref.quantize_int8_rowwise(x, seed)
    assert torch.equal(s.cpu(), sr)
    assert same(q, qr, "stochastic codes")
    q0, _ = pkg.quantize_int8_rowwise(xd)
    assert not torch.equal(q.cpu(), q0.cpu())


def test_quantize_minus_128_cases(pkg, dev):
    say("quantize -128 cases")
    vals = torch.arange(0x3f80, 0x4000, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    x = torch.stack((-vals.float(), vals.float(), vals.float() * 0.5), dim=1).to(torch.bfloat16)
    q, s = pkg.quantize_int8_rowwise(x.to(dev))
    qr, sr = cpu_ref.quantize_int8_rowwise(x)
    assert (qr[:, 0] == -128).any()
    assert torch.equal(q.cpu(), qr) and torch.equal(s.cpu(), sr)


def test_quantize_with_gelu_input_act(pkg, dev):
    say("quantize gelu input act")
    from x_minimaxh3_amd import backend

    h = outlier_acts(513, 13824, seed=3) * 0.5   # fc2 width: four waves per row, GELU in registers
    q, s = backend._quantize(h.to(dev), 1)
    torch.cuda.synchronize()
    g = cpu_ref.gelu_tanh(h)
    qr, sr = cpu_ref.quantize_int8_rowwise(g)
    mism = (q.cpu() != qr).float().mean().item()
    dq = (q.cpu().int() - qr.int()).abs().max().item()
    say(f"  gelu->int8 code mismatch rate {mism:.2e}, max code delta {dq}")
    assert torch.allclose(s.cpu(), sr, rtol=2 ** -7, atol=0)
    assert mism < 1e-3 and dq <= 1


# --------------------------------------------------------------------------- GEMM

@pytest.mark.parametrize("m,n,k", [
    (1024, 6144, 1536),     # the small MLP's fc1
    (300, 200, 272),        # tails in every dim, K % 128 != 0
    (256, 256, 128),
    (1, 16, 16),
    (777, 5120, 13824),     # fc2 shape, ragged M
])
def test_gemm_int32_bit_exact(pkg, dev, m, n, k):
    say(f"gemm int32 m={m} n={n} k={k}")
    from x_minimaxh3_amd import backend

    g = torch.Generator().manual_seed(m + n + k)
    a = torch.randint(-128, 128, (m, k), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8)
    a[0] = -128
    w[0] = -128
    acc = backend._gemm(a.to(dev), None, w.to(dev), None, None, torch.float32, epilogue=2)
    torch.cuda.synchronize()
    assert torch.equal(acc.cpu(), cpu_ref.int8_mm(a, w))


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("per_channel,with_bias", [(True, False), (False, True), (True, True)])
def test_int8_linear_bit_exact(pkg, dev, out_dtype, per_channel, with_bias):
    say(f"int8_linear {out_dtype} per_channel={per_channel} bias={with_bias}")
    x = outlier_acts(389, 1536, seed=1)
    g = torch.Generator().manual_seed(2)
    w = torch.randint(-127, 128, (640, 1536), generator=g, dtype=torch.int8)
    sw = torch.rand(640 if per_channel else 1, generator=g) * 1e-3
    bias = torch.randn(640, generator=g).to(out_dtype) if with_bias else None
    y = pkg.int8_linear(x.to(dev), w.to(dev), sw.to(dev), None if bias is None else bias.to(dev), out_dtype)
    torch.cuda.synchronize()
    yr = cpu_ref.int8_linear(x, w, sw, bias=bias, out_dtype=out_dtype)
    assert y.dtype == out_dtype
    assert same(y, yr, "int8_linear")


def test_dequant_bf16_ties_round_to_even(pkg, dev):
    """acc = n with unit scales: bf16 has 8 significant bits, so every odd
    n in (256, 512) lies exactly halfway between two bf16 values; the epilogue
    must round those ties to even like the reference's fp32 -> bf16 cast."""
    say("dequant bf16 ties")
    from x_minimaxh3_amd import backend

    k = 512
    a = torch.ones(4, k, dtype=torch.int8)
    w = (torch.arange(k).view(1, -1) < torch.arange(k).view(-1, 1)).to(torch.int8)   # row n has n ones
    one = torch.ones(1)
    out = backend._gemm(a.to(dev), one.expand(4).contiguous().to(dev), w.to(dev), one.to(dev), None,
                        torch.bfloat16)
    torch.cuda.synchronize()
    want = cpu_ref.dequant(cpu_ref.int8_mm(a, w), one.expand(4).reshape(-1, 1), one)
    assert want[0, 257].item() == 256.0 and want[0, 259].item() == 260.0
    assert same(out, want, "ties")


def test_int8_linear_leading_dims_and_strided_input(pkg, dev):
    say("int8_linear 3D / strided")
    x = outlier_acts(2 * 65, 512, seed=4).reshape(2, 65, 512)
    big = torch.zeros(2, 65, 640, dtype=torch.bfloat16)
    big[..., :512] = x
    w = torch.randint(-127, 128, (96, 512), dtype=torch.int8)
    sw = torch.rand(96) * 1e-3
    y = pkg.int8_linear(big.to(dev)[..., :512], w.to(dev), sw.to(dev))
    torch.cuda.synchronize()
    assert y.shape == (2, 65, 96)
    assert torch.equal(y.cpu(), cpu_ref.int8_linear(x, w, sw))


def test_int8_linear_gelu_input_act(pkg, dev):
    say("int8_linear input_act=gelu_tanh")
    h = outlier_acts(300, 2048, seed=5) * 0.3
    w = torch.randint(-127, 128, (256, 2048), dtype=torch.int8)
    sw = torch.rand(256) * 1e-3
    y = pkg.int8_linear(h.to(dev), w.to(dev), sw.to(dev), input_act="gelu_tanh")
    torch.cuda.synchronize()
    close(y, cpu_ref.int8_linear(h, w, sw, input_act="gelu_tanh"), "int8_linear(gelu)")


# --------------------------------------------------------------------------- MLP

def _mlp_stages(pkg, dev, inp):
    """The MLP as the GELU-epilogue chain (fc1 epilogue 1 with the row |max|,
    then the requant entry point), one kernel at a time through the C ABI,
    returning every intermediate."""
    from x_minimaxh3_amd import _lib

    x = inp["x"].to(dev)
    w1, s1, w2, s2 = (inp[k].to(dev) for k in ("w1", "s1", "w2", "s2"))
    m, d = x.shape
    f = w1.shape[0]
    st = _lib.stream_of(x)
    q1 = torch.empty(m, d, dtype=torch.int8, device=dev)
    sx = torch.empty(m, dtype=torch.float32, device=dev)
    g = torch.empty(m, f, dtype=torch.bfloat16, device=dev)
    amax = torch.full((m,), -1, dtype=torch.int32, device=dev)      # cleared by the quant kernel
    _lib.call("xmh3_quantize_int8_rowwise_ex", x.data_ptr(), 2, 0, m, d, d, q1.data_ptr(), sx.data_ptr(),
              amax.data_ptr(), st)
    _lib.call("xmh3_int8_gemm", q1.data_ptr(), d, w1.data_ptr(), d, m, f, d, sx.data_ptr(), s1.data_ptr(), 1,
              None, g.data_ptr(), 2, f, 1, amax.data_ptr(), st)
    q2 = torch.empty(m, f, dtype=torch.int8, device=dev)
    sg = torch.empty(m, dtype=torch.float32, device=dev)
    _lib.call("xmh3_requant_int8_rows", g.data_ptr(), 2, m, f, f, amax.data_ptr(), q2.data_ptr(), sg.data_ptr(), st)
    y = torch.empty(m, d, dtype=torch.bfloat16, device=dev)
    _lib.call("xmh3_int8_gemm", q2.data_ptr(), f, w2.data_ptr(), f, m, d, f, sg.data_ptr(), s2.data_ptr(), 1,
              None, y.data_ptr(), 2, d, 0, None, st)
    torch.cuda.synchronize()
    return {"q1": q1.cpu(), "sx": sx.cpu(), "g": g.cpu(), "amax": amax.cpu().view(torch.float32),
            "q2": q2.cpu(), "sg": sg.cpu(), "y": y.cpu()}


def test_mlp_small_stagewise(pkg, dev):
    say("w8a8 mlp 1024x1536x6144 stagewise")
    from x_minimaxh3_amd import workloads

    inp = workloads.mlp_inputs(**workloads.CONFIGS["mlp_small"], seed=0)
    st = _mlp_stages(pkg, dev, inp)
    yr, p = cpu_ref.w8a8_mlp(inp["x"], inp["w1"], inp["s1"], inp["w2"], inp["s2"], return_parts=True)
    assert torch.equal(st["q1"], p["q1"]) and torch.equal(st["sx"], p["s1"].reshape(-1))
    # fc1 epilogue: h = bf16(acc*(sx*sw)) is exact; g = bf16(gelu(h)) uses the device tanh
    g_ref = cpu_ref.gelu_tanh(p["h"])
    gm = (st["g"] != g_ref).float().mean().item()
    ulp = cpu_ref.bf16_ulp_diff(st["g"], g_ref)
    big = g_ref.float().abs() > 1e-3
    say(f"  gelu stage: mismatch rate {gm:.2e}, max ulp (|g|>1e-3) {ulp[big].max().item():.1f}")
    assert ulp[big].max().item() <= 1.0 and gm < 1e-2
    # row amax is exactly max|g| of the GPU's own g
    assert torch.equal(st["amax"], st["g"].float().abs().amax(dim=1))
    # requant of the GPU's g is bit-exact against the oracle quantizer on that g
    q2r, s2r = cpu_ref.quantize_int8_rowwise(st["g"])
    assert torch.equal(st["q2"], q2r) and torch.equal(st["sg"], s2r.reshape(-1))
    # fc2 + dequant bit-exact given the GPU's q2
    yr2 = cpu_ref.dequant(cpu_ref.int8_mm(st["q2"], inp["w2"]), st["sg"], inp["s2"])
    assert torch.equal(st["y"], yr2)
    q2_mism = (st["q2"] != p["q2"]).float().mean().item()
    say(f"  requant code mismatch vs oracle end-to-end: {q2_mism:.2e}")
    close(st["y"], yr, "mlp output")


def test_mlp_small_quantizer_gelu_chain(pkg, dev):
    """The chain xmh3_w8a8_mlp runs: quant -> fc1 with the dequant epilogue
    (h) -> per-token quant with the GELU input act -> fc2; every stage against
    the oracle, and the fused entry point equal to the stages bit for bit."""
    say("w8a8 mlp 1024x1536x6144: quantizer-GELU chain stagewise")
    from x_minimaxh3_amd import _lib

    from x_minimaxh3_amd import workloads

    inp = workloads.mlp_inputs(**workloads.CONFIGS["mlp_small"], seed=0)
    yr, p = cpu_ref.w8a8_mlp(inp["x"], inp["w1"], inp["s1"], inp["w2"], inp["s2"], return_parts=True)
    x = inp["x"].to(dev)
    w1, s1, w2, s2 = (inp[k].to(dev) for k in ("w1", "s1", "w2", "s2"))
    m, d = x.shape
    f = w1.shape[0]
    st = _lib.stream_of(x)
    q1 = torch.empty(m, d, dtype=torch.int8, device=dev)
    sx = torch.empty(m, dtype=torch.float32, device=dev)
    h = torch.empty(m, f, dtype=torch.bfloat16, device=dev)
    q2 = torch.empty(m, f, dtype=torch.int8, device=dev)
    sg = torch.empty(m, dtype=torch.float32, device=dev)
    y = torch.empty(m, d, dtype=torch.bfloat16, device=dev)
    _lib.call("xmh3_quantize_int8_rowwise", x.data_ptr(), 2, 0, m, d, d, q1.data_ptr(), sx.data_ptr(), st)
    _lib.call("xmh3_int8_gemm", q1.data_ptr(), d, w1.data_ptr(), d, m, f, d, sx.data_ptr(), s1.data_ptr(), 1,
              None, h.data_ptr(), 2, f, 0, None, st)
    _lib.call("xmh3_quantize_int8_rowwise", h.data_ptr(), 2, 1, m, f, f, q2.data_ptr(), sg.data_ptr(), st)
    _lib.call("xmh3_int8_gemm", q2.data_ptr(), f, w2.data_ptr(), f, m, d, f, sg.data_ptr(), s2.data_ptr(), 1,
              None, y.data_ptr(), 2, d, 0, None, st)
    yf = pkg.w8a8_mlp(x, w1, s1, w2, s2)
    torch.cuda.synchronize()
    assert same(q1, p["q1"], "q1") and same(h, p["h"], "h")
    g_ref = cpu_ref.gelu_tanh(p["h"])
    q2r, s2r = cpu_ref.quantize_int8_rowwise(g_ref)
    mism, dq = _code_stats(q2, q2r, "gelu quant codes")
    assert mism < 1e-3 and dq <= 1
    assert torch.allclose(sg.cpu(), s2r.reshape(-1), rtol=2 ** -7, atol=0)
    yr2 = cpu_ref.dequant(cpu_ref.int8_mm(q2.cpu(), inp["w2"]), sg.cpu(), inp["s2"])
    assert same(y, yr2, "fc2 given the GPU's q2")
    assert same(yf, y.cpu(), "fused entry point vs stages")
    close(y, yr, "mlp output")


def test_mlp_fused_op_small(pkg, dev):
    say("w8a8 mlp fused op 1024x1536x6144")
    from x_minimaxh3_amd import workloads

    inp = workloads.mlp_inputs(**workloads.CONFIGS["mlp_small"], seed=0)
    y = pkg.w8a8_mlp(*(inp[k].to(dev) for k in ("x", "w1", "s1", "w2", "s2")))
    torch.cuda.synchronize()
    st = _mlp_stages(pkg, dev, inp)
    assert torch.equal(y.cpu(), st["y"])       # the fused op runs the same kernels
    close(y, cpu_ref.w8a8_mlp(inp["x"], inp["w1"], inp["s1"], inp["w2"], inp["s2"]), "fused mlp")


def test_mlp_720p_row_sample(pkg, dev):
    """Full 720p shape on the GPU; rows are independent (per-token quant), so
    the oracle checks a sample of rows including the partial last tile."""
    say("w8a8 mlp 25200x5120x13824")
    from x_minimaxh3_amd import workloads

    inp = workloads.mlp_inputs(**workloads.CONFIGS["mlp_720p"], seed=0)
    y = pkg.w8a8_mlp(*(inp[k].to(dev) for k in ("x", "w1", "s1", "w2", "s2"))).cpu()
    g = torch.Generator().manual_seed(1)
    rows = torch.cat((torch.randperm(25200 - 200, generator=g)[:200], torch.arange(25200 - 200, 25200)))
    yr = cpu_ref.w8a8_mlp(inp["x"][rows], inp["w1"], inp["s1"], inp["w2"], inp["s2"])
    close(y[rows], yr, "720p mlp rows")
    assert torch.isfinite(y.float()).all()


def test_w4_decode_bit_exact(pkg, dev):
    say("w4 decode")
    from x_minimaxh3_amd import backend

    g = torch.Generator().manual_seed(8)
    w = torch.randn(384, 1024, generator=g) * 0.02
    for gs in (128, 64, 32, 16, 8):
        packed, srel, _ = cpu_ref.quantize_w4_weight(w, gs)
        # x40: most levels saturate at +-127; the clamp and the rounding must
        # still agree with the oracle's rint-then-clamp
        for srel_t in (srel, srel.to(torch.bfloat16), srel * 40):
            out = backend.dequant_int4_grouped_to_int8(packed.to(dev), srel_t.to(dev), None, gs)
            torch.cuda.synchronize()
            assert torch.equal(out.cpu(), cpu_ref.dequant_int4_grouped_to_int8(packed, srel_t.float(), gs))
    cb = torch.linspace(-1, 1, 16) * 7.3
    packed, srel, _ = cpu_ref.quantize_w4_weight(w, 128)
    out = backend.dequant_int4_grouped_to_int8(packed.to(dev), srel.to(dev), cb.to(dev), 128)
    assert torch.equal(out.cpu(), cpu_ref.dequant_int4_grouped_to_int8(packed, srel, 128, codebook=cb))


def test_w4a8_linear_and_mlp(pkg, dev):
    say("w4a8 linear + mlp 1024x1536x6144")
    from x_minimaxh3_amd import workloads

    inp = workloads.mlp_inputs(**workloads.CONFIGS["mlp_small"], seed=0, weights="w4a8")
    x = inp["x"]
    y = pkg.w4a8_int8_linear(x.to(dev), inp["w1_packed"].to(dev), inp["w1_srel"].to(dev),
                             inp["w1_schannel"].to(dev), group_size=128, convrot_groupsize=128, convrot=False)
    torch.cuda.synchronize()
    yr = cpu_ref.w4a8_linear(x, inp["w1_packed"], inp["w1_srel"].float(), inp["w1_schannel"], 128)
    assert torch.equal(y.cpu(), yr)
    ym = pkg.w4a8_mlp(x.to(dev), *(inp[k].to(dev) for k in ("w1_packed", "w1_srel", "w1_schannel",
                                                             "w2_packed", "w2_srel", "w2_schannel")), 128)
    torch.cuda.synchronize()
    ymr = cpu_ref.w4a8_mlp(x, inp["w1_packed"], inp["w1_srel"].float(), inp["w1_schannel"],
                           inp["w2_packed"], inp["w2_srel"].float(), inp["w2_schannel"], 128)
    close(ym, ymr, "w4a8 mlp")


@pytest.mark.parametrize("m", [500, 1000, 2000])
def test_w4a8_mlp_decoded_weights_share_the_workspace(pkg, dev, m):
    """The W4A8 MLP decodes W1 into q2's workspace region and W2 into h's when
    they fit (d=1536: W1 needs m >= 1536, W2 m >= 768), else into segments of
    their own: at all three token counts it equals the W8A8 MLP on the decoded
    weights bit for bit, from a workspace filled with garbage."""
    say(f"w4a8 mlp workspace sharing m={m}")
    from x_minimaxh3_amd import _lib, backend, workloads

    inp = workloads.mlp_inputs(**workloads.CONFIGS["mlp_small"], seed=1, weights="w4a8")
    x = inp["x"][:m].to(dev)
    w = {k: inp[k].to(dev) for k in ("w1_packed", "w1_srel", "w1_schannel", "w2_packed", "w2_srel", "w2_schannel")}
    d, f = x.shape[1], w["w1_packed"].shape[0]
    nbytes = _lib.load().xmh3_w4a8_mlp_workspace_bytes(m, d, f, 128)
    assert (nbytes == _lib.load().xmh3_w8a8_mlp_workspace_bytes(m, d, f)) == (m >= d)
    ws = torch.full((nbytes,), 0x5A, dtype=torch.uint8, device=dev)
    y = backend.w4a8_mlp(x, *w.values(), 128, workspace=ws)
    w1 = backend.dequant_int4_grouped_to_int8(w["w1_packed"], w["w1_srel"], None, 128)
    w2 = backend.dequant_int4_grouped_to_int8(w["w2_packed"], w["w2_srel"], None, 128)
    want = backend.w8a8_mlp(x, w1, w["w1_schannel"], w2, w["w2_schannel"])
    torch.cuda.synchronize()
    assert same(y, want.cpu(), "w4a8 mlp vs w8a8 mlp on the decoded weights")


@pytest.mark.parametrize("m,n,k,srel_dtype,srel_pad,bias", [
    (777, 1000, 768, torch.bfloat16, 1, False),
    (300, 512, 1024, torch.float32, 0, True),
    (256, 256, 256, torch.bfloat16, 0, False),
    (1030, 2304, 5120, torch.bfloat16, 3, True),
])
def test_w4a8_gemm_lds_decode(pkg, dev, m, n, k, srel_dtype, srel_pad, bias):
    """xmh3_w4a8_gemm (int4 codes unpacked in LDS inside the GEMM, group 128)
    against the oracle's decode + int8 linear, bit for bit: ragged M and N,
    bf16 / fp32 s_rel, s_rel rows padded to an odd stride (bf16 values in both
    halves of their dwords), optional bias."""
    say(f"w4a8 gemm lds decode m={m} n={n} k={k} s_rel={srel_dtype} pad={srel_pad} bias={bias}")
    from x_minimaxh3_amd import _lib, workloads

    g = torch.Generator().manual_seed(m + n)
    x = outlier_acts(m, k, seed=n)
    w = torch.randn(n, k, generator=g) * 0.02
    packed, srel, sch = workloads.quantize_weight_w4(w, 128, srel_dtype)
    wide = torch.zeros(n, k // 128 + srel_pad, dtype=srel_dtype)
    wide[:, : k // 128] = srel
    srel_v = wide.to(dev)[:, : k // 128]                      # row stride k/128 + pad
    b = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16) if bias else None
    q, xs = cpu_ref.quantize_int8_rowwise(x)
    qd, xsd = q.to(dev), xs.to(dev)
    pd, schd = packed.to(dev), sch.to(dev)
    bd = None if b is None else b.to(dev)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
    rc = _lib.load().xmh3_w4a8_gemm(qd.data_ptr(), k, pd.data_ptr(), k // 2, srel_v.data_ptr(),
                                    _lib.DTYPE_CODE[srel_dtype], srel_v.stride(0), m, n, k, 128, xsd.data_ptr(),
                                    schd.data_ptr(), None if bd is None else bd.data_ptr(), out.data_ptr(), 2, n,
                                    _lib.stream_of(qd))
    assert rc == 0, _lib.load().xmh3_last_error()
    torch.cuda.synchronize()
    want = cpu_ref.w4a8_linear(x, packed, srel.float(), sch, 128, bias=b)
    assert same(out, want, "w4a8 gemm")
    if not srel_pad:
        # the torch-facing wrapper and the decode-once linear agree with it
        from x_minimaxh3_amd import backend
        got = backend.w4a8_linear_lds_decode(x.to(dev), pd, srel.to(dev), schd, bd)
        ref = pkg.w4a8_int8_linear(x.to(dev), pd, srel.to(dev), schd, bias=bd, group_size=128, convrot=False)
        assert same(got, want, "lds-decode wrapper") and same(ref, want, "decode-once linear")


def test_w4a8_mlp_720p_row_sample(pkg, dev):
    """C4 at its full shape: 25,200 tokens, 5120 -> 13824 -> 5120, int4 group
    128 (40 groups along fc1's K, 108 along fc2's), bf16 s_rel. Both linears
    alone are bit-exact on sampled rows; the MLP is checked on 400 rows
    including the last, partial row tile."""
    say("w4a8 mlp 25200x5120x13824 g128")
    from x_minimaxh3_amd import workloads

    inp = workloads.mlp_inputs(**workloads.CONFIGS["mlp_720p"], seed=0, weights="w4a8")
    names = ("w1_packed", "w1_srel", "w1_schannel", "w2_packed", "w2_srel", "w2_schannel")
    w = {n: inp[n].to(dev) for n in names}
    x = inp["x"]
    g = torch.Generator().manual_seed(2)
    rows = torch.cat((torch.randperm(25200 - 200, generator=g)[:200], torch.arange(25200 - 200, 25200)))
    y = pkg.w4a8_mlp(x.to(dev), *(w[n] for n in names), 128).cpu()
    yr = cpu_ref.w4a8_mlp(x[rows], inp["w1_packed"], inp["w1_srel"].float(), inp["w1_schannel"],
                          inp["w2_packed"], inp["w2_srel"].float(), inp["w2_schannel"], 128)
    close(y[rows], yr, "720p w4a8 mlp rows")
    assert torch.isfinite(y.float()).all()
    say("w4a8 linear K=5120 (40 groups) and K=13824 (108 groups)")
    h = pkg.w4a8_int8_linear(x[rows].to(dev), w["w1_packed"], w["w1_srel"], w["w1_schannel"], group_size=128,
                             convrot_groupsize=128, convrot=False).cpu()
    assert same(h, cpu_ref.w4a8_linear(x[rows], inp["w1_packed"], inp["w1_srel"].float(), inp["w1_schannel"], 128),
         "w4a8 fc1 rows")
    x2 = (torch.randn(300, 13824, generator=g) * 0.3).to(torch.bfloat16)
    y2 = pkg.w4a8_int8_linear(x2.to(dev), w["w2_packed"], w["w2_srel"], w["w2_schannel"], group_size=128,
                              convrot_groupsize=128, convrot=False).cpu()
    assert same(y2, cpu_ref.w4a8_linear(x2, inp["w2_packed"], inp["w2_srel"].float(), inp["w2_schannel"], 128),
         "w4a8 fc2 rows")


# --------------------------------------------------------------------------- norm / rope

def test_norm_rope_720p(pkg, dev):
    say("norm_rope 25200x5120")
    from x_minimaxh3_amd import workloads

    nr = workloads.norm_rope_inputs(grid=(7, 45, 80))
    qo, ko = pkg.norm_rope(nr["q"].to(dev), nr["k"].to(dev), nr["scale"].to(dev), nr["shift"].to(dev),
                           nr["freqs"].to(dev), nr["eps"], 128)
    torch.cuda.synchronize()
    for got, x, name in ((qo, nr["q"], "Q"), (ko, nr["k"], "K")):
        want = cpu_ref.norm_rope(x, nr["scale"], nr["shift"], nr["freqs"], 128, nr["eps"])
        close(got, want, f"norm_rope {name}")
        assert same(got, want, f"norm_rope {name}")   # reference reduction order -> bit exact


@pytest.mark.parametrize("grid", [(7, 45, 80), (1, 20, 50), (1, 1, 37)])
def test_norm_rope_in_place(pkg, dev, grid):
    """The cooperative norm-rope in place: at 720p 65 or 66 row groups per
    block (with and without the redo of a block's last iteration) and the
    last partial group; 1000 tokens give 2 or 3 row groups per block, 37
    tokens one. Equal to the out-of-place result bit for bit."""
    say(f"norm_rope grid {grid} in place")
    from x_minimaxh3_amd import backend, workloads

    nr = workloads.norm_rope_inputs(grid=grid)
    qd, kd = nr["q"].to(dev), nr["k"].to(dev)
    scd, shd, fd = nr["scale"].to(dev), nr["shift"].to(dev), nr["freqs"].to(dev)
    qo, ko = backend.norm_rope(qd, kd, scd, shd, fd, nr["eps"], 128)
    qi, ki = qd.clone(), kd.clone()
    backend.norm_rope(qi, ki, scd, shd, fd, nr["eps"], 128, inplace=True)
    torch.cuda.synchronize()
    assert torch.equal(qi, qo) and torch.equal(ki, ko)


@pytest.mark.parametrize("d,m,with_k,tab_dtype,bcast,dtype", [
    (5120, 37, True, torch.float32, False, torch.bfloat16),    # cooperative kernel, fewer tokens than blocks
    (5120, 1000, True, torch.float32, False, torch.bfloat16),   # 2 or 3 row groups per block
    (2048, 1900, True, torch.float32, False, torch.bfloat16),   # 3 or 4 row groups per block
    (5120, 1000, False, torch.float32, False, torch.bfloat16),  # Q only
    (3072, 1000, True, torch.bfloat16, False, torch.bfloat16),  # bf16 table
    (1024, 4099, True, torch.float32, True, torch.bfloat16),    # one broadcast table row
    (4096, 1, True, torch.float32, False, torch.bfloat16),      # a single token
    (8192, 333, True, torch.float32, False, torch.bfloat16),    # 16 waves per block
    (8192, 120, False, torch.float32, False, torch.bfloat16),   # Q only, 8 waves per row
    (2048, 700, True, torch.float16, False, torch.float16),     # fp16 rows and table
    (5120, 257, True, torch.float32, False, torch.float16),     # fp16 rows, fp32 table
    (1536, 300, True, torch.float32, False, torch.bfloat16),    # width not a multiple of 1024 -> row kernel
])
def test_norm_rope_shapes(pkg, dev, d, m, with_k, tab_dtype, bcast, dtype):
    say(f"norm_rope d={d} m={m} k={with_k} table={tab_dtype} broadcast={bcast} x={dtype}")
    g = torch.Generator().manual_seed(d + m)
    q = torch.randn(m, d, generator=g).to(dtype)
    k = torch.randn(m, d, generator=g).to(dtype)
    scale = (torch.randn(1, d, generator=g) * 0.1).to(dtype)
    shift = (torch.randn(1, d, generator=g) * 0.1).to(dtype)
    ang = torch.rand(1, 1 if bcast else m, 1, 64, generator=g) * 40
    c, s = torch.cos(ang), torch.sin(ang)
    tab = torch.stack((c, -s, s, c), -1).reshape(1, ang.shape[1], 1, 64, 2, 2).to(tab_dtype)
    from x_minimaxh3_amd import backend

    qo, ko = backend.norm_rope(q.to(dev), k.to(dev) if with_k else None, scale.to(dev), shift.to(dev),
                               tab.to(dev), 1e-6, 128)
    torch.cuda.synchronize()
    ftab = tab.expand(1, m, 1, 64, 2, 2)
    outs = ((qo, q), (ko, k)) if with_k else ((qo, q),)
    if not with_k:
        assert ko is None
    for got, x in outs:
        want = cpu_ref.norm_rope(x, scale, shift, ftab, 128, 1e-6)
        assert same(got, want, f"norm_rope d={d} m={m}")


def test_norm_rope_per_sample_modulation(pkg, dev):
    say("norm_rope with two modulation rows (two samples of 300 tokens)")
    g = torch.Generator().manual_seed(5)
    d, t = 5120, 300
    q = torch.randn(2, t, d, generator=g).to(torch.bfloat16)
    k = torch.randn(2, t, d, generator=g).to(torch.bfloat16)
    scale = (torch.randn(2, 1, d, generator=g) * 0.1).to(torch.bfloat16)
    shift = (torch.randn(2, 1, d, generator=g) * 0.1).to(torch.bfloat16)
    ang = torch.rand(1, 2 * t, 1, 64, generator=g) * 40
    c, s = torch.cos(ang), torch.sin(ang)
    tab = torch.stack((c, -s, s, c), -1).reshape(1, 2 * t, 1, 64, 2, 2)
    qo, ko = pkg.norm_rope(q.to(dev), k.to(dev), scale.to(dev), shift.to(dev), tab.to(dev), 1e-6, 128)
    torch.cuda.synchronize()
    for got, x in ((qo, q), (ko, k)):
        for b in range(2):
            want = cpu_ref.norm_rope(x[b], scale[b], shift[b], tab[:, b * t:(b + 1) * t], 128, 1e-6)
            assert same(got[b], want, f"norm_rope sample {b}")



@pytest.mark.parametrize("d,m,with_k", [(5120, 1000, True), (3072, 777, True), (2048, 300, False)])
def test_norm_rope_abi_without_modulation(pkg, dev, d, m, with_k):
    """xmh3_norm_rope with scale = shift = NULL (RMSNorm + rotation, the
    cooperative kernel without AdaLN), through the C ABI: equal to the
    oracle's norm-rope with zero scale and shift (1 + 0 and + 0 are exact)."""
    say(f"norm_rope C ABI without modulation d={d} m={m} k={with_k}")
    from x_minimaxh3_amd import _lib

    g = torch.Generator().manual_seed(d + 3 * m)
    q = torch.randn(m, d, generator=g).to(torch.bfloat16)
    k = torch.randn(m, d, generator=g).to(torch.bfloat16)
    ang = torch.rand(1, m, 1, 64, generator=g) * 40
    c, s_ = torch.cos(ang), torch.sin(ang)
    tab = torch.stack((c, -s_, s_, c), -1).reshape(1, m, 1, 64, 2, 2)
    qd, kd, td = q.to(dev), k.to(dev), tab.to(dev).contiguous()
    qo = torch.empty_like(qd)
    ko = torch.empty_like(kd) if with_k else None
    st = _lib.stream_of(qd)
    _lib.call("xmh3_norm_rope", qd.data_ptr(), qo.data_ptr(), kd.data_ptr() if with_k else None,
              ko.data_ptr() if with_k else None, 2, m, d, d, d, None, None, 2, 0, m,
              td.data_ptr(), 0, 256, 128, 1e-6, st)
    torch.cuda.synchronize()
    zero = torch.zeros(1, d, dtype=torch.bfloat16)
    for got, x in ((qo, q), (ko, k)) if with_k else ((qo, q),):
        want = cpu_ref.norm_rope(x, zero, zero, tab, 128, 1e-6)
        assert same(got, want, f"norm_rope without modulation d={d}")

def test_rope_only_bit_exact(pkg, dev):
    say("apply_rope_split_half fp32 + bf16 tables")
    g = torch.Generator().manual_seed(21)
    xq = torch.randn(2, 50, 8, 128, generator=g).to(torch.bfloat16)
    xk = torch.randn(2, 50, 8, 128, generator=g).to(torch.bfloat16)
    ang = torch.rand(1, 50, 1, 64, generator=g) * 50
    c, s = torch.cos(ang), torch.sin(ang)
    tab = torch.stack((c, -s, s, c), -1).reshape(1, 50, 1, 64, 2, 2)
    for t in (tab, tab.to(torch.bfloat16)):
        oq, ok = pkg.apply_rope_split_half(xq.to(dev), xk.to(dev), t.to(dev))
        torch.cuda.synchronize()
        assert torch.equal(oq.cpu(), cpu_ref.apply_rope_split_half1(xq, t))
        assert torch.equal(ok.cpu(), cpu_ref.apply_rope_split_half1(xk, t))
    q2 = xq.to(dev).clone()
    k2 = xk.to(dev).clone()
    pkg.apply_rope_split_half_(q2, k2, tab.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(q2.cpu(), cpu_ref.apply_rope_split_half1(xq, tab))


@pytest.mark.parametrize("heads,per_head_table", [(2, False), (8, True), (56, False)])
def test_rope_table_paths(pkg, dev, heads, per_head_table):
    """The head-span kernel stages a token's table row in LDS when every head
    shares it and a block spans few tokens; per-head tables and few heads per
    token take the direct loads. Both against the oracle, bit for bit."""
    say(f"rope table paths heads={heads} per_head_table={per_head_table}")
    g = torch.Generator().manual_seed(24 + heads)
    S, D = 45, 96
    xq = torch.randn(1, S, heads, D, generator=g).to(torch.bfloat16)
    xk = torch.randn(1, S, heads, D, generator=g).to(torch.bfloat16)
    th = heads if per_head_table else 1
    ang = torch.rand(1, S, th, D // 2, generator=g) * 40
    c, sn = torch.cos(ang), torch.sin(ang)
    tab = torch.stack((c, -sn, sn, c), -1).reshape(1, S, th, D // 2, 2, 2)
    qw = (torch.rand(D, generator=g) + 0.5).to(torch.bfloat16)
    kw = (torch.rand(D, generator=g) + 0.5).to(torch.bfloat16)
    q2, k2 = xq.to(dev), xk.to(dev)
    pkg.rms_rope_split_half_(q2, k2, tab.to(dev), qw.to(dev), kw.to(dev), 1e-5, D)
    torch.cuda.synchronize()
    assert same(q2, cpu_ref.rms_rope_split_half1(xq, tab, qw, 1e-5, D), "q")
    assert same(k2, cpu_ref.rms_rope_split_half1(xk, tab, kw, 1e-5, D), "k")


@pytest.mark.parametrize("S,H,D,tdtype,wdtype,dtype,inplace", [
    (3001, 56, 96, torch.float32, torch.bfloat16, torch.bfloat16, True),    # H3 heads, many iterations
    (517, 24, 64, torch.bfloat16, torch.float32, torch.bfloat16, False),
    (389, 40, 128, torch.float32, torch.bfloat16, torch.bfloat16, True),
    (211, 30, 96, torch.float16, torch.float16, torch.float16, False),
    (5, 7, 96, torch.float32, torch.bfloat16, torch.bfloat16, True),        # fewer heads than a part holds
    (1, 1, 64, torch.float32, torch.bfloat16, torch.bfloat16, False),       # one token, one head
    (257, 16, 64, torch.bfloat16, torch.bfloat16, torch.bfloat16, True),    # exactly one part per token
])
def test_qk_rope_pair_launch(pkg, dev, S, H, D, tdtype, wdtype, dtype, inplace):
    """Q and K through one call of the pair entry (one launch of the
    cooperative QK kernel when the strides match): full split-half rotation
    with per-head RMSNorm, distinct Q and K weights, against the oracle bit
    for bit."""
    say(f"qk rope pair S={S} H={H} D={D} table={tdtype} weight={wdtype} {dtype} inplace={inplace}")
    g = torch.Generator().manual_seed(S + H + D)
    xq = torch.randn(1, S, H, D, generator=g).to(dtype)
    xk = torch.randn(1, S, H, D, generator=g).to(dtype)
    tab = _angle_table((1, S, 1), D // 2, S + 1, tdtype)
    qw = (torch.rand(D, generator=g) + 0.5).to(wdtype)
    kw = (torch.rand(D, generator=g) + 0.5).to(wdtype)
    q2, k2 = xq.to(dev), xk.to(dev)
    if inplace:
        pkg.rms_rope_split_half_(q2, k2, tab.to(dev), qw.to(dev), kw.to(dev), 1e-5, 0)
        oq, ok = q2, k2
    else:
        oq, ok = pkg.rms_rope_split_half(q2, k2, tab.to(dev), qw.to(dev), kw.to(dev), 1e-5, 0)
    torch.cuda.synchronize()
    assert same(oq, cpu_ref.rms_rope_split_half1(xq, tab, qw, 1e-5, 0), "q")
    assert same(ok, cpu_ref.rms_rope_split_half1(xk, tab, kw, 1e-5, 0), "k")


def test_qk_rope_pair_packed_qkv_full_rotation(pkg, dev):
    """Full 128-wide rotation in place on the Q and K views of a packed QKV
    tensor (token stride 3·H·D, shared by Q and K): the pair launch with a
    token stride other than H·D; V is untouched."""
    say("rms_rope_split_half_ full rotation on packed qkv views")
    g = torch.Generator().manual_seed(31)
    S, H, D = 1031, 12, 128
    qkv = torch.randn(1, S, 3, H, D, generator=g).to(torch.bfloat16)
    tab = _angle_table((1, S, 1), D // 2, 32, torch.float32)
    qw = (torch.rand(D, generator=g) + 0.5).to(torch.bfloat16)
    kw = (torch.rand(D, generator=g) + 0.5).to(torch.bfloat16)
    dq = qkv.to(dev)
    pkg.rms_rope_split_half_(dq[:, :, 0], dq[:, :, 1], tab.to(dev), qw.to(dev), kw.to(dev), 1e-5, 0)
    torch.cuda.synchronize()
    out = dq.cpu()
    assert same(out[:, :, 0], cpu_ref.rms_rope_split_half1(qkv[:, :, 0], tab, qw, 1e-5, 0), "q")
    assert same(out[:, :, 1], cpu_ref.rms_rope_split_half1(qkv[:, :, 1], tab, kw, 1e-5, 0), "k")
    assert torch.equal(out[:, :, 2], qkv[:, :, 2])    # v untouched


def test_h3_qknorm_rope_partial_inplace(pkg, dev):
    """H3 call form: per-head RMSNorm with weight, eps 1e-5, partial rotary 96
    of 128 with a bf16 table, in place on views of a packed QKV tensor."""
    say("rms_rope_split_half_ rot 96 bf16 table, packed qkv views")
    g = torch.Generator().manual_seed(22)
    S, H, D = 333, 6, 128
    qkv = torch.randn(1, S, 3, H, D, generator=g).to(torch.bfloat16)
    ang = torch.rand(1, S, 1, 48, generator=g) * 30
    c, s = torch.cos(ang), torch.sin(ang)
    tab = torch.stack((c, -s, s, c), -1).reshape(1, S, 1, 48, 2, 2).to(torch.bfloat16)
    qw = (torch.rand(D, generator=g) + 0.5).to(torch.bfloat16)
    kw = (torch.rand(D, generator=g) + 0.5).to(torch.bfloat16)
    dq = qkv.to(dev)
    pkg.rms_rope_split_half_(dq[:, :, 0], dq[:, :, 1], tab.to(dev), qw.to(dev), kw.to(dev), 1e-5, 96)
    torch.cuda.synchronize()
    out = dq.cpu()
    wq = cpu_ref.rms_rope_split_half1(qkv[:, :, 0], tab, qw, 1e-5, 96)
    wk = cpu_ref.rms_rope_split_half1(qkv[:, :, 1], tab, kw, 1e-5, 96)
    close(out[:, :, 0], wq, "q")
    close(out[:, :, 1], wk, "k")
    assert same(out[:, :, 0], wq, "q") and same(out[:, :, 1], wk, "k")
    assert torch.equal(out[:, :, 2], qkv[:, :, 2])    # v untouched


def test_h3_qknorm_rope_angle_form(pkg, dev):
    """H3's apply_qknorm_rope with [S, rot] angles (96 of 128): the table the
    device builds (torch's cos / sin on the GPU, rounded to bf16) is within
    one bf16 step of the CPU's; given that table, q and k equal the oracle
    restatement of the reference's angle branch bit for bit; the inputs are
    left unchanged (the branch returns new tensors)."""
    say("apply_qknorm_rope angle form rot 96 of 128")
    from x_minimaxh3_amd import h3

    g = torch.Generator().manual_seed(27)
    S, H, D, rot = 299, 6, 128, 96
    q = torch.randn(S, H, D, generator=g).to(torch.bfloat16)
    k = torch.randn(S, H, D, generator=g).to(torch.bfloat16)
    qw = (torch.rand(D, generator=g) + 0.5).to(torch.bfloat16)
    kw = (torch.rand(D, generator=g) + 0.5).to(torch.bfloat16)
    half = torch.rand(S, rot // 2, generator=g) * 60
    angles = torch.cat((half, half), -1)
    qd, kd = q.to(dev), k.to(dev)
    oq, ok = h3.apply_qknorm_rope(qd, kd, q_weight=qw.to(dev), k_weight=kw.to(dev), frequencies=angles.to(dev),
                                  eps=1e-5)
    tab = h3.angle_rotation_table(angles.to(dev), torch.bfloat16).cpu()
    torch.cuda.synchronize()
    c_dev, s_dev = tab[0, :, 0, :, 0, 0], tab[0, :, 0, :, 1, 0]
    c_cpu, s_cpu = torch.cos(half).to(torch.bfloat16), torch.sin(half).to(torch.bfloat16)
    assert (cpu_ref.bf16_ulp_diff(c_dev, c_cpu) <= 1).all() and (cpu_ref.bf16_ulp_diff(s_dev, s_cpu) <= 1).all()
    say(f"  device cos/sin differ from the CPU's at {(c_dev != c_cpu).sum().item() + (s_dev != s_cpu).sum().item()}"
        f" of {2 * c_cpu.numel()} entries")
    assert torch.equal(tab[0, :, 0, :, 0, 1], -s_dev) and torch.equal(tab[0, :, 0, :, 1, 1], c_dev)
    wq = cpu_ref.qknorm_rope_angles(q, qw, angles, 1e-5, cos_sin=(c_dev, s_dev))
    wk = cpu_ref.qknorm_rope_angles(k, kw, angles, 1e-5, cos_sin=(c_dev, s_dev))
    assert same(oq, wq, "q") and same(ok, wk, "k")
    assert same(qd, q, "q input") and same(kd, k, "k input")


@pytest.mark.parametrize("mod_dtype", [torch.bfloat16, torch.float32])
def test_rms_adaln(pkg, dev, mod_dtype):
    say(f"rms_adaln scale/shift {mod_dtype}")
    g = torch.Generator().manual_seed(23)
    # 301 tokens per sample: with one block of rows per CU, a block straddles
    # the sample boundary, so both modulation sources of the kernel run
    x = torch.randn(2, 301, 5120, generator=g).to(torch.bfloat16)
    sc = (torch.randn(2, 1, 5120, generator=g) * 0.1).to(mod_dtype)
    sh = (torch.randn(2, 1, 5120, generator=g) * 0.1).to(mod_dtype)
    out = pkg.rms_adaln(x.to(dev), sc.to(dev), sh.to(dev), 1e-6)
    torch.cuda.synchronize()
    want = cpu_ref.rms_adaln(x, sc, sh, 1e-6)
    assert out.dtype == want.dtype
    close(out, want, "rms_adaln")
    assert same(out, want, "rms_adaln")


@pytest.mark.parametrize("rows,width,segs", [
    (1000, 1024, ((0, 77, 0), (77, 200, 1), (200, 1000, 2))),
    # H3's width (672 8-element items: the last 64-item step is half full),
    # segment boundaries inside blocks of rows
    (1500, 5376, ((0, 101, 0), (101, 513, 1), (513, 1500, 2))),
    # the widest row of the pipelined kernel, the first one past it (one row
    # per wave), and a width whose last 64-item step holds one item
    (300, 6144, ((0, 7, 0), (7, 150, 1), (150, 300, 2))),
    (300, 6152, ((0, 7, 0), (7, 150, 1), (150, 300, 2))),
    (257, 520, ((0, 3, 0), (3, 100, 1), (100, 257, 2))),
    # cooperative plan (rows split over waves of 1024 elements): one i-step
    # past the last full chunk (1056), a short last part with no partial
    # chunk (2560), twelve parts and one row per block (11776)
    (700, 1056, ((0, 50, 0), (50, 600, 1), (600, 700, 2))),
    (500, 2560, ((0, 1, 0), (1, 499, 1), (499, 500, 2))),
    (200, 11776, ((0, 13, 0), (13, 100, 1), (100, 200, 2))),
    # tiny rows: one 32-element part (no full chunk), one row, two rows
    (5, 32, ((0, 1, 0), (1, 2, 1), (2, 5, 2))),
    (1, 1024, ((0, 1, 1),)),
    (2, 5376, ((0, 1, 2), (1, 2, 0))),
])
def test_h3_segmented_rms_adaln(pkg, dev, rows, width, segs):
    say(f"h3 segmented rms_adaln rows={rows} width={width}")
    from x_minimaxh3_amd import h3

    g = torch.Generator().manual_seed(24)
    x = torch.randn(rows, width, generator=g).to(torch.bfloat16)
    w = (torch.rand(width, generator=g) + 0.5).to(torch.bfloat16)
    sc = (torch.randn(3, width, generator=g) * 0.1).to(torch.bfloat16)
    sh = (torch.randn(3, width, generator=g) * 0.1).to(torch.bfloat16)
    out = h3.rms_adaln(x.to(dev), w.to(dev), sh.to(dev), sc.to(dev), segs, eps=1e-5)
    torch.cuda.synchronize()
    want = cpu_ref.rms_adaln_segmented(x, w, sh, sc, segs, eps=1e-5)
    close(out, want, "segmented rms_adaln")
    assert same(out, want, "segmented rms_adaln")


@pytest.mark.parametrize("rows,width", [(777, 5376), (3, 2048)])
def test_rms_adaln_rows_without_norm_weight(pkg, dev, rows, width):
    """The row-map form with no norm weight (plain rms_norm before the
    modulation), against the oracle bit for bit."""
    say(f"rms_adaln rows without weight rows={rows} width={width}")
    from x_minimaxh3_amd import backend

    g = torch.Generator().manual_seed(rows + width)
    x = torch.randn(rows, width, generator=g).to(torch.bfloat16)
    sc = (torch.randn(2, width, generator=g) * 0.1).to(torch.bfloat16)
    sh = (torch.randn(2, width, generator=g) * 0.1).to(torch.bfloat16)
    cut = rows // 2
    rm = torch.cat((torch.zeros(cut, dtype=torch.int32), torch.ones(rows - cut, dtype=torch.int32)))
    out = backend.rms_adaln_rows(x.to(dev), None, sc.to(dev), sh.to(dev), rm.to(dev), 1e-6)
    torch.cuda.synchronize()
    segs = ((0, cut, 0), (cut, rows, 1)) if cut else ((0, rows, 1),)
    want = cpu_ref.rms_adaln_segmented(x, None, sh, sc, segs, eps=1e-6)
    assert same(out, want, "rms_adaln without weight")


def test_h3_segmented_rms_adaln_many_iterations(pkg, dev):
    """H3's width over enough rows that each block of the cooperative kernel
    runs past 64 row groups, where its per-lane table of modulation rows is
    refilled: the rows of iterations 62-66 of every block are checked against
    the oracle (a window of the output, the oracle run on that window)."""
    from x_minimaxh3_amd import h3

    width, rows_per_group = 5376, 2                  # 6 waves of 1024 per row, 2 rows per block
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    rows = 68 * cus * rows_per_group + 7             # 68 iterations, a partial last group
    say(f"h3 segmented rms_adaln rows={rows} width={width} (modulation refill)")
    g = torch.Generator().manual_seed(25)
    x = torch.randn(rows, width, generator=g).to(torch.bfloat16)
    w = (torch.rand(width, generator=g) + 0.5).to(torch.bfloat16)
    sc = (torch.randn(3, width, generator=g) * 0.1).to(torch.bfloat16)
    sh = (torch.randn(3, width, generator=g) * 0.1).to(torch.bfloat16)
    lo, hi = 62 * cus * rows_per_group, 67 * cus * rows_per_group
    cut = (lo + hi) // 2 + 3                         # a segment boundary inside the window
    segs = ((0, 1000, 0), (1000, cut, 1), (cut, rows, 2))
    out = h3.rms_adaln(x.to(dev), w.to(dev), sh.to(dev), sc.to(dev), segs, eps=1e-5)
    torch.cuda.synchronize()
    window = ((lo, cut, 1), (cut, hi, 2))
    want = cpu_ref.rms_adaln_segmented(x[lo:hi], w, sh, sc, tuple((a - lo, b - lo, r) for a, b, r in window),
                                       eps=1e-5)
    got = out[lo:hi].cpu()
    assert same(got, want, "segmented rms_adaln (iterations 62-66)")
    tail = cpu_ref.rms_adaln_segmented(x[-300:], w, sh, sc, ((0, 300, 2),), eps=1e-5)
    assert same(out[-300:].cpu(), tail, "segmented rms_adaln (last rows)")


# --------------------------------------------------------------------------- token-chunked driver

def test_long_driver_chunks_match_whole(pkg, dev):
    """Chunking is exact (every op is per token): the chunked resident run and
    the double-buffered host-streamed run both equal one whole-sequence call."""
    say("long driver: 868 tokens in chunks of 256, resident and streamed")
    from x_minimaxh3_amd import backend, driver, workloads

    m, d, f, chunk = 868, 1024, 2048, 256
    inp = workloads.mlp_inputs(M=m, d=d, ffn=f, n_outlier=4, seed=7)
    g = torch.Generator().manual_seed(8)
    q = torch.randn(m, d, generator=g).to(torch.bfloat16)
    k = torch.randn(m, d, generator=g).to(torch.bfloat16)
    scale = (torch.randn(1, d, generator=g) * 0.1).to(torch.bfloat16)
    shift = (torch.randn(1, d, generator=g) * 0.1).to(torch.bfloat16)
    freqs = workloads.rope_table_3d((2, 14, 31)).to(dev)
    x, w1, s1, w2, s2 = (inp[n].to(dev) for n in ("x", "w1", "s1", "w2", "s2"))
    qd, kd, scd, shd = q.to(dev), k.to(dev), scale.to(dev), shift.to(dev)
    drv = driver.LongBlockDriver(w1, s1, w2, s2, scd, shd, chunk=chunk)
    qo, ko, y = drv.run_resident(qd, kd, x, freqs)
    wq, wk = backend.norm_rope(qd, kd, scd, shd, freqs)
    wy = backend.w8a8_mlp(x, w1, s1, w2, s2)
    torch.cuda.synchronize()
    assert torch.equal(qo, wq) and torch.equal(ko, wk) and torch.equal(y, wy)
    host = {n: torch.empty(m, d, dtype=torch.bfloat16, pin_memory=True) for n in ("qo", "ko", "y")}
    drv.run_streamed(q.pin_memory(), k.pin_memory(), inp["x"].pin_memory(), freqs, host["qo"], host["ko"], host["y"])
    assert torch.equal(host["qo"], wq.cpu()) and torch.equal(host["ko"], wk.cpu()) and torch.equal(host["y"], wy.cpu())
    close(host["y"], cpu_ref.w8a8_mlp(inp["x"], inp["w1"], inp["s1"], inp["w2"], inp["s2"]), "streamed mlp vs oracle")


def test_long_grid_full_resident_and_streamed(pkg, dev):
    """C5 at its full size: 130,560 tokens (16x68x120), d 5120, ffn 13824,
    16,384-token chunks (seven full, one of 15,872). The streamed run equals
    the resident run bit for bit, and every chunk's first, last and 22 random
    rows meet the oracle (norm-rope bit-exact, MLP to the fp bar)."""
    say("long grid 130560 tokens: inputs")
    from x_minimaxh3_amd import driver, workloads

    cfg = workloads.CONFIGS["long_16x68x120"]
    m, d, f, chunk = 130560, cfg["d"], cfg["ffn"], cfg["chunk"]
    wts = workloads.mlp_inputs(M=1, d=d, ffn=f, n_outlier=cfg["n_outlier"], seed=0)
    w1, s1, w2, s2 = (wts[n].to(dev) for n in ("w1", "s1", "w2", "s2"))
    gg = torch.Generator(device=dev).manual_seed(11)
    q = torch.randn(m, d, generator=gg, device=dev).to(torch.bfloat16)
    k = torch.randn(m, d, generator=gg, device=dev).to(torch.bfloat16)
    xf = torch.randn(m, d, generator=gg, device=dev)
    xf[:, wts["outliers"].to(dev)] *= 20.0
    x = xf.to(torch.bfloat16)
    del xf
    gc = torch.Generator().manual_seed(12)
    scale = (torch.randn(1, d, generator=gc) * 0.1).to(torch.bfloat16)
    shift = (torch.randn(1, d, generator=gc) * 0.1).to(torch.bfloat16)
    freqs_h = workloads.rope_table_3d(cfg["grid"])
    freqs = freqs_h.to(dev)
    drv = driver.LongBlockDriver(w1, s1, w2, s2, scale.to(dev), shift.to(dev), chunk=chunk)
    say("long grid: resident run")
    qo, ko, y = drv.run_resident(q, k, x, freqs)
    torch.cuda.synchronize()
    say("long grid: streamed run")
    host_in = {n: t.cpu().pin_memory() for n, t in (("q", q), ("k", k), ("x", x))}
    host_out = {n: torch.empty(m, d, dtype=torch.bfloat16, pin_memory=True) for n in ("qo", "ko", "y")}
    drv.run_streamed(host_in["q"], host_in["k"], host_in["x"], freqs, host_out["qo"], host_out["ko"],
                     host_out["y"])
    assert torch.equal(host_out["qo"], qo.cpu()) and torch.equal(host_out["ko"], ko.cpu())
    assert torch.equal(host_out["y"], y.cpu())
    say("long grid: oracle on every chunk")
    rows = []
    for a in range(0, m, chunk):
        b = min(m, a + chunk)
        rows += [a, b - 1] + (a + torch.randperm(b - a - 2, generator=gc)[:22] + 1).tolist()
    rows = torch.tensor(sorted(set(rows)))
    assert rows[-1] == m - 1 and (rows >= 114688).sum() >= 24      # the 15,872-token tail is sampled
    xq, xk, xx = host_in["q"][rows], host_in["k"][rows], host_in["x"][rows]
    fr = freqs_h[:, rows]
    assert same(host_out["qo"][rows], cpu_ref.norm_rope(xq, scale, shift, fr, 128, 1e-6), "long q rows")
    assert same(host_out["ko"][rows], cpu_ref.norm_rope(xk, scale, shift, fr, 128, 1e-6), "long k rows")
    close(host_out["y"][rows], cpu_ref.w8a8_mlp(xx, wts["w1"], wts["s1"], wts["w2"], wts["s2"]), "long mlp rows")


# --------------------------------------------------------------------------- ConvRot / swiglu quantizer

def _code_stats(q, qr, what):
    q, qr = q.cpu(), qr
    mism = (q != qr).float().mean().item()
    dq = (q.int() - qr.int()).abs().max().item() if q.numel() else 0
    say(f"  {what}: code mismatch rate {mism:.2e}, max code delta {dq}")
    return mism, dq


@pytest.mark.parametrize("m,k,act", [
    (333, 1024, None),
    (64, 5120, "gelu_tanh"),
    (250, 13824, "swiglu"),       # raw rows 27648 wide: [gate | up]
    (5, 256, "swiglu"),
    (17, 16384, None),            # the widest activated row
])
def test_convrot_quantizer(pkg, dev, m, k, act):
    say(f"convrot quantizer m={m} k={k} act={act}")
    from x_minimaxh3_amd import backend

    width = 2 * k if act == "swiglu" else k
    x = outlier_acts(m, width, seed=m + k) * 0.5
    q, s = backend.quantize_int8_rowwise_convrot64(x.to(dev), 256, input_act=act)
    torch.cuda.synchronize()
    qr, sr, r = cpu_ref.quantize_convrot(x, 256, act)
    assert q.shape == qr.shape and s.shape == sr.shape
    assert torch.allclose(s.cpu(), sr, rtol=2 ** -7, atol=0)
    mism, dq = _code_stats(q, qr, "convrot codes")
    assert mism < 2e-3 and dq <= 1
    # for information: the reference's own quantization error in code steps
    # (rint, the bf16 rounding of r / bf16(s), and bf16(s) against s)
    err = (q.cpu().float() * s.cpu() - r.float()).abs() / s.cpu()
    say(f"  max |q*s - r| / s = {err.max().item():.3f} (reference rule; codes compared above)")


def test_convrot_quantizer_exact_rows(pkg, dev):
    """Rows whose rotation is exact in fp32 in any summation order
    (small integers: every partial sum is an integer below 2^24) must give
    the oracle's codes and scales bit for bit; a zero row gives zero codes and
    the 1e-30 scale floor; a strided view reads the same rows."""
    say("convrot quantizer on exact rows, zero rows, strided rows")
    from x_minimaxh3_amd import backend

    g = torch.Generator().manual_seed(77)
    m, k = 67, 4096
    x = torch.randint(-40, 41, (m, k), generator=g).float()
    x[5] = 0.0
    x[9, :] = 0.0
    x[9, 300] = -1000.0      # a single spike spreads over its group
    x = x.to(torch.bfloat16)
    q, s = backend.quantize_int8_rowwise_convrot64(x.to(dev), 256)
    torch.cuda.synchronize()
    qr, sr, _ = cpu_ref.quantize_convrot(x, 256, None)
    assert same(q, qr, "exact-row codes") and same(s, sr, "exact-row scales")
    assert (q[5] == 0).all() and s[5].item() == pytest.approx(1e-30, rel=1e-6)
    # the same rows inside a wider buffer (ldx = k + 512)
    wide = torch.zeros(m, k + 512, dtype=torch.bfloat16)
    wide[:, :k] = x
    qv, sv = backend.quantize_int8_rowwise_convrot64(wide.to(dev)[:, :k], 256)
    torch.cuda.synchronize()
    assert same(qv, qr, "strided codes") and same(sv, sr, "strided scales")


@pytest.mark.parametrize("group", [4, 16, 64, 1024])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_convrot_quantizer_group_sizes(pkg, dev, group, dtype):
    """ConvRot groups other than 256 (the eager path takes any power of 4):
    integer rows (every partial sum exact, so any summation order agrees)
    are bit-exact with the oracle, a spike spreads over exactly its own
    group; N(0, 1) rows with outliers, with GELU, meet the code-mismatch bar
    of the 256 case."""
    say(f"convrot quantizer group {group} {dtype}")
    from x_minimaxh3_amd import backend

    g = torch.Generator().manual_seed(group)
    m, k = 45, 3072 if group < 1024 else 4096
    x = torch.randint(-30, 31, (m, k), generator=g).float()
    x[7] = 0.0
    x[7, 1000] = 500.0
    x = x.to(dtype)
    q, s = backend.quantize_int8_rowwise_convrot64(x.to(dev), group)
    torch.cuda.synchronize()
    qr, sr, _ = cpu_ref.quantize_convrot(x, group, None)
    assert same(q, qr, "exact-row codes") and same(s, sr, "exact-row scales")
    lo = 1000 // group * group
    nz = (q[7].cpu() != 0).nonzero().flatten()
    assert nz.min().item() >= lo and nz.max().item() < lo + group and nz.numel() == group
    xo = (outlier_acts(m, k, seed=group + 1) * 0.5).to(dtype)
    q2, s2 = backend.quantize_int8_rowwise_convrot64(xo.to(dev), group, input_act="gelu_tanh")
    torch.cuda.synchronize()
    qr2, sr2, _ = cpu_ref.quantize_convrot(xo, group, "gelu_tanh")
    assert torch.allclose(s2.cpu(), sr2, rtol=2 ** -7, atol=0)
    mism, dq = _code_stats(q2, qr2, f"group {group} codes")
    assert mism < 2e-3 and dq <= 1


@pytest.mark.parametrize("dtype,group,act,seed", [
    (torch.bfloat16, 256, None, 5),
    (torch.bfloat16, 64, "swiglu", (3 << 32) + 9),
    (torch.float16, 256, "gelu_tanh", 77),
    (torch.float16, 1024, None, 2 ** 64 - 3),
])
def test_convrot_quantizer_stochastic(pkg, dev, dtype, group, act, seed):
    """Stochastic rounding in the ConvRot quantizer on integer rows (the
    rotation exact in any order, so the rotated row is the oracle's): codes
    and scales bit-exact with the oracle's noise at each code's index in the
    [M, K] output (mirrored lanes store to the right slots), and they differ
    from the nearest codes."""
    say(f"convrot stochastic {dtype} group {group} act={act} seed={seed}")
    from x_minimaxh3_amd import backend

    g = torch.Generator().manual_seed(group + 3)
    m, k = 23, 2048
    width = 2 * k if act == "swiglu" else k
    if act == "swiglu":
        x = torch.randint(-3, 4, (m, width), generator=g).float()   # silu(gate) * up rounds; tolerance below
    else:
        x = torch.randint(-30, 31, (m, width), generator=g).float()
    x = x.to(dtype)
    if act == "gelu_tanh":
        x = (x.float() * 0.05).to(dtype)
    q, s = backend.quantize_int8_rowwise_convrot64(x.to(dev), group, stochastic_rounding=seed, input_act=act)
    q0, _ = backend.quantize_int8_rowwise_convrot64(x.to(dev), group, input_act=act)
    torch.cuda.synchronize()
    qr, sr, _ = cpu_ref.quantize_convrot(x, group, act, stochastic_rounding=seed)
    if act is None:
        assert same(q, qr, "stochastic convrot codes") and same(s, sr, "scales")
    else:
        assert torch.allclose(s.cpu(), sr, rtol=2 ** -7, atol=0)
        mism, dq = _code_stats(q, qr, "stochastic convrot codes")
        assert mism < 2e-3 and dq <= 1
    assert not torch.equal(q.cpu(), q0.cpu())


@pytest.mark.parametrize("act", [None, "gelu_tanh", "swiglu"])
def test_convrot_quantizer_fp16(pkg, dev, act):
    say(f"convrot quantizer, fp16 rows, act={act}")
    from x_minimaxh3_amd import backend

    m, k = 150, 3072
    width = 2 * k if act == "swiglu" else k
    x = (outlier_acts(m, width, seed=5) * 0.5).to(torch.float16)
    q, s = backend.quantize_int8_rowwise_convrot64(x.to(dev), 256, input_act=act)
    torch.cuda.synchronize()
    qr, sr, _ = cpu_ref.quantize_convrot(x, 256, act)
    assert torch.allclose(s.cpu(), sr, rtol=2 ** -10, atol=0)
    mism, dq = _code_stats(q, qr, "fp16 convrot codes")
    assert mism < 2e-3 and dq <= 1


def test_swiglu_quantizer_without_rotation(pkg, dev):
    say("swiglu quantizer, no rotation")
    from x_minimaxh3_amd import backend

    x = outlier_acts(100, 2 * 2048, seed=4)
    q, s = backend._quantize(x.to(dev), 2)
    torch.cuda.synchronize()
    qr, sr = cpu_ref.quantize_int8_rowwise(cpu_ref.apply_input_act(x, "swiglu"))
    assert torch.allclose(s.cpu(), sr, rtol=2 ** -7, atol=0)
    mism, dq = _code_stats(q, qr, "swiglu codes")
    assert mism < 2e-3 and dq <= 1


def test_int8_linear_convrot_swiglu(pkg, dev):
    """The H3 fc2 boundary: int8_linear(raw, W_rot, s, convrot=True,
    convrot_groupsize=256, input_act="swiglu") on [gate | up] rows."""
    say("int8_linear convrot + swiglu")
    g = torch.Generator().manual_seed(31)
    m, k, n = 300, 2048, 640
    # gate/up of unit scale and fc2-like weights keep |y| near 1, where the
    # 2e-2 bound sits above one bf16 step: the rotated row's last fp32 bit
    # depends on the summation order, so a few codes may move by one
    raw = torch.randn(m, 2 * k, generator=g).to(torch.bfloat16)
    w = torch.randn(n, k, generator=g) * 0.01
    w_rot = cpu_ref.rotate_weight(w, 256)
    qw, sw = cpu_ref.quantize_int8_rowwise(w_rot)
    y = pkg.int8_linear(raw.to(dev), qw.to(dev), sw.reshape(-1).to(dev), None, torch.bfloat16, convrot=True,
                        convrot_groupsize=256, input_act="swiglu")
    torch.cuda.synchronize()
    yr = cpu_ref.int8_linear(raw, qw, sw.reshape(-1), input_act="swiglu", convrot=True, convrot_groupsize=256)
    close(y, yr, "int8_linear convrot swiglu")
    # rotation cancels: close to the unrotated float product
    yf = (cpu_ref.apply_input_act(raw, "swiglu").float() @ w.T)
    cs = cos_sim(y.cpu().float(), yf)
    say(f"  cosine to the unrotated fp32 product: {cs:.5f}")
    assert cs > 0.999


def test_w4a8_linear_convrot(pkg, dev):
    say("w4a8 linear with ConvRot (the reference's default)")
    from x_minimaxh3_amd import backend

    g = torch.Generator().manual_seed(32)
    m, k, n = 129, 1536, 384
    x = outlier_acts(m, k, seed=33)
    w_rot = cpu_ref.rotate_weight(torch.randn(n, k, generator=g) * 0.02, 256)
    packed, srel, sch = cpu_ref.quantize_w4_weight(w_rot, 128)
    y = backend.w4a8_int8_linear(x.to(dev), packed.to(dev), srel.to(dev), sch.to(dev), group_size=128,
                                 convrot_groupsize=256)
    torch.cuda.synchronize()
    yr = cpu_ref.w4a8_linear(x, packed, srel.float(), sch, 128, convrot=True, convrot_groupsize=256)
    close(y, yr, "w4a8 linear convrot")


@pytest.mark.parametrize("m,n,k,dt,gate_dt,bias", [
    (300, 640, 2048, torch.bfloat16, torch.float32, False),    # K % 256 == 0: the DMA main loop
    (77, 260, 1040, torch.bfloat16, torch.bfloat16, True),     # K % 128 != 0: register-staged loop
    (513, 384, 1536, torch.float16, torch.float16, True),
])
def test_int8_gemm_gated_residual(pkg, dev, m, n, k, dt, gate_dt, bias):
    """fc2 with the gated residual in its epilogue against int8_linear then
    addcmul_ per segment (no rotation and no act here, so every code and
    accumulator is exact and the result must be bit-exact)."""
    say(f"gated residual epilogue m={m} n={n} k={k} {dt} gate {gate_dt} bias={bias}")
    from x_minimaxh3_amd import backend

    g = torch.Generator().manual_seed(m + n)
    x = outlier_acts(m, k, seed=m).to(dt)
    w, sw = cpu_ref.quantize_int8_rowwise(torch.randn(n, k, generator=g) * 0.02)
    b = (torch.randn(n, generator=g) * 0.1).to(dt) if bias else None
    res = torch.randn(m, n, generator=g).to(dt)
    gate = (torch.randn(4, n, generator=g) * 0.3).to(gate_dt)
    cut = m // 3
    segments = ((0, cut, 2), (cut, m, 1))
    rows = cpu_ref.segment_row_map(m, segments)
    want = cpu_ref.int8_linear_gated_residual_(x, w, sw.reshape(-1), b, res.clone(), gate, segments,
                                               convrot=False, input_act=None)
    got = res.to(dev)
    backend.int8_linear_gated_residual_(x.to(dev), w.to(dev), sw.reshape(-1).to(dev),
                                        None if b is None else b.to(dev), got, gate.to(dev), rows.to(dev),
                                        convrot=False, input_act=None)
    torch.cuda.synchronize()
    assert same(got, want, "gated residual")


def test_int8_gemm_gated_residual_clamps_rows(pkg, dev):
    """A gate row index past the table reads its last row (no read past it)."""
    say("gated residual: out-of-range gate rows are clamped")
    from x_minimaxh3_amd import backend

    g = torch.Generator().manual_seed(3)
    m, n, k = 64, 256, 512
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w, sw = cpu_ref.quantize_int8_rowwise(torch.randn(n, k, generator=g) * 0.02)
    res = torch.randn(m, n, generator=g).to(torch.bfloat16)
    gate = torch.randn(2, n, generator=g)
    rows_bad = torch.full((m,), 7, dtype=torch.int32)
    want = cpu_ref.int8_linear_gated_residual_(x, w, sw.reshape(-1), None, res.clone(), gate, ((0, m, 1),),
                                               convrot=False, input_act=None)
    got = res.to(dev)
    backend.int8_linear_gated_residual_(x.to(dev), w.to(dev), sw.reshape(-1).to(dev), None, got, gate.to(dev),
                                        rows_bad.to(dev), convrot=False, input_act=None)
    torch.cuda.synchronize()
    assert same(got, want, "clamped gate rows")


def test_h3_gated_swiglu_mlp(pkg, dev):
    """The int8 route of the H3 MLP (fc1 ConvRot linear -> SwiGLU + ConvRot
    quantizer -> fc2 with the gated residual), chunked, against the oracle's
    default route (int8_linear twice, then addcmul_ per segment)."""
    say("H3 gated SwiGLU MLP, chunked")
    from x_minimaxh3_amd import h3

    g = torch.Generator().manual_seed(41)
    m, d, f = 300, 512, 1024
    hidden = torch.randn(m, d, generator=g).to(torch.bfloat16)
    w1, s1 = cpu_ref.quantize_int8_rowwise(cpu_ref.rotate_weight(torch.randn(2 * f, d, generator=g) * 0.05, 256))
    w2, s2 = cpu_ref.quantize_int8_rowwise(cpu_ref.rotate_weight(torch.randn(d, f, generator=g) * 0.03, 256))
    res = torch.randn(m, d, generator=g).to(torch.bfloat16)
    gate = torch.randn(2, d, generator=g) * 0.5
    segments = ((0, 120, 1), (120, m, 0))
    raw = cpu_ref.int8_linear(hidden, w1, s1.reshape(-1), None, torch.bfloat16, convrot=True)
    want = cpu_ref.int8_linear_gated_residual_(raw, w2, s2.reshape(-1), None, res.clone(), gate, segments)
    got = res.to(dev)
    h3.gated_swiglu_mlp_(got, hidden.to(dev), w1.to(dev), s1.reshape(-1).to(dev), None, w2.to(dev),
                         s2.reshape(-1).to(dev), None, gate.to(dev), segments, chunk_tokens=128)
    torch.cuda.synchronize()
    close(got, want, "h3 gated swiglu mlp")


@pytest.mark.parametrize("gs", [16, 8, 32])
def test_int8_group_sums(pkg, dev, gs):
    say(f"int8 group sums gs={gs}")
    from x_minimaxh3_amd._lib import DTYPE_CODE, call, stream_of

    g = torch.Generator().manual_seed(gs)
    m, k = 203, 1536
    q = torch.randint(-128, 128, (m, k), generator=g, dtype=torch.int8)
    q[7] = -128
    q[8] = 127
    xs = torch.rand(m, 1, generator=g) * 0.05
    for dt in (torch.bfloat16, torch.float16, torch.float32):
        out = torch.empty(m, k // gs, dtype=dt, device=dev)
        qd, xsd = q.to(dev), xs.to(dev)
        call("xmh3_int8_group_sums", qd.data_ptr(), qd.stride(0), xsd.data_ptr(), m, k, gs, out.data_ptr(),
             DTYPE_CODE[dt], out.stride(0), stream_of(qd))
        torch.cuda.synchronize()
        assert same(out, cpu_ref.int8_group_sums(q, xs, gs, dt), f"group sums {dt}")


def test_w4a8_h3_checkpoint_format(pkg, dev):
    """The H3 W4A8 layout end to end: group 16, fp8-e4m3 s_rel, the
    Lloyd-Max codebook, ConvRot and the asymmetric correction, with a bias,
    through the checkpoint loader."""
    say("w4a8 H3 checkpoint format (group 16, e4m3 s_rel, codebook, correction)")
    from x_minimaxh3_amd import h3

    g = torch.Generator().manual_seed(9)
    m, n, k, gs = 300, 640, 1536, 16
    lut = torch.tensor([-0.980602, -0.794529, -0.638165, -0.500986, -0.377321, -0.263187, -0.155210,
                        -0.050720, 0.052541, 0.156985, 0.265284, 0.379533, 0.502636, 0.638953, 0.794876,
                        0.980671])
    tensors = {
        "fc.weight": torch.randint(-128, 128, (n, k // 2), generator=g, dtype=torch.int8),
        "fc.weight_s_rel": (torch.rand(n, k // gs, generator=g) * 90 + 30).to(torch.float8_e4m3fn),
        "fc.weight_s_channel": torch.rand(n, generator=g) * 2e-4 + 1e-4,
        "fc.weight_codebook": lut,
        "fc.weight_correction": torch.randn(k // gs, n, generator=g) * 2e-3,
        "fc.bias": torch.randn(n, generator=g) * 0.1,
    }
    x = outlier_acts(m, k, seed=10)
    lin = h3.load_w4a8_linear({key: t.to(dev) for key, t in tensors.items()}, "fc")
    y = lin(x.to(dev))
    torch.cuda.synchronize()
    yr = cpu_ref.w4a8_linear_h3(x, tensors["fc.weight"], tensors["fc.weight_s_rel"],
                                tensors["fc.weight_s_channel"], codebook=lut,
                                correction=tensors["fc.weight_correction"], bias=tensors["fc.bias"],
                                group_size=gs, out_dtype=torch.bfloat16)
    close(y, yr, "w4a8 h3 format")
    # without the correction the int8 part alone
    lin0 = h3.load_w4a8_linear({key: t.to(dev) for key, t in tensors.items() if "correction" not in key}, "fc")
    y0 = lin0(x.to(dev))
    torch.cuda.synchronize()
    y0r = cpu_ref.w4a8_linear_h3(x, tensors["fc.weight"], tensors["fc.weight_s_rel"],
                                 tensors["fc.weight_s_channel"], codebook=lut, bias=tensors["fc.bias"],
                                 group_size=gs, out_dtype=torch.bfloat16)
    close(y0, y0r, "w4a8 h3 format, no correction")


@pytest.mark.parametrize("hnd_out", [False, True])
def test_reference_named_rope_launcher(pkg, dev, hnd_out):
    """launch_rms_rope_kernel called with the reference's 46 arguments the way
    the H3 single-sided QK-norm binding forms them: value [tokens, heads, D]
    in place, or into an HND-backed NHD view; rot 96 of 128, bf16 table."""
    say(f"launch_rms_rope_kernel hnd_out={hnd_out}")
    import ctypes

    from x_minimaxh3_amd import _lib

    g = torch.Generator().manual_seed(25)
    T, H, D, rot = 77, 6, 128, 96
    x = torch.randn(T, H, D, generator=g).to(torch.bfloat16)
    ang = torch.rand(1, T, 1, rot // 2, generator=g) * 30
    c, sn = torch.cos(ang), torch.sin(ang)
    tab = torch.stack((c, -sn, sn, c), -1).reshape(1, T, 1, rot // 2, 2, 2).to(torch.bfloat16)
    w = (torch.rand(D, generator=g) + 0.5).to(torch.bfloat16)
    xd, td, wd = x.to(dev), tab.to(dev), w.to(dev)
    if hnd_out:
        backing = torch.zeros(H, T, D, dtype=torch.bfloat16, device=dev)
        out = backing.transpose(0, 1)                 # logical [T, H, D], strides (D, T*D, 1)
    else:
        out = xd
    q4, o4 = xd.unsqueeze(0), out.unsqueeze(0)
    z4 = (0, 0, 0, 0)
    args = ([q4.data_ptr(), None, td.data_ptr(), wd.data_ptr(), None, o4.data_ptr(), None]
            + list(q4.shape[:3]) + [D, rot] + list(td.shape[:3])
            + list(q4.stride()) + list(z4) + list(o4.stride()) + list(z4) + list(td.stride())
            + [wd.stride(0), 0, 1e-5, 2, 2, 2, False, True, torch.cuda.current_stream().cuda_stream])
    assert len(args) == 46
    _lib.load().launch_rms_rope_kernel(*args)
    torch.cuda.synchronize()
    want = cpu_ref.rms_rope_split_half1(x.unsqueeze(0), tab, w, 1e-5, rot)[0]
    assert same(out, want, "launcher output")


def _angle_table(shape_lead, pairs, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    ang = torch.rand(*shape_lead, pairs, generator=g) * 30
    c, sn = torch.cos(ang), torch.sin(ang)
    return torch.stack((c, -sn, sn, c), -1).reshape(*shape_lead, pairs, 2, 2).to(dtype)


@pytest.mark.parametrize("dtype,tdtype,D,norm,inplace", [
    (torch.bfloat16, torch.float32, 128, True, False),
    (torch.bfloat16, torch.float32, 96, True, True),      # 96-wide heads, in place
    (torch.bfloat16, torch.bfloat16, 64, False, False),
    (torch.float16, torch.float32, 128, True, True),
    (torch.float16, torch.float16, 128, False, True),
    (torch.float32, torch.float32, 80, True, False),
])
def test_interleaved_rope_bit_exact(pkg, dev, dtype, tdtype, D, norm, inplace):
    """apply_rope1 / rms_rope1 (pairs (2i, 2i + 1), the rotation's second
    product fused as torch's addcmul_ does) on [B, S, H, D] with a table
    broadcast over heads, against the oracle bit for bit; q and k of
    rms_rope_ / apply_rope_ in place, strided q (a slice of a packed qkv)."""
    say(f"interleaved rope {dtype} table {tdtype} D={D} norm={norm} inplace={inplace}")
    g = torch.Generator().manual_seed(D + 7 * norm)
    B, S, H = 2, 37, 5
    qkv = torch.randn(B, S, 3 * H, D, generator=g).to(dtype)
    q, k = qkv[:, :, :H], qkv[:, :, H:2 * H]
    tab = _angle_table((B, S, 1), D // 2, D, tdtype)
    wq = (torch.rand(D, generator=g) + 0.5).to(dtype)
    wk = (torch.rand(D, generator=g) + 0.5).to(dtype)
    if norm:
        wantq, wantk = cpu_ref.rms_rope1(q, tab, wq, 1e-6), cpu_ref.rms_rope1(k, tab, wk, 1e-6)
    else:
        wantq, wantk = cpu_ref.apply_rope1(q, tab), cpu_ref.apply_rope1(k, tab)
    qkvd, td = qkv.to(dev), tab.to(dev)
    qd, kd = qkvd[:, :, :H], qkvd[:, :, H:2 * H]
    if inplace:
        if norm:
            pkg.rms_rope_(qd, kd, td, wq.to(dev), wk.to(dev))
        else:
            pkg.apply_rope_(qd, kd, td)
        gq, gk = qd, kd
        torch.cuda.synchronize()
        assert same(qkvd[:, :, 2 * H:], qkv[:, :, 2 * H:], "untouched v")
    else:
        if norm:
            gq, gk = pkg.rms_rope(qd, kd, td, wq.to(dev), wk.to(dev))
        else:
            gq, gk = pkg.apply_rope(qd, kd, td)
        torch.cuda.synchronize()
    assert same(gq, wantq, "q") and same(gk, wantk, "k")


@pytest.mark.parametrize("rot", [128, 96])
def test_reference_named_rope_launcher_interleaved(pkg, dev, rot):
    """launch_rms_rope_kernel with split_half = false: interleaved pairs over
    the first rot dims, norm-only tail, into a separate output."""
    say(f"launch_rms_rope_kernel interleaved rot={rot}")
    from x_minimaxh3_amd import _lib

    g = torch.Generator().manual_seed(26 + rot)
    T, H, D = 51, 4, 128
    x = torch.randn(T, H, D, generator=g).to(torch.bfloat16)
    tab = _angle_table((1, T, 1), rot // 2, rot, torch.float32)
    w = (torch.rand(D, generator=g) + 0.5).to(torch.bfloat16)
    xd, td, wd = x.to(dev), tab.to(dev), w.to(dev)
    out = torch.zeros_like(xd)
    q4, o4 = xd.unsqueeze(0), out.unsqueeze(0)
    z4 = (0, 0, 0, 0)
    args = ([q4.data_ptr(), None, td.data_ptr(), wd.data_ptr(), None, o4.data_ptr(), None]
            + list(q4.shape[:3]) + [D, rot] + list(td.shape[:3])
            + list(q4.stride()) + list(z4) + list(o4.stride()) + list(z4) + list(td.stride())
            + [wd.stride(0), 0, 1e-6, 2, 0, 2, False, False, torch.cuda.current_stream().cuda_stream])
    assert len(args) == 46
    _lib.load().launch_rms_rope_kernel(*args)
    torch.cuda.synchronize()
    want = cpu_ref.rms_rope1(x.unsqueeze(0), tab, w, 1e-6, rot)[0]
    assert same(out, want, "launcher output")


def test_empty_token_batches(pkg, dev):
    """A batch of zero tokens returns empty results with the oracle's shapes
    and dtypes (no kernel is launched for an empty grid)."""
    say("empty token batches")
    g = torch.Generator().manual_seed(41)
    x = torch.empty(0, 512, dtype=torch.bfloat16)
    w1 = torch.randint(-127, 128, (256, 512), generator=g, dtype=torch.int8)
    s1 = torch.rand(256, generator=g) * 1e-2
    w2 = torch.randint(-127, 128, (512, 256), generator=g, dtype=torch.int8)
    s2 = torch.rand(512, generator=g) * 1e-2
    scale = torch.zeros(1, 512, dtype=torch.bfloat16)
    shift = torch.zeros(1, 512, dtype=torch.bfloat16)

    def check(got, want, what):
        got = got if isinstance(got, tuple) else (got,)
        want = want if isinstance(want, tuple) else (want,)
        for a, b in zip(got, want):
            say(f"  {what}: {tuple(a.shape)} {a.dtype}")
            assert a.is_cuda and tuple(a.shape) == tuple(b.shape) and a.dtype == b.dtype, (what, a.shape, b.shape)

    from x_minimaxh3_amd import backend

    xd = x.to(dev)
    check(pkg.quantize_int8_rowwise(xd), cpu_ref.quantize_int8_rowwise(x), "quantize_int8_rowwise")
    check(backend.quantize_int8_rowwise_convrot64(xd, 256), cpu_ref.quantize_convrot(x, 256)[:2],
          "convrot quantizer")
    check(pkg.int8_linear(xd, w1.to(dev), s1.to(dev)), cpu_ref.int8_linear(x, w1, s1), "int8_linear")
    check(pkg.w8a8_mlp(xd, w1.to(dev), s1.to(dev), w2.to(dev), s2.to(dev)),
          cpu_ref.w8a8_mlp(x, w1, s1, w2, s2), "w8a8_mlp")
    check(pkg.rms_adaln(xd, scale.to(dev), shift.to(dev)), cpu_ref.rms_adaln(x, scale, shift), "rms_adaln")
    tab = torch.zeros(1, 1, 1, 64, 2, 2)
    qo, ko = pkg.norm_rope(xd, xd, scale.to(dev), shift.to(dev), tab.to(dev), 1e-6, 128)
    # the eager rope's reshape(..., 2, -1) raises on zero elements, so the
    # oracle gives no shape here; the fused op returns Q's and K's empty shape
    check((qo, ko), (x, x), "norm_rope")
    torch.cuda.synchronize()


def test_host_small_operands_follow_the_input(pkg, dev):
    """Scales, shifts, norm weights and RoPE tables given on the host are moved
    to the input's device before the kernels run: the results equal those of
    the all-device calls bit for bit."""
    say("host-side small operands")
    from x_minimaxh3_amd import backend, workloads

    nr = workloads.norm_rope_inputs(grid=(2, 3, 5), d=512, head_dim=128, seed=3)
    q, k = nr["q"].to(dev), nr["k"].to(dev)
    want = backend.norm_rope(q, k, nr["scale"].to(dev), nr["shift"].to(dev), nr["freqs"].to(dev), nr["eps"], 128)
    got = backend.norm_rope(q, k, nr["scale"], nr["shift"], nr["freqs"], nr["eps"], 128)
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
    ra = backend.rms_adaln(q, nr["scale"], nr["shift"])
    assert torch.equal(ra, backend.rms_adaln(q, nr["scale"].to(dev), nr["shift"].to(dev)))
    x4 = q.reshape(1, 30, 4, 128)
    w = (torch.rand(128, generator=torch.Generator().manual_seed(4)) + 0.5).to(torch.bfloat16)
    a = backend.rms_rope_split_half1(x4, nr["freqs"], w, 1e-6)
    b = backend.rms_rope_split_half1(x4, nr["freqs"].to(dev), w.to(dev), 1e-6)
    assert torch.equal(a, b)
