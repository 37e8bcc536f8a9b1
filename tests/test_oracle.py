"""Pins the CPU oracle (oracle/cpu_ref.py) before it is trusted as the checker.

The reference holds no golden vectors for this path (its tests are
cross-path equalities on CUDA), so each oracle function is pinned by an
independent restatement in another form (numpy on bit patterns, exact
rationals, plain C, int64 brute force), by hand-derived known answers and by
mathematical invariants, chosen so that a plausible slip (x*(1/s) instead of
x/s, round-half-away, a +-127 clamp, swapped nibbles, a dropped bf16 rounding,
a transposed table entry) fails at least one test.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import cpu_ref, npref


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16)


def outlier_acts(m, k, seed=0, n_out=8):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g)
    x[:, torch.randperm(k, generator=g)[:n_out]] *= 20
    return x.to(torch.bfloat16)


# --------------------------------------------------------------------------- quantizer

def test_quant_matches_numpy_and_c(corc):
    x = outlier_acts(257, 1536)
    q, s = cpu_ref.quantize_int8_rowwise(x)
    qn, sn = npref.quantize_rows_bf16(bits(x))
    assert np.array_equal(q.numpy(), qn)
    assert np.array_equal(s.numpy().reshape(-1), sn)
    qc = np.empty((257, 1536), np.int8)
    sc = np.empty(257, np.float32)
    xb = np.ascontiguousarray(bits(x))
    corc.orc_quant_rows_bf16(xb.ctypes.data, 257, 1536, qc.ctypes.data, sc.ctypes.data)
    assert np.array_equal(q.numpy(), qc)
    assert np.array_equal(s.numpy().reshape(-1), sc)


def test_quant_exact_rationals_small_rows():
    rng = np.random.default_rng(1)
    rows = [rng.standard_normal(24).astype(np.float32) * s for s in (1.0, 1e-3, 37.0, 1e-20)]
    for r in rows:
        x = torch.from_numpy(r).to(torch.bfloat16).reshape(1, -1)
        q, s = cpu_ref.quantize_int8_rowwise(x)
        qe, se = npref.quantize_row_exact(bits(x)[0].tolist())
        assert q[0].tolist() == qe
        assert s.item() == np.float32(se)


def test_quant_known_answers():
    # amax 1 -> scale 1/127 -> bf16(scale) = 2^-7 * 1.0078125;
    # 1/bf16(s) = 127.0078 -> bf16 127; 0.5 -> 63.5039 -> bf16 63.5 -> ties-to-even 64
    x = torch.tensor([[1.0, -1.0, 0.5, 0.0, -0.5, 0.25]]).to(torch.bfloat16)
    q, s = cpu_ref.quantize_int8_rowwise(x)
    assert q[0].tolist() == [127, -127, 64, 0, -64, 32]
    assert s.item() == np.float32(1.0) / np.float32(127.0)
    # a zero row: scale clamps to 1e-30 (fp32), every code 0
    q, s = cpu_ref.quantize_int8_rowwise(torch.zeros(1, 16, dtype=torch.bfloat16))
    assert q.abs().sum().item() == 0 and s.item() == np.float32(1e-30)


def test_quant_reaches_minus_128_and_clamps_plus_127():
    # search bf16 amax values whose bf16-rounded scale is low enough that
    # amax / bf16(amax/127) rounds (in bf16) to 127.5 -> rint -> 128 (even)
    hits = []
    for b in range(0x3f80, 0x4000):           # bf16 values in [1, 2)
        a = float(npref.bf16_bits_to_f32(np.array([b], np.uint16))[0])
        x = torch.tensor([[-a, a]]).to(torch.bfloat16)
        q, _ = cpu_ref.quantize_int8_rowwise(x)
        qe, _ = npref.quantize_row_exact(bits(x)[0].tolist())
        assert q[0].tolist() == qe
        if q[0, 0].item() == -128:
            hits.append(a)
            assert q[0, 1].item() == 127      # +127.5 -> 128 clamps to 127
    assert hits, "the [-128, 127] clamp range is never exercised"


def test_stochastic_hash_matches_c_and_fills_24_bits(corc):
    """The noise hash: the numpy and C restatements agree on 2^20 inputs; its
    top 24 bits (the noise) span [0, 2^24) and are uniform over 256 buckets
    (chi-square, 255 degrees of freedom, far below the 0.1 % tail)."""
    import ctypes

    x = np.random.default_rng(1).integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    x[:4] = (0, 1, 0xFFFFFFFF, 0x80000000)
    h = cpu_ref.pcg_hash(x)
    hc = np.empty_like(x)
    corc.orc_pcg_hash(x.ctypes.data_as(ctypes.c_void_p), x.size, hc.ctypes.data_as(ctypes.c_void_p))
    assert np.array_equal(h, hc)
    u = h >> np.uint32(8)
    assert u.max() > (1 << 24) - 64 and u.min() < 64
    counts = np.bincount((u >> np.uint32(16)).astype(np.int64), minlength=256)
    e = x.size / 256
    assert ((counts - e) ** 2 / e).sum() < 330.0


def test_round_to_dtype_matches_torch_conversions():
    """round_to_dtype (one rounding from float64) equals torch's fp32 -> bf16 /
    fp16 conversions on fp32 inputs, subnormals, ties and overflow-free
    extremes included; fp32 values are fixed points."""
    g = torch.Generator().manual_seed(5)
    x = torch.cat((torch.randn(20000, generator=g) * 100, torch.rand(20000, generator=g) * 2 ** -13,
                   torch.tensor([0.0, -0.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 2 ** -24, 3 * 2 ** -25, 65504.0])))
    x64 = x.double().numpy()
    for dt in (torch.bfloat16, torch.float16):
        assert np.array_equal(cpu_ref.round_to_dtype(x64, dt), x.to(dt).double().numpy()), dt
    assert np.array_equal(cpu_ref.round_to_dtype(x64, torch.float32), x64)


def test_stochastic_noise_keying():
    """key = idx + seed: seed + 1 at idx equals seed at idx + 1; seeds past
    2^32 fold their high word in by xor: (a << 32 | b) at idx equals seed
    (b + idx) ^ a at index 0; the noise lies in [0, 1] and only bf16 can
    round it up to 1."""
    idx = np.arange(5000, dtype=np.uint64)
    for dt in (torch.bfloat16, torch.float16, torch.float32):
        n1 = cpu_ref.stochastic_noise(idx, 1234, dt)
        assert np.array_equal(cpu_ref.stochastic_noise(idx, 1235, dt)[:-1], n1[1:])
        assert n1.min() >= 0.0 and n1.max() <= 1.0
        a, b = 7, 1000
        folded = cpu_ref.stochastic_noise(idx[:100], (a << 32) | b, dt)
        direct = np.array([cpu_ref.stochastic_noise(np.zeros(1, np.uint64), (b + i) ^ a, dt)[0] for i in range(100)])
        assert np.array_equal(folded, direct)
    assert cpu_ref.stochastic_noise(np.arange(1 << 16, dtype=np.uint64), 1, torch.float32).max() < 1.0


def test_stochastic_quant_matches_c_and_is_unbiased(corc):
    """bf16 rows: the oracle's stochastic codes equal the C restatement's for
    several seeds (including one past 2^32); every code is floor(v) or
    floor(v) + 1 of the nearest path's v = bf16(x / bf16(s)); the mean code
    over 400 seeds is within 5 sigma of v where bf16 resolves the sum finely
    (|v| < 2: the reference rounds v + noise to bf16, whose step is 2^-6 at
    2 and 0.5 at 64, so larger codes are biased by design); seed 0 is the
    nearest path. fp32 rows are unbiased at every magnitude."""
    import ctypes

    x = outlier_acts(6, 300, seed=9, n_out=3)
    q0, s0 = cpu_ref.quantize_int8_rowwise(x)
    assert torch.equal(cpu_ref.quantize_int8_rowwise(x, 0)[0], q0)
    v = (x / cpu_ref._int8_scale_for_math(s0, x)).double()
    xb = bits(x)
    for seed in (1, 77, (5 << 32) + 3):
        q, s = cpu_ref.quantize_int8_rowwise(x, seed)
        qc = np.empty((6, 300), np.int8)
        sc = np.empty(6, np.float32)
        corc.orc_quant_rows_sr_bf16(xb.ctypes.data_as(ctypes.c_void_p), 6, 300, seed,
                                    qc.ctypes.data_as(ctypes.c_void_p), sc.ctypes.data_as(ctypes.c_void_p))
        assert np.array_equal(q.numpy(), qc) and np.array_equal(s.numpy()[:, 0], sc) and torch.equal(s, s0)
        d = q.double() - v.floor().clamp(-128, 127)
        assert ((d == 0) | (d == 1)).all()
    acc = torch.zeros_like(v)
    for seed in range(1, 401):
        acc += cpu_ref.quantize_int8_rowwise(x, seed)[0].double()
    mean = acc / 400
    inner = v.abs() < 2
    frac = v - v.floor()
    sigma = (frac * (1 - frac) / 400).sqrt()
    assert inner.float().mean() > 0.2
    assert ((mean - v).abs()[inner] <= 5 * sigma[inner] + 2 ** -6).all()
    xf = x.float()
    q0f, s0f = cpu_ref.quantize_int8_rowwise(xf)
    vf = (xf / s0f).double()
    accf = torch.zeros_like(vf)
    for seed in range(1, 401):
        accf += cpu_ref.quantize_int8_rowwise(xf, seed)[0].double()
    fracf = vf - vf.floor()
    inner = (vf > -127) & (vf < 126)
    sig = (fracf * (1 - fracf) / 400).sqrt()
    assert ((accf / 400 - vf).abs()[inner] <= 5 * sig[inner] + 2 ** -20).all()


def test_quant_half_to_even_ties():
    # row amax 127 -> scale exactly 1.0 in fp32 and bf16; values k + 0.5
    # (bf16-exact) divide exactly and must round to even
    vals = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 100.5, -126.5]
    x = torch.tensor([vals]).to(torch.bfloat16)
    q, s = cpu_ref.quantize_int8_rowwise(x)
    assert s.item() == 1.0
    assert q[0].tolist() == [127, 0, 2, 2, 0, -2, -2, 100, -126]


# --------------------------------------------------------------------------- GEMM / dequant

@pytest.mark.parametrize("m,n,k", [(33, 17, 64), (64, 96, 256), (5, 7, 13)])
def test_int_mm_brute_force(corc, m, n, k):
    g = torch.Generator().manual_seed(m * n + k)
    a = torch.randint(-128, 128, (m, k), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8)
    a[0] = -128
    w[0] = -128                                 # extreme products
    acc = cpu_ref.int8_mm(a, w)
    assert np.array_equal(acc.numpy(), npref.int_mm(a.numpy(), w.numpy()))
    out = np.empty((m, n), np.int32)
    corc.orc_int_mm(a.numpy().ctypes.data, w.numpy().ctypes.data, m, n, k, out.ctypes.data)
    assert np.array_equal(acc.numpy(), out)


def test_dequant_order_and_rounding(corc):
    g = torch.Generator().manual_seed(3)
    acc = torch.randint(-(2 ** 27), 2 ** 27, (64, 48), generator=g, dtype=torch.int32)
    sx = torch.rand(64, 1, generator=g) * 0.1
    sw = torch.rand(48, generator=g) * 0.01
    out = cpu_ref.dequant(acc, sx, sw)
    assert np.array_equal(bits(out), npref.dequant_bf16_bits(acc.numpy(), sx.numpy(), sw.numpy()))
    c = np.empty((64, 48), np.uint16)
    corc.orc_dequant_bf16(acc.numpy().ctypes.data, sx.numpy().ctypes.data, sw.numpy().ctypes.data, 1,
                          64, 48, c.ctypes.data)
    assert np.array_equal(bits(out), c)
    # the float64 closed form agrees to within one bf16 rounding
    exact = acc.double() * sx.double() * sw.double().reshape(1, -1)
    assert (cpu_ref.bf16_ulp_diff(out, exact.float()) <= 1.0).all()


def test_int8_linear_composite_step_by_step():
    x = outlier_acts(40, 256, seed=5)
    g = torch.Generator().manual_seed(6)
    w = torch.randint(-127, 128, (96, 256), generator=g, dtype=torch.int8)
    sw = torch.rand(96, generator=g) * 1e-3
    bias = torch.randn(96, generator=g).to(torch.bfloat16)
    y = cpu_ref.int8_linear(x, w, sw, bias=bias)
    qn, sn = npref.quantize_rows_bf16(bits(x))
    acc = npref.int_mm(qn, w.numpy())
    yb = npref.dequant_bf16_bits(acc, sn, sw.numpy())
    # bias in bf16: bf16(float(y) + float(bias))
    yf = npref.bf16_bits_to_f32(yb) + npref.bf16_bits_to_f32(bits(bias)).reshape(1, -1)
    assert np.array_equal(bits(y), npref.f32_to_bf16_bits(yf.astype(np.float32)))


def test_gelu_against_closed_form():
    h = (torch.randn(1 << 16, generator=torch.Generator().manual_seed(7)) * 4).to(torch.bfloat16)
    g = cpu_ref.gelu_tanh(h)
    hd = h.double()
    exact = 0.5 * hd * (1 + torch.tanh(math.sqrt(2 / math.pi) * (hd + 0.044715 * hd ** 3)))
    ulp = cpu_ref.bf16_ulp_diff(g, exact.float())
    big = exact.abs() > 1e-3
    assert (ulp[big] <= 1.0).all()
    assert ((g.double() - exact).abs()[~big] <= 1e-5).all()


# --------------------------------------------------------------------------- W4

def test_w4_nibble_order_known_answer():
    # byte 0x8F: low nibble 15 (even k) -> level 7, high nibble 8 (odd k) -> level 0
    q = torch.tensor([[0x8F - 256, 0x10]], dtype=torch.int8)
    s = torch.tensor([[3.0]])
    out = cpu_ref.dequant_int4_grouped_to_int8(q, s, group_size=4)
    assert out[0].tolist() == [21, 0, -24, -21]


def test_w4_decode_three_ways(corc):
    g = torch.Generator().manual_seed(9)
    w = torch.randn(24, 256, generator=g) * 0.02
    packed, srel, sch = cpu_ref.quantize_w4_weight(w, group_size=128)
    pn, srn, schn = npref.w4_quantize(w.numpy(), 128)
    assert np.array_equal(packed.numpy(), pn)
    assert np.array_equal(srel.numpy(), srn) and np.array_equal(sch.numpy(), schn)
    dec = cpu_ref.dequant_int4_grouped_to_int8(packed, srel, 128)
    assert np.array_equal(dec.numpy(), npref.w4_decode(packed.numpy(), srel.numpy(), 128))
    out = np.empty((24, 256), np.int8)
    corc.orc_w4_decode(packed.numpy().view(np.uint8).ctypes.data, srel.numpy().ctypes.data, 24, 256, 128,
                       out.ctypes.data)
    assert np.array_equal(dec.numpy(), out)
    small = cpu_ref.dequant_int4_grouped_to_int8(packed[:2, :8], srel[:2, :1], 16)
    assert small.tolist() == npref.w4_decode_loops(packed[:2, :8].numpy(), srel[:2, :1].numpy(), 16)


def test_w4_round_trip_bound():
    g = torch.Generator().manual_seed(10)
    w = torch.randn(32, 512, generator=g) * 0.02
    packed, srel, sch = cpu_ref.quantize_w4_weight(w, group_size=128)
    w8 = cpu_ref.dequant_int4_grouped_to_int8(packed, srel, 128).float()
    rec = w8 * sch.reshape(-1, 1)
    gs = w.view(32, 4, 128).abs().amax(-1, keepdim=True) / 7.0
    # int4 rounding error <= gs/2 plus the int8 re-grid error <= s_channel/2
    bound = (gs / 2).expand(32, 4, 128).reshape(32, 512) + sch.reshape(-1, 1) / 2 + 1e-7
    assert ((rec - w).abs() <= bound).all()


# --------------------------------------------------------------------------- norm / rope

def test_rms_adaln_closed_form_and_reduction():
    g = torch.Generator().manual_seed(11)
    x = torch.randn(16, 5120, generator=g).to(torch.bfloat16)
    sc = (torch.randn(1, 5120, generator=g) * 0.1).to(torch.bfloat16)
    sh = (torch.randn(1, 5120, generator=g) * 0.1).to(torch.bfloat16)
    out = cpu_ref.rms_adaln(x, sc, sh, 1e-6)
    xd = x.double()
    n = xd / torch.sqrt((xd ** 2).mean(-1, keepdim=True) + 1e-6)
    exact = n * (1 + sc.double()) + sh.double()
    # four bf16 roundings (norm, 1+scale, product, sum), each <= 2^-8 relative
    # to the magnitude of the terms entering it
    mag = (n * (1 + sc.double())).abs() + sh.double().abs()
    assert ((out.double() - exact).abs() <= 4 * 2 ** -8 * mag + 1e-6).all()
    z = torch.zeros(1, 5120, dtype=torch.bfloat16)
    assert torch.equal(cpu_ref.rms_adaln(x, z, z, 1e-6), F.rms_norm(x, (5120,), eps=1e-6))


def test_rope_table_closed_form(pkg):
    from x_minimaxh3_amd import workloads

    grid = (3, 4, 5)
    t = cpu_ref.rope_table(cpu_ref.grid_positions(*grid))
    assert torch.equal(t, workloads.rope_table_3d(grid))
    pos = cpu_ref.grid_positions(*grid)
    p = 17
    tt, hh, ww = pos[p].tolist()
    angles = [tt * 10000 ** (-2 * i / 44) for i in range(22)] + \
             [hh * 10000 ** (-2 * i / 42) for i in range(21)] + [ww * 10000 ** (-2 * i / 42) for i in range(21)]
    for i, a in enumerate(angles):
        c, s = math.cos(a), math.sin(a)
        assert torch.allclose(t[0, p, 0, i].double(), torch.tensor([[c, -s], [s, c]], dtype=torch.float64),
                              atol=2e-6)
    assert torch.allclose(t[..., 0, 0] ** 2 + t[..., 1, 0] ** 2, torch.ones(()), atol=1e-6)


def test_rotation_identity_complex_and_norm():
    g = torch.Generator().manual_seed(12)
    x = torch.randn(1, 7, 3, 128, generator=g).to(torch.bfloat16)
    ident = torch.zeros(1, 7, 1, 64, 2, 2)
    ident[..., 0, 0] = 1
    ident[..., 1, 1] = 1
    assert torch.equal(cpu_ref.apply_rope_split_half1(x, ident), x)
    ang = torch.rand(1, 7, 1, 64, generator=g) * 6.28
    c, s = torch.cos(ang), torch.sin(ang)
    tab = torch.stack((c, -s, s, c), -1).reshape(1, 7, 1, 64, 2, 2)
    out = cpu_ref.apply_rope_split_half1(x, tab)
    z = torch.complex(x[..., :64].double(), x[..., 64:].double()) * torch.polar(torch.ones_like(ang.double()), ang.double())
    exact = torch.cat((z.real, z.imag), -1)
    assert ((out.double() - exact).abs() <= 2 ** -8 * exact.abs() + 1e-6).all()
    n0 = x[..., :64].double() ** 2 + x[..., 64:].double() ** 2
    n1 = out[..., :64].double() ** 2 + out[..., 64:].double() ** 2
    assert ((n0 - n1).abs() <= 2 ** -6 * n0 + 1e-6).all()


def test_interleaved_rope_against_split_half_and_fma():
    """apply_rope1 (pairs (2i, 2i+1)): with an fp32 table each output equals
    the float64 f0*x0 rounded to fp32, plus f1*x1, rounded once (the fused
    addcmul_), bit for bit; regrouping the pairs (de-interleave, rotate
    split-half, re-interleave) gives the same result within one fp32
    rounding before the final bf16 cast; an identity table returns x and
    rms_rope1 with it returns F.rms_norm; a longer table is trimmed."""
    g = torch.Generator().manual_seed(14)
    x = torch.randn(1, 5, 3, 96, generator=g).to(torch.bfloat16)
    ang = torch.rand(1, 5, 1, 48, generator=g) * 6.28
    c, s = torch.cos(ang), torch.sin(ang)
    tab = torch.stack((c, -s, s, c), -1).reshape(1, 5, 1, 48, 2, 2)
    out = cpu_ref.apply_rope1(x, tab)
    x0, x1 = x[..., 0::2].double(), x[..., 1::2].double()
    f = tab.double()
    want = torch.empty(1, 5, 3, 96, dtype=torch.float64)
    for r in range(2):
        p = (f[..., r, 0] * x0).float().double()            # fl32(f0 * x0)
        want[..., r::2] = (p + f[..., r, 1] * x1).float().double()   # one rounding of the sum
    assert torch.equal(out, want.to(torch.bfloat16))
    deint = torch.cat((x[..., 0::2], x[..., 1::2]), -1)
    sh = cpu_ref.apply_rope_split_half1(deint, tab)
    regroup = torch.stack((sh[..., :48], sh[..., 48:]), -1).reshape(x.shape)
    assert (cpu_ref.bf16_ulp_diff(regroup, out) <= 1).all()
    ident = torch.zeros(1, 5, 1, 48, 2, 2)
    ident[..., 0, 0] = 1
    ident[..., 1, 1] = 1
    assert torch.equal(cpu_ref.apply_rope1(x, ident), x)
    w = (1 + 0.1 * torch.randn(96, generator=g)).to(torch.bfloat16)
    assert torch.equal(cpu_ref.rms_rope1(x, ident, w, 1e-6), F.rms_norm(x, (96,), weight=w, eps=1e-6))
    longer = torch.cat((tab, tab[:, :, :1].expand(1, 5, 4, 48, 2, 2)), 2)   # dim 2 is 3 long in x
    assert torch.equal(cpu_ref.apply_rope1(x, longer.contiguous()), cpu_ref.apply_rope1(x, tab.expand(1, 5, 3, 48, 2, 2)))


def test_angle_form_qknorm_rope_equals_the_table_form():
    """H3's angle-table branch (active * cos + (-second, first) * sin in the
    value dtype) equals the split-half table form with the table (cos, -sin,
    sin, cos) in the value dtype, bit for bit, partial rotation and
    pass-through tail included; and with an fp32 table it differs (the
    rounding point of the table matters)."""
    g = torch.Generator().manual_seed(15)
    S, H, D, rot = 41, 3, 128, 96
    x = torch.randn(S, H, D, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    half_angles = torch.rand(S, rot // 2, generator=g) * 40
    angles = torch.cat((half_angles, half_angles), -1)
    want = cpu_ref.qknorm_rope_angles(x, w, angles, 1e-5)
    c, s = torch.cos(half_angles), torch.sin(half_angles)
    tab16 = torch.stack((c, -s, s, c), -1).reshape(1, S, 1, rot // 2, 2, 2).to(torch.bfloat16)
    got = cpu_ref.rms_rope_split_half1(x.unsqueeze(0), tab16, w, 1e-5, rot)[0]
    assert torch.equal(got, want)
    tab32 = torch.stack((c, -s, s, c), -1).reshape(1, S, 1, rot // 2, 2, 2)
    assert not torch.equal(cpu_ref.rms_rope_split_half1(x.unsqueeze(0), tab32, w, 1e-5, rot)[0], want)
    assert torch.equal(want[..., rot:], F.rms_norm(x, (D,), weight=w, eps=1e-5)[..., rot:])


def test_rms_rope_partial_tail_is_norm_only():
    g = torch.Generator().manual_seed(13)
    x = torch.randn(1, 5, 2, 128, generator=g).to(torch.bfloat16)
    w = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16)
    ang = torch.rand(1, 5, 1, 48, generator=g)
    c, s = torch.cos(ang), torch.sin(ang)
    tab = torch.stack((c, -s, s, c), -1).reshape(1, 5, 1, 48, 2, 2).to(torch.bfloat16)
    out = cpu_ref.rms_rope_split_half1(x, tab, w, 1e-5, rot_dim=96)
    nrm = F.rms_norm(x, (128,), weight=w, eps=1e-5)
    assert torch.equal(out[..., 96:], nrm[..., 96:])
    assert not torch.equal(out[..., :96], nrm[..., :96])


def test_segmented_adaln_matches_per_segment_rms_adaln():
    g = torch.Generator().manual_seed(14)
    x = torch.randn(30, 256, generator=g).to(torch.bfloat16)
    sc = (torch.randn(3, 256, generator=g) * 0.1).to(torch.bfloat16)
    sh = (torch.randn(3, 256, generator=g) * 0.1).to(torch.bfloat16)
    segs = ((0, 7, 2), (7, 20, 0), (20, 30, 1))
    out = cpu_ref.rms_adaln_segmented(x, None, sh, sc, segs, eps=1e-5)
    for a, b, r in segs:
        assert torch.equal(out[a:b], cpu_ref.rms_adaln(x[a:b], sc[r:r + 1], sh[r:r + 1], 1e-5))


@pytest.mark.parametrize("d", [5120, 5376, 128, 1000, 96, 16384, 13824, 72])
def test_rms_norm_reduction_order_is_pinned(d):
    """The GPU norms sum squares in the order torch's CPU reduction uses on this
    image; the numpy restatement of that order must reproduce torch's sum (and
    through it F.rms_norm) exactly, or the order claim is wrong."""
    g = torch.Generator().manual_seed(d)
    xb = (torch.randn(24, d, generator=g) * torch.rand(24, 1, generator=g) * 10).to(torch.bfloat16)
    xf = xb.float()
    sq = (xf * xf).numpy()
    emu = np.array([npref.torch_cpu_sum_order(r) for r in sq])
    assert np.array_equal(emu.view(np.uint32), xf.pow(2).sum(-1).numpy().view(np.uint32))
    rr = (np.float32(1) / np.sqrt(((emu / np.float32(d)).astype(np.float32) + np.float32(1e-6)).astype(np.float32)))
    out = torch.from_numpy((xf.numpy() * rr.astype(np.float32)[:, None]).astype(np.float32)).to(torch.bfloat16)
    assert torch.equal(out, F.rms_norm(xb, (d,), eps=1e-6))


# --------------------------------------------------------------------------- ConvRot

def test_hadamard_closed_form_and_involution():
    """H[p][q] = prod over base-4 digits d of H4[p_d][q_d] / 16 (the regular
    Hadamard matrix built by Kronecker powers), symmetric, H @ H = I."""
    h4 = [[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]]
    h = cpu_ref.build_hadamard(256).double()
    want = torch.empty(256, 256, dtype=torch.float64)
    for p in range(256):
        for q in range(256):
            v = 1
            for d in range(4):
                v *= h4[(p >> (2 * d)) & 3][(q >> (2 * d)) & 3]
            want[p, q] = v / 16.0
    assert torch.equal(h, want)
    assert torch.equal(h, h.T)
    assert torch.equal(h @ h, torch.eye(256, dtype=torch.float64))
    # H4 has -1 exactly on its anti-diagonal (the identity the GPU stages use)
    assert all((h4[i][j] == -1) == (i + j == 3) for i in range(4) for j in range(4))
    for size in (4, 16, 64):
        hs = cpu_ref.build_hadamard(size).double()
        assert torch.allclose(hs @ hs, torch.eye(size, dtype=torch.float64), atol=1e-12)
    with pytest.raises(ValueError):
        cpu_ref.build_hadamard(128)


def test_rotate_activation_against_float64():
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(37, 1024, generator=g) * 3).to(torch.bfloat16)
    r = cpu_ref.rotate_activation(x, 256)
    h = cpu_ref.build_hadamard(256).double()
    exact = (x.double().reshape(37, 4, 256) @ h).reshape(37, 1024)
    ulp = torch.pow(2.0, torch.floor(torch.log2(exact.abs().clamp(min=2.0 ** -100))) - 7)
    assert ((r.double() - exact).abs() <= ulp).all()      # one bf16 rounding of the exact sum
    # integer-valued rows: every fp32 partial sum is exact, so the rotation is
    # the exact product rounded once to bf16, bit for bit
    xi = torch.randint(-40, 41, (23, 1024), generator=g).to(torch.bfloat16)
    ri = cpu_ref.rotate_activation(xi, 256)
    exact_i = (xi.double().reshape(23, 4, 256) @ h).reshape(23, 1024)
    assert torch.equal(ri, exact_i.to(torch.bfloat16))
    # a one-hot input picks a row of H (orientation of x @ H)
    e = torch.zeros(1, 256, dtype=torch.bfloat16)
    e[0, 37] = 1
    assert torch.equal(cpu_ref.rotate_activation(e, 256).double(), h[37].reshape(1, 256))
    # rotating weights offline and activations online leaves x @ W^T unchanged
    w = torch.randn(16, 256, generator=g, dtype=torch.float64)
    xd = torch.randn(5, 256, generator=g, dtype=torch.float64)
    rw = cpu_ref.rotate_weight(w, 256)
    assert torch.allclose((xd @ h) @ rw.T, xd @ w.T, atol=1e-10)


def test_quantize_convrot_swiglu_composition():
    """swiglu halves the row: gate | up -> silu(gate) * up, rotated per 256
    columns, quantized per token."""
    g = torch.Generator().manual_seed(12)
    raw = torch.randn(9, 1024, generator=g).to(torch.bfloat16)
    q, s, r = cpu_ref.quantize_convrot(raw, 256, "swiglu")
    assert q.shape == (9, 512) and s.shape == (9, 1) and r.shape == (9, 512)
    act = torch.nn.functional.silu(raw[:, :512]) * raw[:, 512:]
    assert torch.equal(act, cpu_ref.apply_input_act(raw, "swiglu"))
    qq, ss = cpu_ref.quantize_int8_rowwise(cpu_ref.rotate_activation(act, 256))
    assert torch.equal(q, qq) and torch.equal(s, ss)


def test_gated_residual_closed_form_and_row_map():
    """residual.addcmul_(y, T(gate[row])) per segment: the product of two bf16
    values is exact in fp32, so each output is r + y*g rounded once to fp32,
    then to bf16; the segment form equals a per-token gather through the row
    map."""
    g = torch.Generator().manual_seed(21)
    m, n = 97, 320
    segments = ((0, 40, 2), (40, 41, 0), (41, 97, 1))
    res = torch.randn(m, n, generator=g).to(torch.bfloat16)
    upd = torch.randn(m, n, generator=g).to(torch.bfloat16)
    gate = torch.randn(3, n, generator=g) * 0.3          # fp32, as the modulation chunk
    out = cpu_ref.gated_residual_(res.clone(), upd, gate, segments)
    rows = cpu_ref.segment_row_map(m, segments)
    assert rows.dtype == torch.int32 and rows[39] == 2 and rows[40] == 0 and rows[41] == 1
    gt = gate.to(torch.bfloat16)[rows.long()].double()
    exact = (res.double() + upd.double() * gt).float().to(torch.bfloat16)
    assert torch.equal(out, exact)
    with pytest.raises(ValueError):
        cpu_ref.segment_row_map(m, ((0, 40, 0), (41, 97, 1)))
    with pytest.raises(ValueError):
        cpu_ref.gated_residual_(res.clone(), upd, gate, ((0, 50, 0),))


def test_w4a8_correction_route_against_float_weight():
    """The GPU dispatcher's asymmetric route (int8 linear + group sums of the
    codes times the correction) against the eager float route
    (CK/backends/eager/w4a8_int8.py:405-491: W = rotate(w8 * s_channel +
    correction), x @ W^T): equal up to the activation quantization error, and
    a transposed or dropped correction is far off."""
    g = torch.Generator().manual_seed(5)
    m, n, k, gs = 48, 96, 512, 16
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    codes = torch.randint(-128, 128, (n, k // 2), generator=g, dtype=torch.int8)
    srel = (torch.rand(n, k // gs, generator=g) * 80 + 40).to(torch.float8_e4m3fn)
    sch = torch.rand(n, generator=g) * 2e-3 + 1e-3
    cb = torch.linspace(-0.98, 0.98, 16)
    corr = torch.randn(k // gs, n, generator=g) * 0.05
    got = cpu_ref.w4a8_linear_h3(x, codes, srel, sch, codebook=cb, correction=corr, group_size=gs,
                                 out_dtype=torch.float32)
    w8 = cpu_ref.dequant_int4_grouped_to_int8(codes, srel.float(), gs, codebook=cb).double()
    w_rot = (w8.view(n, k // gs, gs) * sch.double().view(n, 1, 1) + corr.double().T.unsqueeze(-1)).view(n, k)
    h = cpu_ref.build_hadamard(256).double()
    w_phys = (w_rot.view(n, k // 256, 256) @ h).view(n, k)
    want = x.double() @ w_phys.T
    cos = torch.nn.functional.cosine_similarity(got.double().flatten(), want.flatten(), dim=0).item()
    assert cos > 0.9999
    no_corr = cpu_ref.w4a8_linear_h3(x, codes, srel, sch, codebook=cb, group_size=gs, out_dtype=torch.float32)
    assert torch.nn.functional.cosine_similarity(no_corr.double().flatten(), want.flatten(), dim=0).item() < 0.999
    # group sums: brute force
    q = torch.randint(-128, 128, (5, 64), generator=g, dtype=torch.int8)
    xs = torch.rand(5, 1, generator=g)
    sums = cpu_ref.int8_group_sums(q, xs, 16, torch.float32)
    for r in range(5):
        for grp in range(4):
            total = torch.tensor(float(int(q[r, 16 * grp:16 * grp + 16].int().sum())))
            assert sums[r, grp].item() == (total * xs[r, 0]).item()      # one fp32 product


# --------------------------------------------------------------------------- composites

def _rand_scales(n, seed, lo=1e-4, hi=1e-3):
    g = torch.Generator().manual_seed(seed)
    return torch.rand(n, generator=g) * (hi - lo) + lo


def _bf16_chain_linear(x_bits, w, sw):
    """Step-by-step W8A8 linear on bit patterns: quantize (numpy rule), int64
    matmul, fp32 dequant rounded once to bf16. Returns bf16 bits."""
    q, s = npref.quantize_rows_bf16(x_bits)
    acc = npref.int_mm(q, w)
    return npref.dequant_bf16_bits(acc, s, sw)


def test_w8a8_mlp_composite_step_by_step():
    """cpu_ref.w8a8_mlp = fc1 int8 linear, GELU-tanh on the bf16 h (the library
    routine on bf16, the reference's materialisation point), per-token requant,
    fc2 int8 linear. A GELU applied to the fp32 accumulators, after the
    requant, or a skipped bf16 rounding of h changes bits here."""
    m, d, f = 64, 256, 512
    x = outlier_acts(m, d, seed=31, n_out=4)
    g = torch.Generator().manual_seed(32)
    w1 = torch.randint(-127, 128, (f, d), generator=g, dtype=torch.int8)
    w2 = torch.randint(-127, 128, (d, f), generator=g, dtype=torch.int8)
    s1, s2 = _rand_scales(f, 33, 1e-4, 4e-4), _rand_scales(d, 34, 1e-4, 4e-4)
    y = cpu_ref.w8a8_mlp(x, w1, s1, w2, s2)
    h = _bf16_chain_linear(bits(x), w1.numpy(), s1.numpy())
    gl = F.gelu(from_bits(h), approximate="tanh")
    assert gl.dtype == torch.bfloat16
    yn = _bf16_chain_linear(bits(gl), w2.numpy(), s2.numpy())
    assert np.array_equal(bits(y), yn)
    # the GELU input is h itself (not the fp32 accumulators): a chain that
    # rounds GELU of the unrounded dequant differs somewhere
    q1, sx1 = npref.quantize_rows_bf16(bits(x))
    acc1 = npref.int_mm(q1, w1.numpy())
    h32 = (acc1.astype(np.float32) * (sx1[:, None] * s1.numpy()[None, :]).astype(np.float32)).astype(np.float32)
    g32 = F.gelu(torch.from_numpy(h32), approximate="tanh").to(torch.bfloat16)
    assert not torch.equal(g32, gl)


def test_w4a8_linear_and_mlp_composite_step_by_step():
    """cpu_ref.w4a8_linear / w4a8_mlp = grouped int4 decode to the int8 grid
    (numpy restatement), then the W8A8 chain with s_channel as the
    per-channel weight scale."""
    m, d, f, gs = 64, 256, 512, 128
    x = outlier_acts(m, d, seed=35, n_out=4)
    g = torch.Generator().manual_seed(36)
    w1 = torch.randn(f, d, generator=g) * 0.02
    w2 = torch.randn(d, f, generator=g) * 0.02
    p1, r1, c1 = cpu_ref.quantize_w4_weight(w1, gs)
    p2, r2, c2 = cpu_ref.quantize_w4_weight(w2, gs)
    w8_1 = npref.w4_decode(p1.numpy(), r1.numpy(), gs)
    w8_2 = npref.w4_decode(p2.numpy(), r2.numpy(), gs)
    h = _bf16_chain_linear(bits(x), w8_1, c1.numpy())
    assert np.array_equal(bits(cpu_ref.w4a8_linear(x, p1, r1, c1, gs)), h)
    gl = F.gelu(from_bits(h), approximate="tanh")
    yn = _bf16_chain_linear(bits(gl), w8_2, c2.numpy())
    assert np.array_equal(bits(cpu_ref.w4a8_mlp(x, p1, r1, c1, p2, r2, c2, gs)), yn)
    # a decode with swapped nibbles is a different weight grid
    swapped = ((p1.numpy().view(np.uint8) >> 4) | (p1.numpy().view(np.uint8) << 4)).astype(np.uint8).view(np.int8)
    assert not np.array_equal(npref.w4_decode(swapped, r1.numpy(), gs), w8_1)


def test_int8_linear_gated_residual_composite():
    """The H3 fc2 boundary without rotation: the int8 projection in the
    residual's dtype, then residual[t] += y[t] * bf16(gate[row(t)]) with the
    exact fp32 product and one fp32 and one bf16 rounding of the sum."""
    m, k, n = 50, 256, 192
    x = outlier_acts(m, k, seed=37, n_out=4)
    g = torch.Generator().manual_seed(38)
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    sw = _rand_scales(n, 39, 1e-4, 4e-4)
    res = torch.randn(m, n, generator=g).to(torch.bfloat16)
    gate = torch.randn(3, n, generator=g) * 0.3
    segs = ((0, 11, 1), (11, 30, 2), (30, 50, 0))
    out = cpu_ref.int8_linear_gated_residual_(x, w, sw, None, res.clone(), gate, segs, convrot=False,
                                              input_act=None)
    y = from_bits(_bf16_chain_linear(bits(x), w.numpy(), sw.numpy())).double()
    rows = torch.tensor([r for a, b, r in segs for _ in range(a, b)])
    want = (res.double() + y * gate.to(torch.bfloat16)[rows].double()).float().to(torch.bfloat16)
    assert torch.equal(out, want)


def test_norm_rope_composite():
    """cpu_ref.norm_rope = rms_adaln over the whole row, then the split-half
    rotation per head of head_dim columns: an identity table gives rms_adaln
    bit for bit; a float64 per-head complex product (heads laid out as
    consecutive column blocks, pairs (i, i + head_dim/2)) matches within one
    bf16 rounding; tokens are independent, so swapping two tokens together
    with their table rows swaps the outputs exactly."""
    g = torch.Generator().manual_seed(41)
    m, heads, hd = 6, 5, 128
    d = heads * hd
    x = torch.randn(m, d, generator=g).to(torch.bfloat16)
    sc = (torch.randn(1, d, generator=g) * 0.1).to(torch.bfloat16)
    sh = (torch.randn(1, d, generator=g) * 0.1).to(torch.bfloat16)
    ident = torch.zeros(1, m, 1, hd // 2, 2, 2)
    ident[..., 0, 0] = 1
    ident[..., 1, 1] = 1
    a = cpu_ref.rms_adaln(x, sc, sh, 1e-6)
    assert torch.equal(cpu_ref.norm_rope(x, sc, sh, ident, hd, 1e-6), a)
    ang = torch.rand(m, hd // 2, generator=g) * 6.28
    c, s = torch.cos(ang), torch.sin(ang)
    tab = torch.stack((c, -s, s, c), -1).reshape(1, m, 1, hd // 2, 2, 2)
    out = cpu_ref.norm_rope(x, sc, sh, tab, hd, 1e-6).double()
    ad = a.double()
    exact = torch.empty(m, d, dtype=torch.float64)
    for h in range(heads):
        lo, hi = ad[:, h * hd: h * hd + hd // 2], ad[:, h * hd + hd // 2: (h + 1) * hd]
        z = torch.complex(lo, hi) * torch.polar(torch.ones_like(ang.double()), ang.double())
        exact[:, h * hd: h * hd + hd // 2] = z.real
        exact[:, h * hd + hd // 2: (h + 1) * hd] = z.imag
    assert ((out - exact).abs() <= 2 ** -8 * exact.abs() + 1e-6).all()
    perm = torch.tensor([3, 1, 2, 0, 5, 4])
    out_p = cpu_ref.norm_rope(x[perm], sc, sh, tab[:, perm], hd, 1e-6)
    assert torch.equal(out_p, cpu_ref.norm_rope(x, sc, sh, tab, hd, 1e-6)[perm])
