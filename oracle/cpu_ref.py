"""torch-CPU restatement of the reference's eager path (the oracle).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): imported by tests,
by ``__graft_entry__.smoke()`` as the checker and by ``bench.py``'s
``cpu_baseline`` leg. The product path never imports it.

Citations are relative to the reference root; ``CK/`` abbreviates the
vendored kernel library ``backends/turbo/vendor/comfy_kitchen/``.

Every function follows the reference's op order exactly and calls the same
torch CPU routines the reference calls (``torch._int_mm``, ``F.gelu``,
``F.rms_norm``), so the rounding points (each bf16 materialisation) are the
reference's own.

Pinning (what checks each function independently of this file; the tests
live in ``tests/test_oracle.py``):

* ``quantize_int8_rowwise``  -- numpy restatement (``npref``), the C
  restatement (``c/oracle.c``) and hand-built special cases (zero row,
  -127.5 -> -128, +127.5 -> 127, half-to-even ties). Its stochastic form:
  the C restatement of the bf16 case (fp32 add then one bf16 rounding, a
  different route to the same single rounding), ``round_to_dtype`` against
  torch's own fp32 -> bf16 / fp16 conversions, the keying identities of the
  noise (seed + 1 at idx == seed at idx + 1; the 64-bit fold), the range
  and uniformity of the hash output, codes in {floor(v), floor(v) + 1} and
  their mean over seeds against v (unbiasedness).
* ``int8_mm``                -- int64 brute force (numpy and C).
* ``dequant``/``int8_linear``-- float64 closed form + the C restatement of
  the fp32 epilogue; composite order vs a step-by-step numpy restatement.
* ``gelu_tanh``              -- the library routine itself (``F.gelu``),
  checked against the float64 closed form within 1 bf16 ulp.
* ``quantize_w4_weight`` / ``dequant_int4_grouped_to_int8`` -- numpy
  restatement, pure-Python loops on tiny inputs, nibble-order and
  round-trip invariants.
* ``build_hadamard`` / ``rotate_activation`` / ``rotate_weight`` -- the
  closed form H[p][q] = prod_d H4[p_d][q_d] / 16 over base-4 digits,
  symmetry and H @ H = I, one-hot columns, and float64 x @ H within one bf16
  rounding, bit-exact on integer-valued rows (exact fp32 sums);
  ``quantize_convrot`` is their composition with ``quantize_int8_rowwise``
  (parity unpinned at the last bit of the rotated row where its fp32 sums are
  inexact: the reference's bf16 matmul accumulates in a library-defined
  order).
* ``segment_row_map`` / ``gated_residual_`` / ``int8_linear_gated_residual_``
  -- the same torch ``addcmul_`` the reference calls; pinned by the float64
  closed form (the product of two bf16 values is exact in fp32, so the result
  is the exact r + y*g rounded once to fp32 and once to bf16) and by the
  row-map equivalence with a per-token gather.
* ``rms_adaln`` / ``rms_norm`` -- float64 closed form within 1 bf16 ulp and
  the special case scale=shift=0 reducing to ``F.rms_norm``.
* ``rope_table``             -- closed form (cos/sin of integer position
  times theta^(-2i/dim)) and the unit-modulus invariant.
* ``apply_rope_split_half1`` -- complex-multiplication form, identity table
  reduces to the input, norm-preservation invariant.
* ``apply_rope1`` / ``rms_rope1`` (interleaved pairs) -- the split-half form
  on the de-interleaved head (same rotation, pairs regrouped) within one
  rounding of the table dtype, the addcmul_ step equal to a float64 fused
  multiply-add rounded once, identity table reduces to the input (or to
  ``F.rms_norm``).
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

DTYPE_CODE_TO_DTYPE = {0: torch.float32, 1: torch.float16, 2: torch.bfloat16}


# ---------------------------------------------------------------------------
# a1: per-token dynamic int8 quantisation
# ---------------------------------------------------------------------------

def _int8_scale_for_math(scale: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """CK/backends/eager/quantization.py:815-818: the scale in x's dtype,
    zeros replaced by that dtype's smallest normal."""
    scale = scale.to(dtype=x.dtype)
    tiny = torch.finfo(x.dtype).tiny
    return torch.where(scale == 0, torch.full_like(scale, tiny), scale)


def quantize_int8_rowwise(x: torch.Tensor, stochastic_rounding: int | None = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """CK/backends/eager/quantization.py:857-875 (with _round_int8 :821-826).

    amax in x's dtype; scale = max(amax.float()/127, 1e-30) (fp32, true
    division); v = x / scale.to(x.dtype) in x's dtype; round half to even;
    clamp [-128, 127]. Returns (int8 [...,K], fp32 [...,1]) with the
    unrounded fp32 scale.

    stochastic_rounding = seed > 0: v as above, then floor(T(v + noise)) with
    the reference CUDA quantizer's deterministic noise of each element
    (``stochastic_noise``; CK/backends/cuda/ops/int8_linear.cu:186-195), the
    sum rounded once to x's dtype. The eager backend draws its noise from a
    seeded torch generator (:803-812), whose stream depends on the device and
    the torch build, so its stochastic codes cannot be reproduced elsewhere;
    the CUDA backend's hash is the reproducible definition.
    """
    abs_max = x.abs().amax(dim=-1, keepdim=True)
    scale = (abs_max.float() / 127.0).clamp(min=1e-30)
    scaled = x / _int8_scale_for_math(scale, x)
    if stochastic_rounding is not None and stochastic_rounding > 0:
        idx = np.arange(x.numel(), dtype=np.uint64)          # row * K + col of the [..., K] matrix
        noise = stochastic_noise(idx, int(stochastic_rounding), x.dtype).reshape(tuple(x.shape))
        summed = round_to_dtype(scaled.double().numpy() + noise, x.dtype)   # exact sum, one rounding
        q = torch.from_numpy(np.floor(summed)).clamp_(-128.0, 127.0).to(torch.int8)
        return q, scale
    q = scaled.round_().clamp_(-128.0, 127.0).to(torch.int8)
    return q, scale


def pcg_hash(x: np.ndarray) -> np.ndarray:
    """The 32-bit PCG-RXS-M-XS output hash (O'Neill's PCG family, as the GPU
    hash of Jarzynski and Olano, "Hash Functions for GPU Rendering", JCGT 9(3)
    2020) that keys the reference's stochastic rounding noise
    (CK/backends/cuda/ops/int8_linear.cu:79-83). uint32 in, uint32 out."""
    x = np.asarray(x, dtype=np.uint32)
    with np.errstate(over="ignore"):
        state = x * np.uint32(747796405) + np.uint32(2891336453)
        word = ((state >> ((state >> np.uint32(28)) + np.uint32(4))) ^ state) * np.uint32(277803737)
    return (word >> np.uint32(22)) ^ word


def round_to_dtype(x64: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """float64 values -> the nearest value of ``dtype`` (bf16, fp16 or fp32),
    ties to even, in one rounding, subnormals included; returned as float64."""
    p, emin = {torch.bfloat16: (8, -126), torch.float16: (11, -14), torch.float32: (24, -126)}[dtype]
    x64 = np.asarray(x64, dtype=np.float64)
    _, e = np.frexp(x64)                                   # x = m * 2^e, 0.5 <= |m| < 1
    quantum = np.maximum(e - 1, emin) - (p - 1)            # exponent of the last significand bit
    return np.ldexp(np.rint(np.ldexp(x64, -quantum)), quantum)


def stochastic_noise(idx: np.ndarray, seed: int, dtype: torch.dtype) -> np.ndarray:
    """CK/backends/cuda/ops/int8_linear.cu:85-91: key = idx + seed (uint64,
    wrapping), folded = lo32(key) ^ hi32(key), u = (pcg_hash(folded) >> 8) *
    2^-24 in [0, 1), rounded to ``dtype`` (bf16 can round it up to 1.0).
    float64 out."""
    with np.errstate(over="ignore"):
        key = np.asarray(idx, dtype=np.uint64) + np.uint64(seed)
    folded = ((key & np.uint64(0xFFFFFFFF)) ^ (key >> np.uint64(32))).astype(np.uint32)
    u = (pcg_hash(folded) >> np.uint32(8)).astype(np.float64) * 2.0 ** -24
    return round_to_dtype(u, dtype)


# ---------------------------------------------------------------------------
# a2: input activation
# ---------------------------------------------------------------------------

def apply_input_act(x: torch.Tensor, input_act: str | None) -> torch.Tensor:
    """CK/backends/_activations.py:40-53."""
    if input_act in (None, "none"):
        return x
    if input_act == "gelu_tanh":
        return F.gelu(x, approximate="tanh")
    if input_act == "swiglu":
        gate, up = x.chunk(2, dim=-1)
        return F.silu(gate).mul_(up)
    raise ValueError(f"unsupported input_act: {input_act!r}")


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    return apply_input_act(x, "gelu_tanh")


# ---------------------------------------------------------------------------
# a3/a4: int8 GEMM and the dequant epilogue
# ---------------------------------------------------------------------------

def int8_mm(a: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """CK/backends/eager/quantization.py:749-783 on CPU: int32 accumulators of
    a[M,K] @ w[N,K]^T. On CPU the reference pads K to a multiple of 8 and N to
    a multiple of 8 with zeros (no effect on the sums) and calls torch._int_mm."""
    m, k = a.shape
    n = w.shape[0]
    b = w.t().contiguous()
    if m == 0 or k == 0:
        return torch.zeros(m, n, dtype=torch.int32)
    pk = (k + 7) // 8 * 8
    if pk != k:
        a = torch.cat((a, torch.zeros(m, pk - k, dtype=a.dtype)), dim=1)
        b = torch.cat((b, torch.zeros(pk - k, n, dtype=b.dtype)), dim=0)
    pn = (n + 7) // 8 * 8
    if pn != n:
        b = torch.cat((b, torch.zeros(b.shape[0], pn - n, dtype=b.dtype)), dim=1)
    return torch._int_mm(a, b)[:, :n]


def dequant(acc: torch.Tensor, x_scale: torch.Tensor, w_scale: torch.Tensor,
            out_dtype: torch.dtype = torch.bfloat16,
            bias: torch.Tensor | None = None) -> torch.Tensor:
    """CK/backends/eager/quantization.py:1028-1054: out = (acc.float() *
    (x_scale * w_scale)).to(out_dtype), the scale product formed first in
    fp32, then bias added in out_dtype."""
    ws = w_scale.to(torch.float32).reshape(1, -1)
    out = (acc.float() * (x_scale.to(torch.float32).reshape(-1, 1) * ws)).to(out_dtype)
    if bias is not None:
        out = out + bias.to(dtype=out.dtype).reshape(1, -1)
    return out


# ---------------------------------------------------------------------------
# ConvRot: the online Hadamard rotation of the rotated linears
# ---------------------------------------------------------------------------

def build_hadamard(size: int, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """CK/tensor/int8_utils.py:11-39: the regular Hadamard matrix
    H4 (x) H4 (x) ... (size a power of 4), normalised by 1/sqrt(size)."""
    if size < 4 or (size & (size - 1)) != 0 or math.log(size, 4) % 1 != 0:
        raise ValueError(f"Regular Hadamard size must be a power of 4, got {size}")
    h4 = torch.tensor([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=dtype)
    h = h4
    n = 4
    while n < size:
        h = torch.kron(h, h4)
        n *= 4
    return h / (size ** 0.5)


def rotate_activation(x: torch.Tensor, group_size: int) -> torch.Tensor:
    """CK/tensor/int8_utils.py:58-74 as called by the eager int8_linear
    (CK/backends/eager/quantization.py:1012-1017): per group of group_size
    columns x_g @ H, H built in x's dtype, the matmul in x's dtype."""
    k = x.shape[-1]
    if k % group_size != 0:
        raise ValueError(f"features {k} not divisible by group_size {group_size}")
    h = build_hadamard(group_size).to(x.dtype)
    return torch.matmul(x.reshape(-1, k // group_size, group_size), h).reshape(x.shape)


def rotate_weight(w: torch.Tensor, group_size: int) -> torch.Tensor:
    """CK/tensor/int8_utils.py:42-55: W_rot = W_g @ H^T offline (fp32)."""
    n, k = w.shape
    h = build_hadamard(group_size).to(w.dtype)
    return torch.matmul(w.reshape(n, k // group_size, group_size), h.T).reshape(n, k)


def quantize_convrot(x: torch.Tensor, group_size: int = 256, input_act: str | None = None,
                     stochastic_rounding: int | None = 0):
    """The quantizer of a rotated linear: act -> rotate -> quantize_int8_rowwise
    (the eager order of CK/backends/eager/quantization.py:998-1023); with a
    seed, the codes are rounded stochastically with the noise of each code's
    index in the [M, K] output (CK/backends/cuda/ops/int8_linear.cu:1019-1021)."""
    a = apply_input_act(x, input_act)
    r = rotate_activation(a, group_size)
    q, s = quantize_int8_rowwise(r.reshape(-1, r.shape[-1]), stochastic_rounding)
    return q, s, r


def int8_linear(x: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
                bias: torch.Tensor | None = None,
                out_dtype: torch.dtype = torch.bfloat16,
                input_act: str | None = None,
                return_parts: bool = False,
                convrot: bool = False, convrot_groupsize: int = 256):
    """CK/backends/eager/quantization.py:971-1056:
    act -> (rotate) -> rowwise quant -> int8 GEMM -> fp32 dequant -> cast -> bias."""
    x = apply_input_act(x, input_act)
    if convrot:
        x = rotate_activation(x, convrot_groupsize)
    if x.shape[-1] != weight.shape[-1]:
        raise ValueError("Input and weight inner dimensions must match")
    ws = weight_scale.to(torch.float32).reshape(-1)
    if ws.numel() not in (1, weight.shape[0]):
        raise ValueError("INT8 weight scale must be scalar or per-output-channel")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    q, s = quantize_int8_rowwise(x2)
    acc = int8_mm(q, weight)
    out = dequant(acc, s, ws, out_dtype, bias).reshape(*lead, weight.shape[0])
    if return_parts:
        return out, {"act": x2, "q": q, "scale": s, "acc": acc}
    return out


# ---------------------------------------------------------------------------
# the H3 fc2 boundary: projection, then the AdaLN-gated residual update
# ---------------------------------------------------------------------------

def segment_row_map(length: int, segments) -> torch.Tensor:
    """int32 [length]: the modulation row of every token
    (h3serve/native_engine/model/fused_mlp.py:34-55; the segments must be an
    ordered partition of [0, length))."""
    out = torch.empty(length, dtype=torch.int32)
    previous = 0
    for start, stop, row in segments:
        if start != previous or stop <= start:
            raise ValueError("modulation segments must be an ordered partition")
        out[start:stop] = row
        previous = stop
    if previous != length:
        raise ValueError("modulation segments do not cover the packed sequence")
    return out


def gated_residual_(residual: torch.Tensor, update: torch.Tensor, gate: torch.Tensor, segments) -> torch.Tensor:
    """residual[a:b].addcmul_(update[a:b], gate[row].to(update.dtype)) per
    segment (h3serve/native_engine/model/layers.py:937-953), in place."""
    previous = 0
    for start, stop, row in segments:
        if start != previous or stop <= start:
            raise ValueError("modulation segments must be an ordered partition")
        residual[start:stop].addcmul_(update[start:stop], gate[row].to(update.dtype))
        previous = stop
    if previous != residual.shape[0]:
        raise ValueError("modulation segments do not cover the packed sequence")
    return residual


def int8_linear_gated_residual_(x: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
                                bias: torch.Tensor | None, residual: torch.Tensor, gate: torch.Tensor,
                                segments, convrot: bool = True, convrot_groupsize: int = 256,
                                input_act: str | None = "swiglu") -> torch.Tensor:
    """The default fc2 route of the H3 block
    (h3serve/native_engine/model/fused_mlp.py:396-426): int8_linear in the
    residual's dtype, then the gated residual update per segment."""
    projected = int8_linear(x, weight, weight_scale, bias, out_dtype=residual.dtype, input_act=input_act,
                            convrot=convrot, convrot_groupsize=convrot_groupsize)
    return gated_residual_(residual, projected, gate, segments)


# ---------------------------------------------------------------------------
# a5/a6: the W8A8 MLP block  y = fc2(gelu_tanh(fc1(x)))
# ---------------------------------------------------------------------------

def w8a8_mlp(x: torch.Tensor, w1: torch.Tensor, s1: torch.Tensor,
             w2: torch.Tensor, s2: torch.Tensor, return_parts: bool = False):
    """fc1 = int8_linear(x, W1, s1); fc2 = int8_linear(fc1, W2, s2,
    input_act="gelu_tanh") -- the reference op API form of the GELU-tanh MLP
    (CK/__init__.py:722-764; the H3 driver's fc2 call with a fused input act,
    h3serve/native_engine/model/fused_mlp.py:396-405)."""
    h, p1 = int8_linear(x, w1, s1, return_parts=True)
    y, p2 = int8_linear(h, w2, s2, input_act="gelu_tanh", return_parts=True)
    if return_parts:
        return y, {"q1": p1["q"], "s1": p1["scale"], "acc1": p1["acc"], "h": h,
                   "g": p2["act"], "q2": p2["q"], "s2": p2["scale"], "acc2": p2["acc"]}
    return y


# ---------------------------------------------------------------------------
# a7/a8: W4A8 (int4 grouped, uniform levels, no rotation)
# ---------------------------------------------------------------------------

def quantize_w4_weight(weight: torch.Tensor, group_size: int = 128):
    """CK/backends/eager/w4a8_int8.py:122-209, branch symmetric=True,
    codebook=False, scale_dtype=float32 (:169-173, :188-191):

    gs = max(amax_g/7, 1e-8); signed = clamp(round(w/gs), -8, 7);
    u = signed + 8; s_channel = max(amax_n(|signed*gs|)/127, 1e-8);
    s_rel = gs / s_channel; byte = (u[2j] & 0xF) | (u[2j+1] << 4).
    Returns (packed int8 [N,K/2], s_rel fp32 [N,K/G], s_channel fp32 [N]).
    """
    n, k = weight.shape
    groups = k // group_size
    gw = weight.float().view(n, groups, group_size)
    group_scale = (gw.abs().amax(dim=-1, keepdim=True) / 7.0).clamp(min=1e-8)
    signed = (gw / group_scale).round().clamp(-8, 7).to(torch.int32)
    unsigned = (signed + 8).view(n, k)
    shifted = signed * group_scale
    s_channel = (shifted.abs().amax(dim=(1, 2)) / 127.0).clamp(min=1e-8)
    s_rel = (group_scale.squeeze(-1) / s_channel.unsqueeze(1)).float().contiguous()
    packed = ((unsigned[:, 0::2] & 0xF) | ((unsigned[:, 1::2] & 0xF) << 4)).to(torch.int8).contiguous()
    return packed, s_rel, s_channel.float().contiguous()


def dequant_int4_grouped_to_int8(qdata: torch.Tensor, s_rel: torch.Tensor,
                                 group_size: int, codebook: torch.Tensor | None = None) -> torch.Tensor:
    """CK/backends/eager/w4a8_int8.py:344-363: code[2j] = b & 0xF,
    code[2j+1] = (b >> 4) & 0xF; level = code - 8 (or codebook[code]);
    int8 = clamp(round(level * s_rel.float()), -127, 127)."""
    n, k_half = qdata.shape
    k = k_half * 2
    groups = k // group_size
    packed = qdata.to(torch.int32) & 0xFF
    quantized = torch.empty(n, k, dtype=torch.int32)
    quantized[:, 0::2] = packed & 0xF
    quantized[:, 1::2] = (packed >> 4) & 0xF
    if codebook is not None:
        values = codebook.to(torch.float32)[quantized]
    else:
        values = quantized.float() - 8.0
    values = values.view(n, groups, group_size) * s_rel.float().unsqueeze(-1)
    return values.view(n, k).round().clamp_(-127, 127).to(torch.int8)


def w4a8_linear(x: torch.Tensor, qdata: torch.Tensor, s_rel: torch.Tensor,
                s_channel: torch.Tensor, group_size: int = 128,
                bias: torch.Tensor | None = None, out_dtype: torch.dtype = torch.bfloat16,
                input_act: str | None = None, convrot: bool = False,
                convrot_groupsize: int = 256) -> torch.Tensor:
    """CK/backends/eager/w4a8_int8.py:457-508: decode to the int8 grid, then
    int8_linear with s_channel as the per-channel weight scale (the reference
    always passes convrot=True; False gives the unrotated GELU-MLP form)."""
    w8 = dequant_int4_grouped_to_int8(qdata, s_rel, group_size)
    return int8_linear(x, w8, s_channel, bias=bias, out_dtype=out_dtype, input_act=input_act,
                       convrot=convrot, convrot_groupsize=convrot_groupsize)


def int8_group_sums(q: torch.Tensor, xs: torch.Tensor, group_size: int, out_dtype: torch.dtype) -> torch.Tensor:
    """CK/backends/cuda/__init__.py:2294-2296: the per-group sums of the
    activation codes in out_dtype, times the row scale in out_dtype."""
    m, k = q.shape
    sx = q.view(m, k // group_size, group_size).sum(-1, dtype=torch.int32).to(out_dtype)
    return sx * xs.reshape(m, 1).to(out_dtype)


def w4a8_linear_h3(x: torch.Tensor, qdata: torch.Tensor, s_rel: torch.Tensor, s_channel: torch.Tensor,
                   codebook: torch.Tensor | None = None, correction: torch.Tensor | None = None,
                   bias: torch.Tensor | None = None, group_size: int = 16, convrot_groupsize: int = 256,
                   out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """The H3 checkpoint form of w4a8_int8_linear (group 16, fp8 s_rel, codebook,
    ConvRot, asymmetric correction), as the reference's GPU dispatcher runs it
    (CK/backends/cuda/__init__.py:2164-2298): ConvRot row quantizer, codebook
    decode to the int8 grid, int8 linear with s_channel, and with a correction
    out.addmm_(int8_group_sums(q, xs), correction.to(out_dtype)). (The eager
    reference, CK/backends/eager/w4a8_int8.py:457-491, takes the asymmetric
    case through a floating dequantised weight instead; the two agree to the
    activation quantization error.)"""
    lead = x.shape[:-1]
    k = x.shape[-1]
    x2 = rotate_activation(x.reshape(-1, k), convrot_groupsize)
    q, xs = quantize_int8_rowwise(x2)
    w8 = dequant_int4_grouped_to_int8(qdata, s_rel.float(), group_size, codebook=codebook)
    ws = s_channel.to(torch.float32).reshape(-1)
    out = dequant(int8_mm(q, w8), xs, ws, out_dtype, bias)
    if correction is not None:
        out.addmm_(int8_group_sums(q, xs, group_size, out_dtype), correction.to(out_dtype))
    return out.reshape(*lead, qdata.shape[0])


def w4a8_mlp(x, w1_packed, w1_srel, w1_sch, w2_packed, w2_srel, w2_sch, group_size=128):
    h = w4a8_linear(x, w1_packed, w1_srel, w1_sch, group_size)
    return w4a8_linear(h, w2_packed, w2_srel, w2_sch, group_size, input_act="gelu_tanh")


# ---------------------------------------------------------------------------
# a9: (segmented) AdaLN-modulated RMSNorm
# ---------------------------------------------------------------------------

def rms_adaln(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor,
              eps: float = 1e-6) -> torch.Tensor:
    """CK/backends/eager/adaln.py:17-20:
    F.rms_norm(x, (D,), eps) * (1 + scale) + shift, every op in torch's
    promoted dtype (bf16 x and bf16 scale/shift round after each op)."""
    normalized = F.rms_norm(x, x.shape[-1:], eps=eps)
    return normalized * (1 + scale) + shift


def rms_norm(x: torch.Tensor, weight: torch.Tensor | None, eps: float) -> torch.Tensor:
    """h3serve/native_engine/model/layers.py:39-48 (RMSNorm.forward)."""
    w = None if weight is None else weight.to(dtype=x.dtype)
    return F.rms_norm(x, (x.shape[-1],), weight=w, eps=eps)


def rms_adaln_segmented(value: torch.Tensor, norm_weight: torch.Tensor | None,
                        shift: torch.Tensor, scale: torch.Tensor,
                        segments, eps: float = 1e-5) -> torch.Tensor:
    """h3serve/native_engine/model/kernels.py:7623-7634 (the eager order of
    rms_adaln with segments): hidden = RMSNorm(value); per segment
    hidden.mul_(1 + scale[row]).add_(shift[row])."""
    hidden = rms_norm(value, norm_weight, eps)
    previous = 0
    for start, stop, row in segments:
        if start != previous or stop <= start:
            raise ValueError("modulation segments must be an ordered partition")
        hidden[start:stop].mul_(1.0 + scale[row].to(hidden.dtype)).add_(shift[row].to(hidden.dtype))
        previous = stop
    if previous != hidden.shape[0]:
        raise ValueError("modulation segments do not cover the packed sequence")
    return hidden


# ---------------------------------------------------------------------------
# a10: RoPE table for a T x H x W token grid
# ---------------------------------------------------------------------------

def grid_positions(t: int, h: int, w: int) -> torch.Tensor:
    """t-major integer positions [(t,h,w)] (h3serve/native_engine/model/packed.py:343)."""
    tt, hh, ww = torch.meshgrid(torch.arange(t), torch.arange(h), torch.arange(w), indexing="ij")
    return torch.stack((tt.reshape(-1), hh.reshape(-1), ww.reshape(-1)), dim=-1)


def axis_inv_freq(dims=(44, 42, 42), theta: float = 10000.0) -> list[torch.Tensor]:
    """theta^(-2i/dim) for i < dim/2, per axis: evaluated in float64, then
    rounded once to fp32."""
    return [(1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float64) / d))).float() for d in dims]


def rope_table(positions: torch.Tensor, dims=(44, 42, 42), theta: float = 10000.0,
               dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """h3serve/native_engine/model/layers.py:51-69: per-axis angles pos*inv_freq
    concatenated [t|h|w]; table = stack(cos, -sin, sin, cos) as
    [1, S, 1, half, 2, 2] in ``dtype``."""
    inv = axis_inv_freq(dims, theta)
    per_axis = [positions[:, a:a + 1].float() * inv[a].reshape(1, -1) for a in range(3)]
    angles = torch.cat(per_axis, dim=-1)              # [S, half]
    cosine, sine = torch.cos(angles), torch.sin(angles)
    half = angles.shape[-1]
    return torch.stack((cosine, -sine, sine, cosine), dim=-1).reshape(
        1, angles.shape[0], 1, half, 2, 2).to(dtype)


# ---------------------------------------------------------------------------
# a11/a12: split-half RoPE, with or without the per-head RMSNorm
# ---------------------------------------------------------------------------

def apply_rope_split_half1(x: torch.Tensor, freqs_cis: torch.Tensor) -> torch.Tensor:
    """CK/backends/eager/rope.py:39-42: rotate pairs (i, i+D/2) in the table's
    dtype: out0 = f00*x0 + f01*x1, out1 = f10*x0 + f11*x1, then cast back."""
    t_ = x.reshape(*x.shape[:-1], 2, -1).movedim(-2, -1).unsqueeze(-2).to(freqs_cis.dtype)
    t_out = freqs_cis[..., 0] * t_[..., 0] + freqs_cis[..., 1] * t_[..., 1]
    return t_out.movedim(-1, -2).reshape(*x.shape).type_as(x)


def rms_rope_split_half1(x: torch.Tensor, freqs_cis: torch.Tensor, weight: torch.Tensor,
                         eps: float = 1e-6, rot_dim: int = 0) -> torch.Tensor:
    """CK/backends/eager/rope.py:67-92 (split_half=True): per-head
    F.rms_norm with weight, rotate the first rot_dim dims, tail norm-only."""
    x_norm = F.rms_norm(x, (x.shape[-1],), weight=weight, eps=eps)
    if rot_dim and rot_dim != x.shape[-1]:
        rotated = apply_rope_split_half1(x_norm[..., :rot_dim], freqs_cis)
        return torch.cat((rotated, x_norm[..., rot_dim:]), dim=-1)
    return apply_rope_split_half1(x_norm, freqs_cis)


def apply_rope1(x: torch.Tensor, freqs_cis: torch.Tensor) -> torch.Tensor:
    """CK/backends/eager/rope.py:10-16: interleaved pairs (2i, 2i+1) in the
    table's dtype: out_r = f[r, 0] * x0, then addcmul_(f[r, 1], x1) (torch's
    CPU addcmul evaluates that as one fused multiply-add), cast back. The
    table is trimmed to x's sequence dim as the reference does
    (CK/_rope_utils.py:4-13)."""
    x_ = x.to(dtype=freqs_cis.dtype).reshape(*x.shape[:-1], -1, 1, 2)
    if x.ndim > 2 and freqs_cis.ndim > 2 and x.shape[2] != 1 and freqs_cis.shape[2] > x.shape[2]:
        freqs_cis = freqs_cis[:, :, : x.shape[2]]
    x_out = freqs_cis[..., 0] * x_[..., 0]
    x_out.addcmul_(freqs_cis[..., 1], x_[..., 1])
    return x_out.reshape(*x.shape).type_as(x)


def rms_rope1(x: torch.Tensor, freqs_cis: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
              rot_dim: int = 0) -> torch.Tensor:
    """CK/backends/eager/rope.py:67-101 (split_half=False): per-head
    F.rms_norm with weight, then the interleaved rotation of the first
    rot_dim dims (0 = all), the tail norm-only."""
    x_norm = F.rms_norm(x, (x.shape[-1],), weight=weight, eps=eps)
    if rot_dim and rot_dim != x.shape[-1]:
        return torch.cat((apply_rope1(x_norm[..., :rot_dim], freqs_cis), x_norm[..., rot_dim:]), dim=-1)
    return apply_rope1(x_norm, freqs_cis)


def qknorm_rope_angles(value: torch.Tensor, weight: torch.Tensor, angles: torch.Tensor, eps: float,
                       cos_sin: tuple | None = None) -> torch.Tensor:
    """The angle-table branch of H3's apply_qknorm_rope
    (h3serve/native_engine/model/layers.py:126-149) for one of q or k:
    F.rms_norm with the weight in the value dtype, then active * cos +
    cat(-second, first) * sin in the value dtype over the first rot =
    angles.shape[-1] dims, cos and sin of the first half of the angles cast to
    the value dtype. ``cos_sin`` replaces those two tables (for checking a
    device-computed table)."""
    value = F.rms_norm(value, (value.shape[-1],), weight=weight.to(dtype=value.dtype), eps=eps)
    rot = int(angles.shape[-1])
    half = rot // 2
    if cos_sin is None:
        cosine = torch.cos(angles[:, :half]).to(value.dtype)
        sine = torch.sin(angles[:, :half]).to(value.dtype)
    else:
        cosine, sine = (t.to(value.dtype) for t in cos_sin)
    cosine = torch.cat((cosine, cosine), dim=-1).unsqueeze(1)
    sine = torch.cat((sine, sine), dim=-1).unsqueeze(1)
    active, passthrough = value[..., :rot], value[..., rot:]
    first, second = active.chunk(2, dim=-1)
    perpendicular = torch.cat((-second, first), dim=-1)
    return torch.cat((active * cosine + perpendicular * sine, passthrough), dim=-1)


def norm_rope(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor,
              freqs_cis: torch.Tensor, head_dim: int = 128, eps: float = 1e-6) -> torch.Tensor:
    """The fused AdaLN-RMSNorm + 3D RoPE composite for one of Q or K:
    apply_rope_split_half(rms_adaln(x, scale, shift, eps), freqs) with the
    RMS over the full row and the rotation per head
    (CK/backends/eager/adaln.py:17-20 then CK/backends/eager/rope.py:39-42).
    x: [M, D] with D = heads*head_dim; freqs: [1, M, 1, head_dim/2, 2, 2]."""
    m, d = x.shape
    a = rms_adaln(x, scale, shift, eps)
    a4 = a.reshape(1, m, d // head_dim, head_dim)
    return apply_rope_split_half1(a4, freqs_cis).reshape(m, d)


def bf16_ulp_diff(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """|a-b| in units of bf16 ulp at b's magnitude (helper for tolerances)."""
    bf = b.float().abs().clamp(min=2.0 ** -126)
    ulp = torch.pow(2.0, torch.floor(torch.log2(bf)) - 7)
    return (a.float() - b.float()).abs() / ulp


__all__ = [name for name in dir() if not name.startswith("_") and name not in ("math", "torch", "F")]
