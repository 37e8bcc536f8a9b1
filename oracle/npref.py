"""Independent numpy / exact-arithmetic restatements of the integer parts.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

These are written from the closed-form rules, not from ``cpu_ref``'s torch
calls, and are what pins ``cpu_ref`` (and through it the GPU path):

* bf16 rounding is done on the fp32 bit pattern (round to nearest, ties to
  even), never through a torch dtype cast;
* ``quantize_row_exact`` derives every rounding from exact rationals
  (``fractions.Fraction``), so a wrong division (x * (1/s)), a wrong tie rule
  or a wrong clamp range in the faster restatements shows up on small rows;
* the int GEMM is an int64 brute force;
* the W4 decode is a pure-Python loop over nibbles for tiny inputs.

Reference rules restated (``CK/`` = backends/turbo/vendor/comfy_kitchen/):
row quantizer CK/backends/eager/quantization.py:815-826,857-875;
W4 decode CK/backends/eager/w4a8_int8.py:344-363;
W4 weight generator CK/backends/eager/w4a8_int8.py:169-173,188-191,200-202.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np


# ---------------------------------------------------------------------------
# bf16 <-> fp32 on bit patterns
# ---------------------------------------------------------------------------

def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round fp32 to bf16 (nearest, ties to even); returns uint16 bits."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest bf16 value, returned as fp32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# ---------------------------------------------------------------------------
# row quantizer (bf16 input)
# ---------------------------------------------------------------------------

def quantize_rows_bf16(x_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """x_bits: uint16 [M, K] bf16 bit patterns. Returns (int8 [M,K], fp32 [M])."""
    x = bf16_bits_to_f32(x_bits)
    amax = np.abs(x).max(axis=-1) if x.shape[-1] else np.zeros(x.shape[:-1], np.float32)
    scale = np.maximum(amax.astype(np.float32) / np.float32(127.0), np.float32(1e-30)).astype(np.float32)
    sb = round_bf16(scale)
    sb = np.where(sb == 0, np.float32(np.finfo(np.float32).tiny), sb).astype(np.float32)
    v = (x / sb[..., None]).astype(np.float32)          # fp32 correctly rounded division
    vb = round_bf16(v)
    q = np.clip(np.rint(vb), -128, 127).astype(np.int8)  # rint: ties to even
    return q, scale


def _round_fraction_to_float(fr: Fraction, mant_bits: int, min_exp: int) -> Fraction:
    """Round a rational to the nearest binary float with ``mant_bits``
    significant bits (ties to even); min_exp bounds the exponent of the last
    place (subnormal range). Returns the rounded value as a Fraction."""
    if fr == 0:
        return Fraction(0)
    sign = -1 if fr < 0 else 1
    a = abs(fr)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    ulp_exp = max(e - (mant_bits - 1), min_exp)
    ulp = Fraction(2) ** ulp_exp
    n = a / ulp
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return sign * fl * ulp


def to_f32_exact(fr: Fraction) -> Fraction:
    return _round_fraction_to_float(fr, 24, -149)


def to_bf16_exact(fr: Fraction) -> Fraction:
    return _round_fraction_to_float(fr, 8, -133)


def quantize_row_exact(row_bits: list[int]) -> tuple[list[int], float]:
    """Exact-rational restatement for one bf16 row (pure Python, small rows)."""
    vals = [Fraction(float(bf16_bits_to_f32(np.array([b], np.uint16))[0])) for b in row_bits]
    amax = max((abs(v) for v in vals), default=Fraction(0))
    scale = to_f32_exact(amax / 127)
    floor = Fraction(float(np.float32(1e-30)))
    if scale < floor:
        scale = floor
    sb = to_bf16_exact(scale)
    out = []
    for v in vals:
        qv = to_bf16_exact(to_f32_exact(v / sb))
        fl = qv.numerator // qv.denominator
        rem = qv - fl
        r = fl + (1 if (rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1)) else 0)
        out.append(int(min(127, max(-128, r))))
    return out, float(scale)


# ---------------------------------------------------------------------------
# integer GEMM and the fp32 dequant epilogue
# ---------------------------------------------------------------------------

def int_mm(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """int64 brute force of a[M,K] @ w[N,K]^T, returned as int32."""
    acc = a.astype(np.int64) @ w.astype(np.int64).T
    assert np.abs(acc).max(initial=0) < 2 ** 31
    return acc.astype(np.int32)


def dequant_bf16_bits(acc: np.ndarray, sx: np.ndarray, sw: np.ndarray) -> np.ndarray:
    """bf16(float(acc) * (sx[m] * sw[n])) with fp32 products; uint16 bits."""
    scl = (sx.astype(np.float32).reshape(-1, 1) * sw.astype(np.float32).reshape(1, -1)).astype(np.float32)
    return f32_to_bf16_bits((acc.astype(np.float32) * scl).astype(np.float32))


# ---------------------------------------------------------------------------
# W4 (int4, grouped) weights
# ---------------------------------------------------------------------------

def w4_decode(qdata: np.ndarray, s_rel: np.ndarray, group_size: int) -> np.ndarray:
    """Vectorised nibble decode: low nibble = even k, high = odd k;
    int8 = clip(rint((code-8) * s_rel[n, k // G]), -127, 127)."""
    b = qdata.view(np.uint8).astype(np.int32)
    n, kh = b.shape
    codes = np.empty((n, kh * 2), np.int32)
    codes[:, 0::2] = b & 0xF
    codes[:, 1::2] = (b >> 4) & 0xF
    s = np.repeat(s_rel.astype(np.float32), group_size, axis=1)
    lv = ((codes - 8).astype(np.float32) * s).astype(np.float32)
    return np.clip(np.rint(lv), -127, 127).astype(np.int8)


def w4_decode_loops(qdata: np.ndarray, s_rel: np.ndarray, group_size: int) -> list[list[int]]:
    """Pure-Python loop form of the same decode, for tiny inputs."""
    out = []
    for n in range(qdata.shape[0]):
        row = []
        for j in range(qdata.shape[1]):
            byte = int(qdata[n, j]) & 0xFF
            for code in (byte & 0xF, byte >> 4):
                k = len(row)
                s = Fraction(float(np.float32(s_rel[n, k // group_size])))
                prod = to_f32_exact((code - 8) * s)
                fl = prod.numerator // prod.denominator
                rem = prod - fl
                r = fl + (1 if (rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1)) else 0)
                row.append(int(min(127, max(-127, r))))
        out.append(row)
    return out


def w4_quantize(w: np.ndarray, group_size: int):
    """numpy restatement of the symmetric uniform W4 generator."""
    n, k = w.shape
    g = w.astype(np.float32).reshape(n, k // group_size, group_size)
    gs = np.maximum(np.abs(g).max(-1, keepdims=True) / np.float32(7.0), np.float32(1e-8)).astype(np.float32)
    signed = np.clip(np.rint((g / gs).astype(np.float32)), -8, 7).astype(np.int32)
    shifted = (signed.astype(np.float32) * gs).astype(np.float32)
    sch = np.maximum(np.abs(shifted).max(axis=(1, 2)) / np.float32(127.0), np.float32(1e-8)).astype(np.float32)
    s_rel = (gs[..., 0] / sch[:, None]).astype(np.float32)
    u = (signed + 8).reshape(n, k)
    packed = ((u[:, 0::2] & 0xF) | ((u[:, 1::2] & 0xF) << 4)).astype(np.uint8).view(np.int8)
    return packed, s_rel, sch


# ---------------------------------------------------------------------------
# the reduction order of the reference's rms_norm (torch CPU sum)
# ---------------------------------------------------------------------------

def torch_cpu_sum_order(x: np.ndarray) -> np.float32:
    """fp32 sum of a contiguous row in the order torch's CPU reduction uses for
    it on this image: 8-lane vectors read 4 at a time into 4 accumulator rows
    (32 chains, chain L over positions 32*i + L), each row accumulating in
    chunks of 16 that feed a 4-level cascade (level 2 every 256 steps, level 3
    every 4096), leftover vectors added to row 0, rows combined
    ((r0+r1)+r2)+r3, then a scalar tail and the 8 lanes left to right."""
    x = np.asarray(x, np.float32)
    n = x.shape[0]
    nvec = n // 8
    vecs = x[: nvec * 8].reshape(nvec, 8)
    size = nvec // 4
    rows = vecs[: size * 4].reshape(size, 4, 8)
    acc = np.zeros((4, 4, 8), np.float32)
    i = 0
    while i + 16 <= size:
        for _ in range(16):
            acc[0] = (acc[0] + rows[i]).astype(np.float32)
            i += 1
        for j in range(1, 4):
            acc[j] = (acc[j] + acc[j - 1]).astype(np.float32)
            acc[j - 1] = 0
            if (i & (15 << (4 * j))) != 0:
                break
    while i < size:
        acc[0] = (acc[0] + rows[i]).astype(np.float32)
        i += 1
    for j in range(1, 4):
        acc[0] = (acc[0] + acc[j]).astype(np.float32)
    part = acc[0]
    for r in range(size * 4, nvec):
        part[0] = (part[0] + vecs[r]).astype(np.float32)
    p = part[0]
    for k in range(1, 4):
        p = (p + part[k]).astype(np.float32)
    fin = np.float32(0)
    for t in x[nvec * 8:]:
        fin = np.float32(fin + t)
    for v in range(8):
        fin = np.float32(fin + p[v])
    return fin
