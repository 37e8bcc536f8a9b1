"""The bf16 quantizer's reciprocal form against the exact division (CPU).

The HIP quantizer computes the code of a bf16 value x under the bf16 row
scale sT as rint(bf16(fl32(x * fl32(1/sT)))), where the reference computes
rint(bf16(fl32(x / sT))) (CK/backends/eager/quantization.py:857-875). The two
agree because x/sT is never near a bf16 rounding midpoint when x and sT are
both bf16 (see the kernel's comment). This checks the identity exhaustively
over every finite bf16 x for thousands of scales formed as the quantizer forms
them, including the zero-row floor and powers of two."""

import numpy as np
import pytest


def bf16_round(f32: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 (nearest even) -> fp32, on bit patterns."""
    u = np.ascontiguousarray(f32, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def codes(v: np.ndarray) -> np.ndarray:
    return np.clip(np.rint(v), -128, 127).astype(np.int32)


def all_bf16() -> np.ndarray:
    b = (np.arange(1 << 16, dtype=np.uint32) << 16).view(np.float32)
    return b[np.isfinite(b)]


def row_scales(seed: int, n: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    amax = np.exp(rng.uniform(np.log(1e-30), np.log(3e38), n)).astype(np.float32)
    amax = np.concatenate([amax, [0.0, 1.0, 127.0, 254.0, 3.0e38]]).astype(np.float32)
    s = np.maximum(amax / np.float32(127.0), np.float32(1e-30)).astype(np.float32)
    sT = bf16_round(s)
    sT[sT == 0] = np.float32(2.0 ** -126)
    return np.unique(sT)


@pytest.mark.parametrize("seed", [0, 1])
def test_reciprocal_equals_division_bf16(seed):
    x = all_bf16()
    for st in row_scales(seed, 1500):
        exact = bf16_round((x / st).astype(np.float32))
        prod = bf16_round((x * (np.float32(1.0) / st)).astype(np.float32))
        ok = np.isfinite(exact)
        assert np.array_equal(exact[ok], prod[ok]), (st, x[ok][exact[ok] != prod[ok]][:5])
        assert np.array_equal(codes(exact[ok]), codes(prod[ok]))


def test_reciprocal_differs_for_fp32_inputs():
    """The identity needs x in bf16: for fp32 inputs (24 significant bits) the
    product does round differently from the division somewhere, so the check
    above is not vacuous."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal(1 << 20).astype(np.float32) * np.float32(40.0)
    diffs = 0
    for st in bf16_round(np.array([0.3, 0.7, 1.1, 2.9, 0.0131], dtype=np.float32)):
        exact = bf16_round((x / st).astype(np.float32))
        prod = bf16_round((x * (np.float32(1.0) / st)).astype(np.float32))
        diffs += int((exact != prod).sum())
    assert diffs > 0
