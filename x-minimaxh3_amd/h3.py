"""Drop-in adapters for the H3 engine's call sites of the hot path.

* ``mi355x_int8_kernel`` / ``mi355x_w4a8_kernel`` have the ``Int8Kernel`` and
  ``W4A8Kernel`` callable signatures the engine injects into every quantized
  linear (h3serve/native_engine/model/quantization.py:19-37, injected via
  assembly.py:166-228).
* ``rms_adaln(value, norm, shift, scale, segments)`` is the segmented
  RMSNorm + AdaLN of h3serve/native_engine/model/kernels.py:7586-7634 in one
  launch (row map per token instead of one launch per segment).
* ``apply_qknorm_rope(query, key, *, q_weight, k_weight, frequencies, eps)``
  is the table form of h3serve/native_engine/model/layers.py:72-100.
* ``segment_row_map`` follows h3serve/native_engine/model/fused_mlp.py:34-55.
* ``fused_down_gated_residual`` has the signature of
  h3serve/native_engine/model/fused_mlp.py:157-165 (SwiGLU + ConvRot
  quantizer, fc2 GEMM with the gated residual update in its epilogue), and
  ``gated_swiglu_mlp_`` is the int8 route of ``try_fused_gated_mlp``
  (fused_mlp.py:269-426) over token chunks.
* ``W4A8QuantSpec`` / ``load_w4a8_linear`` read the H3 W4A8 checkpoint layout
  (safetensors keys ``weight``, ``weight_s_rel``, ``weight_s_channel``,
  ``weight_codebook``, ``weight_correction``, ``bias``; quantization.py:153-187,
  416-516, assembly.py:166-228) into a callable linear on the GPU path.
"""

from __future__ import annotations

from collections.abc import Mapping
from dataclasses import dataclass

import torch

from . import backend, ops

_ROW_MAPS: dict[tuple, torch.Tensor] = {}


def segment_row_map(length: int, segments, device, n_rows: int | None = None) -> torch.Tensor:
    """int32 [length]: the modulation row of each token; segments must be an
    ordered partition ``(start, stop, row)`` of [0, length). With ``n_rows``
    (the modulation table's row count) each row is resolved as the
    reference's ``scale[row]`` indexing resolves it: a negative row counts
    from the end, a row outside [-n_rows, n_rows) raises IndexError."""
    norm = []
    for a, b, r in segments:
        r = int(r)
        if n_rows is not None:
            if not -n_rows <= r < n_rows:
                raise IndexError(f"index {r} is out of bounds for dimension 0 with size {n_rows}")
            r = r + n_rows if r < 0 else r
        norm.append((int(a), int(b), r))
    norm = tuple(norm)
    dev = torch.device(device)
    key = (dev.type, dev.index, int(length), norm)
    hit = _ROW_MAPS.get(key)
    if hit is not None:
        return hit
    host = torch.empty(length, dtype=torch.int32)
    prev = 0
    for a, b, r in norm:
        if a != prev or b <= a:
            raise ValueError("modulation segments must be an ordered partition")
        host[a:b] = r
        prev = b
    if prev != length:
        raise ValueError("modulation segments do not cover the packed sequence")
    out = host.to(dev)
    _ROW_MAPS[key] = out
    return out


def rms_adaln(value: torch.Tensor, norm, shift: torch.Tensor, scale: torch.Tensor, segments,
              *, eps: float | None = None) -> torch.Tensor:
    """RMSNorm(value) then per-segment ``* (1 + scale[row]) + shift[row]``.
    ``norm`` is an RMSNorm module (``.weight``, ``.eps``) or a weight tensor
    (then ``eps`` is required)."""
    weight = getattr(norm, "weight", norm)
    if eps is None:
        eps = getattr(norm, "eps", None)
        if eps is None:
            raise ValueError("eps is required when norm is a tensor")
    if value.ndim != 2:
        raise ValueError("value must be [tokens, width]")
    if scale.ndim != 2 or shift.shape != scale.shape:
        raise ValueError("scale and shift must be [rows, width] tables of one shape")
    row_map = segment_row_map(value.shape[0], segments, value.device, n_rows=scale.shape[0])
    return backend.rms_adaln_rows(value, weight, scale.to(value.dtype), shift.to(value.dtype), row_map, eps)


def angle_rotation_table(angles: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """[S, rot] split-half angles -> the packed [1, S, 1, rot/2, 2, 2] table
    (cos, -sin, sin, cos) of their first half in ``dtype``, computed where
    the angles are (H3/layers.py:61-69)."""
    half = angles.shape[-1] // 2
    active = angles[:, :half]
    c, s = torch.cos(active), torch.sin(active)
    return torch.stack((c, -s, s, c), dim=-1).reshape(1, angles.shape[0], 1, half, 2, 2).to(dtype)


def apply_qknorm_rope(query: torch.Tensor, key: torch.Tensor, *, q_weight: torch.Tensor, k_weight: torch.Tensor,
                      frequencies: torch.Tensor, eps: float):
    """Per-head RMSNorm then split-half partial RoPE (H3/layers.py:72-149).

    The packed [1, S, 1, rot/2, 2, 2] table form runs in place, as the
    reference's GPU branch does. The angle form ([S, rot] angles) returns new
    tensors, as the reference does: its rotation active * cos + (-second,
    first) * sin in the value dtype, with cos and sin of the first half of
    the angles rounded to that dtype, is the table form with the table
    (cos, -sin, sin, cos) in the value dtype, so it runs the same kernel on
    ``angle_rotation_table(angles, query.dtype)``."""
    if frequencies.ndim != 6:
        if frequencies.ndim != 2:
            raise ValueError(f"frequencies must be a packed 6-D table or [S, rot] angles, got {tuple(frequencies.shape)}")
        rot = int(frequencies.shape[-1])
        table = angle_rotation_table(frequencies.to(query.device), query.dtype)
        q_out, k_out = ops.rms_rope_split_half(query.unsqueeze(0), key.unsqueeze(0), table,
                                               q_weight.to(device=query.device, dtype=query.dtype),
                                               k_weight.to(device=key.device, dtype=key.dtype), epsilon=eps,
                                               rot_dim=rot)
        return q_out[0], k_out[0]
    rot = int(frequencies.shape[-3]) * 2
    q4, k4 = query.unsqueeze(0), key.unsqueeze(0)
    ops.rms_rope_split_half_(q4, k4, frequencies, q_weight.to(device=query.device, dtype=query.dtype),
                             k_weight.to(device=key.device, dtype=key.dtype), epsilon=eps, rot_dim=rot)
    return q4[0], k4[0]


def mi355x_int8_kernel(value: torch.Tensor, qweight: torch.Tensor, scale: torch.Tensor,
                       bias: torch.Tensor | None, convrot_group_size: int) -> torch.Tensor:
    """``Int8Kernel``: int8_linear(value, qweight, scale, bias, value.dtype,
    convrot=bool(convrot_group_size), ...)."""
    return ops.int8_linear(value, qweight, scale, bias, value.dtype, convrot=bool(convrot_group_size),
                           convrot_groupsize=convrot_group_size or 256)


def mi355x_w4a8_kernel(value, qdata, s_rel, s_channel, codebook, correction, bias, group_size,
                       convrot_group_size, output_dtype):
    """``W4A8Kernel``: w4a8_int8_linear with the engine's arguments (a zero
    convrot group size selects the unrotated form)."""
    return ops.w4a8_int8_linear(value, qdata, s_rel, s_channel, codebook=codebook, correction=correction,
                                bias=bias, group_size=group_size, convrot_groupsize=convrot_group_size or 256,
                                out_dtype=output_dtype, convrot=bool(convrot_group_size))


def fused_down_gated_residual(hidden: torch.Tensor, residual: torch.Tensor, gate: torch.Tensor,
                              gate_rows: torch.Tensor, qweight: torch.Tensor, weight_scale: torch.Tensor,
                              bias: torch.Tensor | None) -> None:
    """residual += fc2(swiglu(hidden)) * gate[gate_rows], in place: ``hidden``
    is the raw fc1 output ``[rows, 2 * ffn]`` ([gate | up]), ``qweight`` the
    ConvRot-rotated int8 fc2 weight, ``gate_rows`` the int32 segment-row map of
    the rows (fused_mlp.py:157-222)."""
    backend.int8_linear_gated_residual_(hidden.reshape(-1, hidden.shape[-1]), qweight, weight_scale, bias,
                                        residual, gate, gate_rows, convrot=True, convrot_groupsize=256,
                                        input_act="swiglu")


def gated_swiglu_mlp_(residual: torch.Tensor, hidden: torch.Tensor, fc1_qweight: torch.Tensor,
                      fc1_scale: torch.Tensor, fc1_bias: torch.Tensor | None, fc2_qweight: torch.Tensor,
                      fc2_scale: torch.Tensor, fc2_bias: torch.Tensor | None, gate: torch.Tensor, segments,
                      *, chunk_tokens: int = 8192) -> torch.Tensor:
    """The int8 route of ``try_fused_gated_mlp`` (fused_mlp.py:340-426): per
    chunk of tokens, raw = fc1(hidden) (ConvRot int8 linear), then the fused
    SwiGLU + ConvRot quantizer and fc2 with the gated residual update. Both
    weights are the checkpoint's rotated int8 ones. Updates ``residual`` in
    place and returns it."""
    if chunk_tokens <= 0:
        raise ValueError("MLP chunk_tokens must be positive")
    if hidden.ndim != 2:
        raise ValueError("hidden must be [tokens, width]")
    rows = segment_row_map(hidden.shape[0], segments, hidden.device, n_rows=gate.shape[0])
    for start in range(0, hidden.shape[0], chunk_tokens):
        stop = min(start + chunk_tokens, hidden.shape[0])
        raw = ops.int8_linear(hidden[start:stop], fc1_qweight, fc1_scale, fc1_bias, hidden.dtype, convrot=True,
                              convrot_groupsize=256)
        backend.int8_linear_gated_residual_(raw, fc2_qweight, fc2_scale, fc2_bias, residual[start:stop], gate,
                                            rows[start:stop], convrot=True, convrot_groupsize=256,
                                            input_act="swiglu")
    return residual


@dataclass(frozen=True)
class W4A8QuantSpec:
    """The layout recorded by the H3 mixed W4A8 checkpoints
    (h3serve/native_engine/model/quantization.py:153-187)."""

    format: str = "asym_w4a8_int8"
    group_size: int = 16
    convrot: bool = True
    convrot_groupsize: int = 256

    @classmethod
    def from_mapping(cls, data: Mapping[str, object]) -> "W4A8QuantSpec":
        return cls(format=str(data.get("format", "")), group_size=int(data.get("group_size", 16)),
                   convrot=bool(data.get("convrot", True)),
                   convrot_groupsize=int(data.get("convrot_groupsize", 256)))

    def validate_supported(self) -> None:
        if self.format != "asym_w4a8_int8":
            raise ValueError(f"native core currently supports asym_w4a8_int8, got {self.format!r}")
        if self.group_size < 4 or (16 % self.group_size != 0 and self.group_size % 16 != 0):
            raise ValueError("W4A8 group size must be >=4 and divide 16 or be a multiple of 16")
        if not self.convrot:
            raise ValueError("the H3 W4A8 checkpoint requires ConvRot")
        size = self.convrot_groupsize
        if size < 4 or size & (size - 1) or size.bit_length() % 2 == 0:
            raise ValueError("ConvRot group size must be a power of four")


class W4A8Linear:
    """A W4A8 linear in the H3 checkpoint layout, computed by
    ``w4a8_int8_linear`` (ConvRot row quantizer, codebook / fp8-scale decode
    to the int8 grid, int8 GEMM, asymmetric correction)."""

    def __init__(self, qdata, s_rel, s_channel, *, codebook=None, correction=None, bias=None,
                 spec: W4A8QuantSpec = W4A8QuantSpec(), output_dtype: torch.dtype | None = None):
        spec.validate_supported()
        if qdata.ndim != 2 or qdata.dtype != torch.int8:
            raise ValueError("packed W4 weight must be a rank-two int8 tensor")
        out_features = qdata.shape[0]
        if bias is not None and bias.numel() != out_features:
            raise ValueError("bias does not match W4A8 output rows")
        backend.validate_w4a8_operands(qdata, s_rel, s_channel, codebook, correction, spec.group_size,
                                       spec.convrot_groupsize)
        self.qdata, self.s_rel, self.s_channel = qdata, s_rel, s_channel
        self.codebook, self.correction, self.bias = codebook, correction, bias
        self.spec = spec
        self.output_dtype = output_dtype

    @property
    def in_features(self) -> int:
        return int(self.qdata.shape[1]) * 2

    @property
    def out_features(self) -> int:
        return int(self.qdata.shape[0])

    def __call__(self, value: torch.Tensor) -> torch.Tensor:
        out_dtype = self.output_dtype or value.dtype
        return backend.w4a8_int8_linear(value, self.qdata, self.s_rel, self.s_channel, codebook=self.codebook,
                                        correction=self.correction, bias=self.bias,
                                        group_size=self.spec.group_size,
                                        convrot_groupsize=self.spec.convrot_groupsize, out_dtype=out_dtype,
                                        convrot=True)


def load_w4a8_linear(tensors: Mapping[str, torch.Tensor], prefix: str, *, spec: Mapping | None = None,
                     device: torch.device | str | None = None,
                     output_dtype: torch.dtype | None = None) -> W4A8Linear:
    """Build a ``W4A8Linear`` from checkpoint tensors named as H3 stores them
    (assembly.py:186-228). ``tensors`` is any mapping (a safetensors
    ``safe_open`` view wrapped in a dict, a state dict); ``spec`` the
    file-level quantization metadata (the H3 layout when absent)."""
    required = (f"{prefix}.weight", f"{prefix}.weight_s_rel", f"{prefix}.weight_s_channel")
    missing = [k for k in required if k not in tensors]
    if missing:
        raise KeyError(f"quantized layer {prefix!r} is not W4A8: missing {missing}")
    qspec = W4A8QuantSpec.from_mapping(spec) if spec is not None else W4A8QuantSpec()

    def get(key):
        t = tensors.get(f"{prefix}.{key}")
        return None if t is None else (t.to(device) if device is not None else t)

    return W4A8Linear(get("weight"), get("weight_s_rel"), get("weight_s_channel"), codebook=get("weight_codebook"),
                      correction=get("weight_correction"), bias=get("bias"), spec=qspec,
                      output_dtype=output_dtype)
