"""Public operator API with the reference's names, signatures and defaults.

Each public function enters a ``torch.library`` custom op in the
``x_minimaxh3_amd`` namespace (with a fake implementation, so the ops trace
under ``torch.compile``), which dispatches through the capability registry
to the ``"mi355x"`` backend. Signatures follow CK/__init__.py (CK =
backends/turbo/vendor/comfy_kitchen):

  quantize_int8_rowwise   CK/__init__.py:702-709
  int8_linear             CK/__init__.py:722-764  (custom op schema of
                          CK/backends/eager/quantization.py:1205-1235)
  w4a8_int8_linear        CK/tensor/w4a8_int8.py:89-115
  rms_adaln               CK/__init__.py:130-150
  apply_rope_split_half(_), apply_rope_split_half1(_)   CK/__init__.py:629-690
  rms_rope_split_half(_), rms_rope_split_half1(_)        CK/__init__.py:549-603
  apply_rope(_), apply_rope1(_), rms_rope(_), rms_rope1(_) (interleaved pairs)
                          CK/backends/eager/rope.py:10-36,95-166

plus the fused entries of the hot path: ``norm_rope``, ``w8a8_mlp``,
``w4a8_mlp``.
"""

from __future__ import annotations

import torch

from . import backend as _backend  # noqa: F401  (registers "mi355x")
from .registry import registry

DTYPE_CODE_TO_DTYPE = {0: torch.float32, 1: torch.float16, 2: torch.bfloat16}
DTYPE_TO_CODE = {v: k for k, v in DTYPE_CODE_TO_DTYPE.items()}


def _impl(name: str, kwargs: dict):
    return registry.get_implementation(name, kwargs=kwargs)


# --------------------------------------------------------------------------- custom ops

@torch.library.custom_op("x_minimaxh3_amd::quantize_int8_rowwise", mutates_args=())
def _op_quantize_int8_rowwise(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    kw = {"x": x, "stochastic_rounding": 0}
    return _impl("quantize_int8_rowwise", kw)(**kw)


@_op_quantize_int8_rowwise.register_fake
def _(x):
    return (torch.empty_like(x, dtype=torch.int8),
            torch.empty(*x.shape[:-1], 1, dtype=torch.float32, device=x.device))


@torch.library.custom_op("x_minimaxh3_amd::int8_linear", mutates_args=())
def _op_int8_linear(x: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
                    bias: torch.Tensor | None, output_dtype_code: int, convrot: bool = False,
                    convrot_groupsize: int = 256, input_act: str | None = None) -> torch.Tensor:
    kw = {"x": x, "weight": weight, "weight_scale": weight_scale, "bias": bias,
          "out_dtype": DTYPE_CODE_TO_DTYPE[output_dtype_code], "convrot": convrot,
          "convrot_groupsize": convrot_groupsize, "input_act": input_act}
    return _impl("int8_linear", kw)(**kw)


@_op_int8_linear.register_fake
def _(x, weight, weight_scale, bias, output_dtype_code, convrot=False, convrot_groupsize=256, input_act=None):
    return torch.empty(*x.shape[:-1], weight.shape[0], dtype=DTYPE_CODE_TO_DTYPE[output_dtype_code],
                       device=x.device)


@torch.library.custom_op("x_minimaxh3_amd::w4a8_int8_linear", mutates_args=())
def _op_w4a8_int8_linear(x: torch.Tensor, qdata: torch.Tensor, s_rel: torch.Tensor, s_channel: torch.Tensor,
                         codebook: torch.Tensor | None, correction: torch.Tensor | None,
                         bias: torch.Tensor | None, group_size: int, convrot_groupsize: int,
                         output_dtype_code: int, convrot: bool) -> torch.Tensor:
    kw = {"x": x, "qdata": qdata, "s_rel": s_rel, "s_channel": s_channel, "codebook": codebook,
          "correction": correction, "bias": bias, "group_size": group_size,
          "convrot_groupsize": convrot_groupsize, "out_dtype": DTYPE_CODE_TO_DTYPE[output_dtype_code],
          "convrot": convrot}
    return _impl("w4a8_int8_linear", kw)(**kw)


@_op_w4a8_int8_linear.register_fake
def _(x, qdata, s_rel, s_channel, codebook, correction, bias, group_size, convrot_groupsize,
      output_dtype_code, convrot):
    return torch.empty(*x.shape[:-1], qdata.shape[0], dtype=DTYPE_CODE_TO_DTYPE[output_dtype_code],
                       device=x.device)


@torch.library.custom_op("x_minimaxh3_amd::rms_adaln", mutates_args=())
def _op_rms_adaln(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor, eps: float) -> torch.Tensor:
    kw = {"x": x, "scale": scale, "shift": shift, "eps": eps}
    return _impl("rms_adaln", kw)(**kw)


@_op_rms_adaln.register_fake
def _(x, scale, shift, eps):
    return torch.empty(x.shape, dtype=torch.promote_types(x.dtype, scale.dtype), device=x.device)


@torch.library.custom_op("x_minimaxh3_amd::norm_rope", mutates_args=())
def _op_norm_rope(q: torch.Tensor, k: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor,
                  freqs_cis: torch.Tensor, eps: float, head_dim: int) -> tuple[torch.Tensor, torch.Tensor]:
    kw = {"q": q, "k": k, "scale": scale, "shift": shift, "freqs_cis": freqs_cis, "eps": eps,
          "head_dim": head_dim}
    return _impl("norm_rope", kw)(**kw)


@_op_norm_rope.register_fake
def _(q, k, scale, shift, freqs_cis, eps, head_dim):
    return torch.empty_like(q), torch.empty_like(k)


@torch.library.custom_op("x_minimaxh3_amd::w8a8_mlp", mutates_args=())
def _op_w8a8_mlp(x: torch.Tensor, w1: torch.Tensor, s1: torch.Tensor, w2: torch.Tensor,
                 s2: torch.Tensor) -> torch.Tensor:
    kw = {"x": x, "w1": w1, "s1": s1, "w2": w2, "s2": s2}
    return _impl("w8a8_mlp", kw)(**kw)


@_op_w8a8_mlp.register_fake
def _(x, w1, s1, w2, s2):
    return torch.empty(*x.shape[:-1], w2.shape[0], dtype=torch.bfloat16, device=x.device)


@torch.library.custom_op("x_minimaxh3_amd::w4a8_mlp", mutates_args=())
def _op_w4a8_mlp(x: torch.Tensor, w1_packed: torch.Tensor, w1_srel: torch.Tensor, w1_schannel: torch.Tensor,
                 w2_packed: torch.Tensor, w2_srel: torch.Tensor, w2_schannel: torch.Tensor,
                 group_size: int) -> torch.Tensor:
    kw = {"x": x, "w1_packed": w1_packed, "w1_srel": w1_srel, "w1_schannel": w1_schannel,
          "w2_packed": w2_packed, "w2_srel": w2_srel, "w2_schannel": w2_schannel, "group_size": group_size}
    return _impl("w4a8_mlp", kw)(**kw)


@_op_w4a8_mlp.register_fake
def _(x, w1_packed, w1_srel, w1_schannel, w2_packed, w2_srel, w2_schannel, group_size):
    return torch.empty(*x.shape[:-1], w2_packed.shape[0], dtype=torch.bfloat16, device=x.device)


@torch.library.custom_op("x_minimaxh3_amd::rms_rope_split_half_", mutates_args=("q", "k"))
def _op_rms_rope_split_half_(q: torch.Tensor, k: torch.Tensor, freqs_cis: torch.Tensor, q_scale: torch.Tensor,
                             k_scale: torch.Tensor | None, epsilon: float, rot_dim: int) -> None:
    kw = {"q": q, "k": k, "freqs_cis": freqs_cis, "q_scale": q_scale, "k_scale": k_scale,
          "epsilon": epsilon, "rot_dim": rot_dim}
    _impl("rms_rope_split_half_", kw)(**kw)


@_op_rms_rope_split_half_.register_fake
def _(q, k, freqs_cis, q_scale, k_scale, epsilon, rot_dim):
    return None


@torch.library.custom_op("x_minimaxh3_amd::apply_rope_split_half_", mutates_args=("xq", "xk"))
def _op_apply_rope_split_half_(xq: torch.Tensor, xk: torch.Tensor, freqs_cis: torch.Tensor) -> None:
    kw = {"xq": xq, "xk": xk, "freqs_cis": freqs_cis}
    _impl("apply_rope_split_half_", kw)(**kw)


@_op_apply_rope_split_half_.register_fake
def _(xq, xk, freqs_cis):
    return None


# --------------------------------------------------------------------------- public API

def quantize_int8_rowwise(x: torch.Tensor, stochastic_rounding: int | None = 0):
    """Quantize tensor to INT8 with per-row scales -> (int8 like x, fp32 [..., 1])."""
    if stochastic_rounding:
        kw = {"x": x, "stochastic_rounding": stochastic_rounding}
        return _impl("quantize_int8_rowwise", kw)(**kw)
    return torch.ops.x_minimaxh3_amd.quantize_int8_rowwise(x)


def int8_linear(x: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
                bias: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
                convrot: bool = False, convrot_groupsize: int = 256,
                input_act: str | None = None) -> torch.Tensor:
    """INT8 linear layer with dynamic per-token activation quantization."""
    if out_dtype is None:
        out_dtype = torch.bfloat16
    return torch.ops.x_minimaxh3_amd.int8_linear(x, weight, weight_scale, bias, DTYPE_TO_CODE[out_dtype],
                                                 convrot, convrot_groupsize, input_act)


def w4a8_int8_linear(x: torch.Tensor, qdata: torch.Tensor, s_rel: torch.Tensor, s_channel: torch.Tensor,
                     codebook: torch.Tensor | None = None, correction: torch.Tensor | None = None,
                     bias: torch.Tensor | None = None, group_size: int = 16, convrot_groupsize: int = 256,
                     out_dtype: torch.dtype = torch.bfloat16, convrot: bool = True) -> torch.Tensor:
    """``x @ W.T + bias`` with grouped int4 weights decoded to the int8 grid
    (CK/tensor/w4a8_int8.py:89-115). ``convrot`` is an extra keyword:
    True (the default, as the reference always rotates) quantizes the
    activations through the fused ConvRot row quantizer (groups of
    ``convrot_groupsize`` = 256) against the checkpoint's offline-rotated
    weights; False selects the unrotated form of the GELU MLP workloads. A
    ``correction`` adds the asymmetric term of the H3 checkpoints (group sums
    of the activation codes times the correction, as the reference's GPU
    dispatcher computes it)."""
    return torch.ops.x_minimaxh3_amd.w4a8_int8_linear(x, qdata, s_rel, s_channel, codebook, correction, bias,
                                                      group_size, convrot_groupsize, DTYPE_TO_CODE[out_dtype],
                                                      convrot)


def rms_adaln(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """rmsnorm(x) * (1 + scale) + shift."""
    return torch.ops.x_minimaxh3_amd.rms_adaln(x, scale, shift, eps)


def apply_rope_split_half(xq: torch.Tensor, xk: torch.Tensor, freqs_cis: torch.Tensor):
    kw = {"xq": xq, "xk": xk, "freqs_cis": freqs_cis}
    return _impl("apply_rope_split_half", kw)(**kw)


def apply_rope_split_half_(xq: torch.Tensor, xk: torch.Tensor, freqs_cis: torch.Tensor):
    torch.ops.x_minimaxh3_amd.apply_rope_split_half_(xq, xk, freqs_cis)
    return xq, xk


def apply_rope_split_half1(x: torch.Tensor, freqs_cis: torch.Tensor) -> torch.Tensor:
    kw = {"x": x, "freqs_cis": freqs_cis}
    return _impl("apply_rope_split_half1", kw)(**kw)


def apply_rope_split_half1_(x: torch.Tensor, freqs_cis: torch.Tensor) -> torch.Tensor:
    kw = {"x": x, "freqs_cis": freqs_cis}
    return _impl("apply_rope_split_half1_", kw)(**kw)


def rms_rope_split_half(q, k, freqs_cis, q_scale, k_scale=None, epsilon: float = 1e-6, rot_dim: int = 0):
    kw = {"q": q, "k": k, "freqs_cis": freqs_cis, "q_scale": q_scale, "k_scale": k_scale,
          "epsilon": epsilon, "rot_dim": rot_dim}
    return _impl("rms_rope_split_half", kw)(**kw)


def rms_rope_split_half_(q, k, freqs_cis, q_scale, k_scale=None, epsilon: float = 1e-6, rot_dim: int = 0):
    """Per-head RMSNorm + split-half RoPE in place (inference only)."""
    torch.ops.x_minimaxh3_amd.rms_rope_split_half_(q, k, freqs_cis, q_scale, k_scale, epsilon, rot_dim)
    return q, k


def rms_rope_split_half1(x, freqs_cis, scale, epsilon: float = 1e-6):
    kw = {"x": x, "freqs_cis": freqs_cis, "scale": scale, "epsilon": epsilon}
    return _impl("rms_rope_split_half1", kw)(**kw)


def rms_rope_split_half1_(x, freqs_cis, scale, epsilon: float = 1e-6):
    kw = {"x": x, "freqs_cis": freqs_cis, "scale": scale, "epsilon": epsilon}
    return _impl("rms_rope_split_half1_", kw)(**kw)


def apply_rope(xq: torch.Tensor, xk: torch.Tensor, freqs_cis: torch.Tensor):
    """RoPE on interleaved pairs (2i, 2i + 1) of q and k."""
    kw = {"xq": xq, "xk": xk, "freqs_cis": freqs_cis}
    return _impl("apply_rope", kw)(**kw)


def apply_rope_(xq: torch.Tensor, xk: torch.Tensor, freqs_cis: torch.Tensor):
    kw = {"xq": xq, "xk": xk, "freqs_cis": freqs_cis}
    return _impl("apply_rope_", kw)(**kw)


def apply_rope1(x: torch.Tensor, freqs_cis: torch.Tensor) -> torch.Tensor:
    kw = {"x": x, "freqs_cis": freqs_cis}
    return _impl("apply_rope1", kw)(**kw)


def apply_rope1_(x: torch.Tensor, freqs_cis: torch.Tensor) -> torch.Tensor:
    kw = {"x": x, "freqs_cis": freqs_cis}
    return _impl("apply_rope1_", kw)(**kw)


def rms_rope(q, k, freqs_cis, q_scale, k_scale=None, epsilon: float = 1e-6):
    """Per-head RMSNorm with weight + RoPE on interleaved pairs."""
    kw = {"q": q, "k": k, "freqs_cis": freqs_cis, "q_scale": q_scale, "k_scale": k_scale, "epsilon": epsilon}
    return _impl("rms_rope", kw)(**kw)


def rms_rope_(q, k, freqs_cis, q_scale, k_scale=None, epsilon: float = 1e-6):
    kw = {"q": q, "k": k, "freqs_cis": freqs_cis, "q_scale": q_scale, "k_scale": k_scale, "epsilon": epsilon}
    return _impl("rms_rope_", kw)(**kw)


def rms_rope1(x, freqs_cis, scale, epsilon: float = 1e-6):
    kw = {"x": x, "freqs_cis": freqs_cis, "scale": scale, "epsilon": epsilon}
    return _impl("rms_rope1", kw)(**kw)


def rms_rope1_(x, freqs_cis, scale, epsilon: float = 1e-6):
    kw = {"x": x, "freqs_cis": freqs_cis, "scale": scale, "epsilon": epsilon}
    return _impl("rms_rope1_", kw)(**kw)


def norm_rope(q: torch.Tensor, k: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor,
              freqs_cis: torch.Tensor, eps: float = 1e-6, head_dim: int = 128):
    """Fused AdaLN-RMSNorm (full row) + split-half 3D RoPE (per head) of Q and K."""
    return torch.ops.x_minimaxh3_amd.norm_rope(q, k, scale, shift, freqs_cis, eps, head_dim)


def w8a8_mlp(x: torch.Tensor, w1: torch.Tensor, s1: torch.Tensor, w2: torch.Tensor,
             s2: torch.Tensor) -> torch.Tensor:
    """y = int8_linear(int8_linear(x, w1, s1), w2, s2, input_act="gelu_tanh"), fused."""
    return torch.ops.x_minimaxh3_amd.w8a8_mlp(x, w1, s1, w2, s2)


def w4a8_mlp(x, w1_packed, w1_srel, w1_schannel, w2_packed, w2_srel, w2_schannel, group_size: int = 128):
    """The same MLP with grouped int4 weights (uniform levels, no rotation)."""
    return torch.ops.x_minimaxh3_amd.w4a8_mlp(x, w1_packed, w1_srel, w1_schannel, w2_packed, w2_srel,
                                              w2_schannel, group_size)


def mm_int8(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """INT8 matmul C[M,N] = A[M,K] @ B[K,N] -> int32 (CK/__init__.py:717-719)."""
    assert a.dtype == torch.int8 and b.dtype == torch.int8 and a.dim() == 2 and b.dim() == 2
    assert a.size(1) == b.size(0), f"K mismatch: {a.size(1)} vs {b.size(0)}"
    return _backend._gemm(a.contiguous(), None, b.t().contiguous(), None, None, torch.float32, epilogue=2)


# backend configuration (CK/__init__.py:772-827)
def set_backend_priority(priority: list[str]) -> None:
    registry.set_priority(priority)


def disable_backend(name: str) -> None:
    registry.disable(name)


def enable_backend(name: str) -> None:
    registry.enable(name)


def list_backends() -> dict:
    return registry.list_backends()


def use_backend(name: str):
    return registry.use_backend(name)
