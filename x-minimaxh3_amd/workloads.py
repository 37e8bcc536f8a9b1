"""Seeded synthetic workloads of the hot path (generated on the CPU).

Every tensor is drawn on the CPU from one ``torch.Generator().manual_seed(seed)``
in a fixed order, so the GPU run, the CPU baseline and the parity tests see
identical bytes. Shapes and value distributions:

* MLP (W8A8): x ~ N(0,1) [M, d] with ``n_outlier`` channels (a random subset)
  scaled x20, cast to bf16; W1 [ffn, d] and W2 [d, ffn] ~ N(0, 0.02) fp32,
  quantised per output channel with the activation rule in fp32
  (s = amax/127, q = clamp(rint(w/s), -128, 127)). Draw order: x, outlier
  set, W1, W2.
* MLP (W4A8): the same x and fp32 weights, quantised to grouped int4
  (symmetric, uniform levels, group 128 along K, bf16 s_rel, fp32 s_channel)
  with the reference's generator rule (CK/backends/eager/w4a8_int8.py:169-173,
  188-191, 200-202; CK = backends/turbo/vendor/comfy_kitchen).
* norm-rope: q, k ~ N(0,1) bf16 [M, d]; shift, scale, gate ~ N(0, 0.1) bf16
  [1, d]; the split-half RoPE table for a T x H x W grid (t-major integer
  positions, per-axis dims 44/42/42, theta 10000), fp32 [1, M, 1, 64, 2, 2]
  (h3serve/native_engine/model/layers.py:51-69 form).

Named configurations (token counts M, model width d, ffn):
  mlp_small   1,024 x 1,536 -> 6,144        (8 outlier channels)
  norm_rope   25,200 = 7x45x80, d 5,120 = 40 heads x 128
  mlp_720p    25,200 x 5,120 -> 13,824      (51 outlier channels)
  long        130,560 = 16x68x120, chunks of 16,384 tokens
"""

from __future__ import annotations

import torch

CONFIGS = {
    "mlp_small": dict(M=1024, d=1536, ffn=6144, n_outlier=8),
    "mlp_720p": dict(M=25200, d=5120, ffn=13824, n_outlier=51),
    "norm_rope_720p": dict(grid=(7, 45, 80), d=5120, head_dim=128),
    "long_16x68x120": dict(grid=(16, 68, 120), d=5120, ffn=13824, n_outlier=51, chunk=16384),
}


def quantize_weight_per_channel(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric per-output-channel int8 of an fp32 [N, K] weight."""
    amax = w.abs().amax(dim=1, keepdim=True)
    s = (amax / 127.0).clamp(min=1e-30)
    q = (w / s).round().clamp(-128, 127).to(torch.int8)
    return q, s.reshape(-1).float()


def quantize_weight_w4(w: torch.Tensor, group_size: int = 128, srel_dtype: torch.dtype = torch.bfloat16):
    """Grouped symmetric int4 (uniform levels) of an fp32 [N, K] weight:
    gs = max(amax_g/7, 1e-8); signed = clamp(round(w/gs), -8, 7);
    s_channel = max(amax_n(|signed*gs|)/127, 1e-8); s_rel = gs/s_channel;
    byte = (signed[2j]+8) | (signed[2j+1]+8) << 4."""
    n, k = w.shape
    g = w.float().view(n, k // group_size, group_size)
    gs = (g.abs().amax(dim=-1, keepdim=True) / 7.0).clamp(min=1e-8)
    signed = (g / gs).round().clamp(-8, 7).to(torch.int32)
    s_channel = ((signed * gs).abs().amax(dim=(1, 2)) / 127.0).clamp(min=1e-8)
    s_rel = (gs.squeeze(-1) / s_channel.unsqueeze(1)).float()
    u = (signed + 8).view(n, k)
    packed = ((u[:, 0::2] & 0xF) | ((u[:, 1::2] & 0xF) << 4)).to(torch.int8).contiguous()
    return packed, s_rel.to(srel_dtype).contiguous(), s_channel.float().contiguous()


def mlp_inputs(M: int, d: int, ffn: int, n_outlier: int, seed: int = 0, weights: str = "w8a8",
               group_size: int = 128) -> dict:
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, d, generator=g)
    idx = torch.randperm(d, generator=g)[:n_outlier]
    x[:, idx] *= 20.0
    x = x.to(torch.bfloat16)
    w1f = torch.randn(ffn, d, generator=g) * 0.02
    w2f = torch.randn(d, ffn, generator=g) * 0.02
    out = {"x": x, "outliers": idx}
    if weights in ("w8a8", "both"):
        out["w1"], out["s1"] = quantize_weight_per_channel(w1f)
        out["w2"], out["s2"] = quantize_weight_per_channel(w2f)
    if weights in ("w4a8", "both"):
        out["w1_packed"], out["w1_srel"], out["w1_schannel"] = quantize_weight_w4(w1f, group_size)
        out["w2_packed"], out["w2_srel"], out["w2_schannel"] = quantize_weight_w4(w2f, group_size)
    return out


def grid_positions(t: int, h: int, w: int) -> torch.Tensor:
    tt = torch.arange(t).view(t, 1, 1).expand(t, h, w)
    hh = torch.arange(h).view(1, h, 1).expand(t, h, w)
    ww = torch.arange(w).view(1, 1, w).expand(t, h, w)
    return torch.stack((tt.reshape(-1), hh.reshape(-1), ww.reshape(-1)), dim=-1)


def rope_table_3d(grid: tuple[int, int, int], dims=(44, 42, 42), theta: float = 10000.0,
                  dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """[1, M, 1, sum(dims)/2, 2, 2] table (cos, -sin, sin, cos) of per-axis
    angles pos * theta^(-2i/dim), concatenated [t | h | w]."""
    pos = grid_positions(*grid)
    parts = []
    for a, dim in enumerate(dims):
        inv = (1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float64) / dim))).float()
        parts.append(pos[:, a:a + 1].float() * inv.view(1, -1))
    ang = torch.cat(parts, dim=-1)
    c, s = torch.cos(ang), torch.sin(ang)
    half = ang.shape[-1]
    return torch.stack((c, -s, s, c), dim=-1).reshape(1, ang.shape[0], 1, half, 2, 2).to(dtype)


def norm_rope_inputs(grid=(7, 45, 80), d: int = 5120, head_dim: int = 128, seed: int = 0,
                     dims=(44, 42, 42)) -> dict:
    g = torch.Generator().manual_seed(seed)
    m = grid[0] * grid[1] * grid[2]
    q = torch.randn(m, d, generator=g).to(torch.bfloat16)
    k = torch.randn(m, d, generator=g).to(torch.bfloat16)
    shift = (torch.randn(1, d, generator=g) * 0.1).to(torch.bfloat16)
    scale = (torch.randn(1, d, generator=g) * 0.1).to(torch.bfloat16)
    gate = (torch.randn(1, d, generator=g) * 0.1).to(torch.bfloat16)
    if sum(dims) != head_dim:
        raise ValueError("axis dims must add up to head_dim")
    freqs = rope_table_3d(grid, dims)
    return {"q": q, "k": k, "shift": shift, "scale": scale, "gate": gate, "freqs": freqs,
            "eps": 1e-6, "head_dim": head_dim}
