"""Token-chunked DiT-block driver: fused norm-rope of Q and K plus the W8A8
MLP over a long token sequence, 16,384 tokens at a time.

The reference drives its MLP in token chunks (8,192 tokens, 4,096 with LoRA)
to bound the fp32/bf16 intermediates on a 24 GB card
(h3serve/native_engine/model/fused_mlp.py:222-266, 314-323). Every op on this
path is per token (quantisation scale, GEMM rows, GELU, requant, RMS, RoPE), so
chunking changes no bit of the result; on a 288 GB MI355X it only bounds the
MLP workspace (q1, g, q2 of one chunk, about 0.8 GB at 16,384 tokens).

Two ways to run it:

* ``run_resident``: Q, K, x and the outputs live in HBM; chunks run back to
  back on the current stream (the compute-only rate).
* ``run_streamed``: Q, K, x and the outputs live in pinned host memory; two
  device slots are double-buffered across three streams (host-to-device
  copies, compute, device-to-host copies), so chunk i+1 is uploaded and chunk
  i-1 downloaded while chunk i computes. All streams keep the default
  priority. End-to-end time is then bound by PCIe when the host link is
  slower than the kernels.
"""

from __future__ import annotations

import torch

from . import backend

__all__ = ["LongBlockDriver"]


class LongBlockDriver:
    """One DiT block's norm-rope + MLP over ``tokens`` tokens in chunks.

    Weights: w1 int8 [F, D], s1 fp32 [F] (or scalar), w2 int8 [D, F], s2.
    Modulation: scale/shift [1, D] in Q's dtype (one sample); RoPE table
    [1, tokens, 1, head_dim/2, 2, 2] on the device.
    """

    def __init__(self, w1: torch.Tensor, s1: torch.Tensor, w2: torch.Tensor, s2: torch.Tensor,
                 scale: torch.Tensor, shift: torch.Tensor, chunk: int = 16384, eps: float = 1e-6,
                 head_dim: int = 128):
        if chunk <= 0:
            raise ValueError("chunk must be positive")
        self.dev = w1.device
        self.w1, self.s1, self.w2, self.s2 = w1, s1, w2, s2
        self.scale, self.shift = scale, shift
        self.chunk, self.eps, self.head_dim = chunk, eps, head_dim
        self.d = w1.shape[1]
        self.f = w1.shape[0]
        # one MLP workspace per device slot (the streamed mode overlaps two chunks)
        nbytes = backend._lib.query("xmh3_w8a8_mlp_workspace_bytes", chunk, self.d, self.f)
        self.ws = [torch.empty(nbytes, dtype=torch.uint8, device=self.dev) for _ in range(2)]
        self._slots = None

    def _chunks(self, tokens: int):
        for start in range(0, tokens, self.chunk):
            yield start, min(tokens, start + self.chunk)

    def _block_inplace(self, q, k, x, freqs, y, slot: int) -> None:
        backend.norm_rope(q, k, self.scale, self.shift, freqs, self.eps, self.head_dim, inplace=True)
        backend.w8a8_mlp(x, self.w1, self.s1, self.w2, self.s2, out=y, workspace=self.ws[slot])

    def run_resident(self, q: torch.Tensor, k: torch.Tensor, x: torch.Tensor, freqs: torch.Tensor,
                     qo: torch.Tensor | None = None, ko: torch.Tensor | None = None,
                     y: torch.Tensor | None = None):
        """All tensors in HBM: q, k, x [tokens, D] -> (qo, ko, y)."""
        tokens = q.shape[0]
        qo = torch.empty_like(q) if qo is None else qo
        ko = torch.empty_like(k) if ko is None else ko
        y = torch.empty(tokens, self.d, dtype=torch.bfloat16, device=self.dev) if y is None else y
        for i, (a, b) in enumerate(self._chunks(tokens)):
            self._block_resident(q[a:b], k[a:b], x[a:b], freqs[:, a:b], qo[a:b], ko[a:b], y[a:b], i & 1)
        return qo, ko, y

    def _block_resident(self, q, k, x, freqs, qo, ko, y, slot):
        # norm-rope writes straight into the output rows, then the MLP
        backend.norm_rope(q, k, self.scale, self.shift, freqs, self.eps, self.head_dim, out=(qo, ko))
        backend.w8a8_mlp(x, self.w1, self.s1, self.w2, self.s2, out=y, workspace=self.ws[slot])

    def run_streamed(self, q_host: torch.Tensor, k_host: torch.Tensor, x_host: torch.Tensor,
                     freqs: torch.Tensor, qo_host: torch.Tensor, ko_host: torch.Tensor,
                     y_host: torch.Tensor) -> None:
        """Inputs and outputs in pinned host memory, double-buffered through
        two device slots; returns when every download has completed."""
        tokens = q_host.shape[0]
        c, d = self.chunk, self.d
        if self._slots is None:
            mk = lambda dt: [torch.empty(c, d, dtype=dt, device=self.dev) for _ in range(2)]
            self._slots = {"q": mk(q_host.dtype), "k": mk(k_host.dtype), "x": mk(x_host.dtype),
                           "y": mk(torch.bfloat16)}
        sl = self._slots
        cur = torch.cuda.current_stream(self.dev)
        up, comp, down = (torch.cuda.Stream(self.dev) for _ in range(3))
        uploaded = [torch.cuda.Event() for _ in range(2)]
        computed = [torch.cuda.Event() for _ in range(2)]
        downloaded = [torch.cuda.Event() for _ in range(2)]
        up.wait_stream(cur)
        for i, (a, b) in enumerate(self._chunks(tokens)):
            s, n = i & 1, b - a
            with torch.cuda.stream(up):
                if i >= 2:
                    up.wait_event(downloaded[s])        # slot s's previous results are on the host
                sl["q"][s][:n].copy_(q_host[a:b], non_blocking=True)
                sl["k"][s][:n].copy_(k_host[a:b], non_blocking=True)
                sl["x"][s][:n].copy_(x_host[a:b], non_blocking=True)
                uploaded[s].record(up)
            with torch.cuda.stream(comp):
                comp.wait_event(uploaded[s])
                self._block_inplace(sl["q"][s][:n], sl["k"][s][:n], sl["x"][s][:n], freqs[:, a:b],
                                    sl["y"][s][:n], s)
                computed[s].record(comp)
            with torch.cuda.stream(down):
                down.wait_event(computed[s])
                qo_host[a:b].copy_(sl["q"][s][:n], non_blocking=True)
                ko_host[a:b].copy_(sl["k"][s][:n], non_blocking=True)
                y_host[a:b].copy_(sl["y"][s][:n], non_blocking=True)
                downloaded[s].record(down)
        down.synchronize()
        cur.wait_stream(down)
