"""Fused SwiGLU MLP -- drop-in for the reference's ``npu/mlp.py:NpuFusedMLP``.

``NpuFusedMLP(w_gate_up, w_down, w_up=...)(x) == F.linear(silu(F.linear(x, G)) *
F.linear(x, U), W_down)`` with the weights staged once in HBM as bf16 (as the
reference stages them, ``npu/mlp.py:379-411``), fp32 activations and fp32
accumulation, run as two kernels (gate/up + SwiGLU, then down).  With
``w_up=None``, ``w_gate_up`` is the stacked ``[2*ffn, hidden]`` gate|up weight.
"""
from __future__ import annotations

import torch

from npu_amd import ops
from npu_amd._dropin import bf16_on_device, run_on_device
from npu_amd.gguf_types import GGMLQuantizationType as QT


class NpuFusedMLP:
    def __init__(self, w_gate_up: torch.Tensor, w_down: torch.Tensor, n_cores: int = 4, *,
                 w_up: torch.Tensor | None = None):
        assert w_gate_up.dim() == 2 and w_down.dim() == 2
        if w_up is not None:
            assert w_up.dim() == 2 and w_gate_up.shape == w_up.shape
            ffn, self.hidden = (int(s) for s in w_gate_up.shape)
            self.ffn2 = 2 * ffn
        else:
            self.ffn2, self.hidden = (int(s) for s in w_gate_up.shape)
        self.hidden_out, self.ffn = (int(s) for s in w_down.shape)
        assert self.ffn2 == 2 * self.ffn
        assert self.hidden_out == self.hidden
        if self.hidden % 32 or self.ffn % 32:
            raise ValueError("hidden and ffn must be multiples of 32")
        self.n_cores = n_cores
        self._src = (w_gate_up, w_up, w_down)
        self._dev: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None

    def _weights(self):
        if self._dev is None:
            if self._src is None:
                raise RuntimeError("source weights were already released")
            gu, up, down = self._src
            if up is None:
                g, u = gu[: self.ffn], gu[self.ffn:]
            else:
                g, u = gu, up
            self._dev = (bf16_on_device(g), bf16_on_device(u), bf16_on_device(down))
            self._src = None
        return self._dev

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        g, u, d = self._weights()
        return run_on_device(x, self.hidden, self.hidden,
                             lambda xd: ops.swiglu_mlp(QT.BF16, g, u, QT.BF16, d, self.hidden, self.ffn, xd),
                             "mlp")
