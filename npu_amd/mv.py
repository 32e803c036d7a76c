"""Dense bf16 matvec operators -- drop-in for the reference's ``npu/mv.py``.

``NpuMatVec(W)(x) == F.linear(x, W)`` with W staged once in HBM as bf16 (the
reference stages bf16 too, ``npu/mv.py:209-220``) and x kept in fp32 (the
reference rounds x to bf16).  ``NpuConcatMatVec`` stacks several weights with
the same input dimension into one device buffer (reference :268-347).
"""
from __future__ import annotations

import torch

from npu_amd import ops
from npu_amd._dropin import bf16_on_device, run_on_device
from npu_amd.gguf_types import GGMLQuantizationType as QT


class NpuMatVec:
    def __init__(self, weight: torch.Tensor, n_cores: int = 8, profile_prefix: str = "mv"):
        assert weight.dim() == 2
        self.out_features, self.in_features = (int(s) for s in weight.shape)
        if self.in_features % 32:
            raise ValueError(f"in_features={self.in_features} must be a multiple of 32")
        self.n_cores = n_cores
        self.profile_prefix = profile_prefix
        self._weight_src: torch.Tensor | None = weight
        self._W: torch.Tensor | None = None

    def _weight(self) -> torch.Tensor:
        if self._W is None:
            if self._weight_src is None:
                raise RuntimeError("source weight was already released")
            self._W = bf16_on_device(self._weight_src)
            self._weight_src = None
        return self._W

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        W = self._weight()
        return run_on_device(x, self.in_features, self.out_features,
                             lambda xd: ops.matvec(QT.BF16, W, self.out_features, self.in_features, xd),
                             self.profile_prefix)


class NpuConcatMatVec(NpuMatVec):
    """``F.linear(x, cat(weights, 0))`` from one stacked bf16 buffer; ``out_splits`` records the parts."""

    def __init__(self, weights: tuple[torch.Tensor, ...], n_cores: int = 8, profile_prefix: str = "mv_concat"):
        if not weights:
            raise ValueError("weights must be non-empty")
        for W in weights:
            assert W.dim() == 2
        in_features = weights[0].shape[1]
        if any(W.shape[1] != in_features for W in weights):
            raise ValueError("all weights must have the same input dimension")
        self.out_splits = tuple(int(W.shape[0]) for W in weights)
        self._parts: tuple[torch.Tensor, ...] | None = weights
        super().__init__(torch.empty(sum(self.out_splits), in_features, device="meta"), n_cores, profile_prefix)
        self._weight_src = None

    def _weight(self) -> torch.Tensor:
        if self._W is None:
            if self._parts is None:
                raise RuntimeError("source weights were already released")
            self._W = torch.cat([bf16_on_device(W) for W in self._parts], dim=0).contiguous()
            self._parts = None
        return self._W
