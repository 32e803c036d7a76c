"""``NpuLinear``: the reference's bf16 linear layer (``npu/linear.py:147-244``) on the GPU.

``NpuLinear(weight[out, in], share_N_pad=None)(x[..., in]) -> y[..., out]`` fp32, equal
to ``F.linear(x, W)`` with W rounded once to bf16 and held in HBM.  Products run on
the dense bf16 kernels of ``gm_matvec``: one token per launch row on the VALU matvec
(``k_mv_bf16``), two or more on ``v_mfma_f32_16x16x32_bf16`` (``k_mv_bf16_mfma``)
with x split into exact bf16 planes, fp32 accumulation in both.

Differences from the reference, none of which changes the call:
* x keeps its fp32 value (the reference rounds x to bf16 before its NPU matmul,
  ``npu/linear.py:219-221``), so the result is closer to F.linear in fp32;
* ``share_N_pad`` picks the XDNA xclbin a set of layers shares; there is no such
  object here, so it is validated as the reference validates it (>= out_features)
  and otherwise ignored;
* ``in_features`` must be a multiple of 32 (the reference's planner needs 64);
* a GPU x returns a GPU tensor without synchronising; a CPU x is copied to the GPU
  and the result back (the reference's host-in / host-out behaviour).
"""
from __future__ import annotations

import torch

from npu_amd.mv import NpuMatVec


class NpuLinear:
    def __init__(self, weight: torch.Tensor, share_N_pad: int | None = None):
        assert weight.dim() == 2, "expected [out, in]"
        self.out_features, self.in_features = (int(s) for s in weight.shape)
        if share_N_pad is not None and int(share_N_pad) < self.out_features:
            raise ValueError(f"share_N_pad={share_N_pad} < out_features={self.out_features}")
        self.share_N_pad = share_N_pad
        self._mv = NpuMatVec(weight, profile_prefix="lin")

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        return self._mv(x)
