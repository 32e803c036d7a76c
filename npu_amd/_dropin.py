"""Shared machinery of the drop-in operators (the ``Npu*`` classes).

Mirrors the reference's operator contract (``npu/quant_mv.py:355-463`` and
siblings): construction validates the weight (``TypeError`` for a wrong dtype,
``ValueError`` for a bad K or byte count), the weight is uploaded to device
memory lazily on the first call and the host staging copy is then released,
and ``__call__(x)`` computes ``F.linear(x, W)`` in fp32.

Differences, by design:
* the weight stays in raw GGUF layout in HBM (no repack);
* ``x`` may be one vector (as in the reference) or ``[..., in_features]``;
* a CPU ``x`` is copied to the GPU and the result copied back (the
  reference's synchronous host-in/host-out behaviour); a GPU ``x`` returns a
  GPU tensor without synchronising.
``n_cores`` / ``m`` are XDNA tiling knobs: accepted for signature
compatibility and ignored.
"""
from __future__ import annotations

import numpy as np
import torch

from npu_amd import _lib, ops
from npu_amd.gguf_types import QK, GGMLQuantizationType as QT, block_bytes
from npu_amd.profiler import profile


def device() -> torch.device:
    _lib.require_gpu()
    return torch.device("cuda", torch.cuda.current_device())


def flatten_input(x: torch.Tensor, in_features: int) -> torch.Tensor:
    if x.numel() == in_features:
        return x.reshape(1, in_features)
    assert x.shape[-1] == in_features, f"x has {x.shape[-1]} features, expected {in_features}"
    return x.reshape(-1, in_features)


def run_on_device(x: torch.Tensor, in_features: int, out_features: int, fn, prefix: str) -> torch.Tensor:
    """Route x to the GPU, run fn(x_dev [n, in]) -> [n, out], restore x's device/shape."""
    on_host = not x.is_cuda
    xf = flatten_input(x, in_features)
    with profile(f"{prefix}.to_device"):
        xd = xf.to(device(), torch.float32, non_blocking=False).contiguous() if on_host else \
            xf.to(torch.float32).contiguous()
    with profile(f"{prefix}.kernel"):
        y = fn(xd)
    if on_host:
        with profile(f"{prefix}.to_host"):
            y = y.cpu()
    return y.reshape(*x.shape[:-1], out_features)


class QuantMatVec:
    """``F.linear(x, W)`` with W as raw GGUF superblocks of one type."""

    QTYPE: int = -1
    PROFILE = "qmv"

    def __init__(self, packed_weight: np.ndarray, M: int, K: int, n_cores: int = 8, m: int | None = None):
        if isinstance(packed_weight, torch.Tensor):
            packed_weight = packed_weight.cpu().numpy()
        if packed_weight.dtype != np.uint8:
            raise TypeError(f"packed_weight must be uint8, got {packed_weight.dtype}")
        if K % QK != 0:
            raise ValueError(f"K={K} must be a multiple of {QK}")
        expected = M * (K // QK) * block_bytes(self.QTYPE)
        if packed_weight.size != expected:
            raise ValueError(f"packed_weight has {packed_weight.size} bytes, expected {expected} for M={M} K={K}")
        self.out_features = int(M)
        self.in_features = int(K)
        self.n_cores = n_cores
        self._W: np.ndarray | None = np.ascontiguousarray(packed_weight).reshape(-1)
        self._dev: torch.Tensor | None = None

    def _weight(self) -> torch.Tensor:
        if self._dev is None:
            if self._W is None:
                raise RuntimeError("weight staging buffer was already released")
            self._dev = torch.from_numpy(self._W).to(device())
            self._W = None
        return self._dev

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        w = self._weight()
        return run_on_device(x, self.in_features, self.out_features,
                             lambda xd: ops.matvec(self.QTYPE, w, self.out_features, self.in_features, xd),
                             self.PROFILE)


def check_type(t, qtype: int, what: str) -> None:
    if int(t.tensor_type) != int(qtype):
        name = getattr(t.tensor_type, "name", str(t.tensor_type))
        raise ValueError(f"need {what} tensor, got {name}")


def raw_rows(t, expert_idx: int | None = None) -> np.ndarray:
    """Raw [out, row_bytes] bytes of a 2-D tensor or of one expert of a stacked tensor (zero-copy)."""
    if expert_idx is None:
        M, K = int(t.shape[1]), int(t.shape[0])
        data = np.ascontiguousarray(t.data).view(np.uint8)
    else:
        if len(t.shape) != 3:
            raise ValueError(f"need 3D stacked expert tensor, got {tuple(t.shape)}")
        n_expert = int(t.shape[-1])
        if not 0 <= expert_idx < n_expert:
            raise IndexError(expert_idx)
        M, K = int(t.shape[1]), int(t.shape[0])
        data = np.ascontiguousarray(t.data[expert_idx]).view(np.uint8)
    return data.reshape(M, (K // QK) * block_bytes(int(t.tensor_type)))


def bf16_on_device(w: torch.Tensor) -> torch.Tensor:
    """fp32/bf16 weight -> bf16 on the GPU (the reference NPU ops also stage bf16)."""
    return w.detach().to(device=device(), dtype=torch.bfloat16).contiguous()


__all__ = ["QuantMatVec", "check_type", "raw_rows", "bf16_on_device", "run_on_device", "device", "QT"]
