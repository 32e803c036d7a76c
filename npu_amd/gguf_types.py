"""GGUF tensor duck types for the drop-in operators.

gguf-py (reference dependency, pinned 0.18.0 at ``uv.lock:132-134``) is not
available here; these stand-ins carry the attributes the reference's
``from_gguf_tensor`` paths read (``npu/quant_mv.py:245-295``,
``qwen/model.py:230-277``): ``tensor_type`` (ggml id), ``shape`` in ggml order
``(in, out[, n_expert])``, ``data`` as uint8 ``(n_expert, out, bytes_per_row)``
(or ``(out, bytes_per_row)`` for 2-D tensors) and ``name``.
"""
from __future__ import annotations

import enum
from dataclasses import dataclass

import numpy as np

QK = 256


class GGMLQuantizationType(enum.IntEnum):
    """ggml tensor type ids (the ids GGUF files store); the kernels here take F32, F16,
    BF16, IQ3_XXS and IQ4_XS."""

    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q8_1 = 9
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15
    IQ2_XXS = 16
    IQ2_XS = 17
    IQ3_XXS = 18
    IQ1_S = 19
    IQ4_NL = 20
    IQ3_S = 21
    IQ2_S = 22
    IQ4_XS = 23
    I8 = 24
    I16 = 25
    I32 = 26
    I64 = 27
    F64 = 28
    IQ1_M = 29
    BF16 = 30
    TQ1_0 = 34
    TQ2_0 = 35


# (weights, bytes) per block of the types the kernels here read
_BLOCKS = {
    GGMLQuantizationType.IQ4_XS: (QK, 136),
    GGMLQuantizationType.IQ3_XXS: (QK, 98),
    GGMLQuantizationType.Q8_0: (32, 34),
    GGMLQuantizationType.Q4_K: (QK, 144),
    GGMLQuantizationType.Q5_K: (QK, 176),
    GGMLQuantizationType.Q6_K: (QK, 210),
    GGMLQuantizationType.BF16: (QK, 2 * QK),
    GGMLQuantizationType.F32: (QK, 4 * QK),
}


def _block(qtype: int) -> tuple[int, int]:
    try:
        return _BLOCKS[GGMLQuantizationType(int(qtype))]
    except (KeyError, ValueError):
        raise ValueError(f"unsupported ggml type {qtype}") from None


def block_bytes(qtype: int) -> int:
    """Bytes of one block (256 weights, or 32 for Q8_0)."""
    return _block(qtype)[1]


def block_weights(qtype: int) -> int:
    return _block(qtype)[0]


def row_bytes(qtype: int, K: int) -> int:
    w = block_weights(qtype)
    if K % w:
        raise ValueError(f"K={K} must be a multiple of {w}")
    return (K // w) * block_bytes(qtype)


@dataclass
class QuantTensor:
    """A GGUF tensor record: raw bytes plus ggml metadata."""

    name: str
    tensor_type: GGMLQuantizationType
    shape: tuple[int, ...]          # ggml order: (in, out[, n_expert])
    data: np.ndarray                # uint8 (n_expert, out, row_bytes) or (out, row_bytes)

    def __post_init__(self) -> None:
        self.tensor_type = GGMLQuantizationType(int(self.tensor_type))
        self.shape = tuple(int(s) for s in self.shape)
        if self.data.dtype != np.uint8:
            raise TypeError("data must be uint8")
        k, m = self.shape[0], self.shape[1]
        rb = row_bytes(self.tensor_type, k)
        want = ((self.shape[2],) if len(self.shape) == 3 else ()) + (m, rb)
        if tuple(self.data.shape) != want:
            raise ValueError(f"{self.name}: data shape {self.data.shape} != {want}")

    @property
    def n_expert(self) -> int:
        return self.shape[2] if len(self.shape) == 3 else 1
