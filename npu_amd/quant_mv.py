"""IQ3_XXS dequant-matvec operator -- drop-in for the reference's ``npu/quant_mv.py``.

``NpuQuantMatVec`` computes ``F.linear(x, dequant(W))`` with W stored in HBM as
raw 98-byte GGUF IQ3_XXS superblocks and dequantised in registers by the gfx950
kernel (``csrc/matvec.hip``).  The reference repacks each superblock to 128
bytes on the host (``npu/quant_mv.py:226-242``); here ``B_BYTES`` is the raw
98 and the ``repack_*`` functions are zero-copy reshapes, so callers that
derive row bytes from ``BLK``/``B_BYTES`` (``qwen/forward.py:542-549``) keep
working unchanged.
"""
from __future__ import annotations

import numpy as np

from npu_amd._dropin import QuantMatVec, check_type, raw_rows
from npu_amd.gguf_types import GGMLQuantizationType as QT

BLK = 256          # K elements per IQ3_XXS superblock
B_BYTES = 98       # bytes per superblock as stored in HBM (raw GGUF)


def repack_iq3_xxs_weight(t) -> np.ndarray:
    """Raw (M=out, K/256*98) bytes of a 2-D GGUF IQ3_XXS tensor (reference :245-269)."""
    check_type(t, QT.IQ3_XXS, "IQ3_XXS")
    return raw_rows(t)


def repack_iq3_xxs_per_expert(t, expert_idx: int) -> np.ndarray:
    """Raw (M, K/256*98) bytes of one expert of a stacked IQ3_XXS tensor (reference :272-295)."""
    check_type(t, QT.IQ3_XXS, "IQ3_XXS")
    return raw_rows(t, expert_idx)


class NpuQuantMatVec(QuantMatVec):
    """``F.linear(x, W)`` with W as raw IQ3_XXS superblocks (reference :355-463)."""

    QTYPE = QT.IQ3_XXS
    PROFILE = "qmv"

    @classmethod
    def from_iq3_xxs_bytes(cls, packed: np.ndarray, M: int, K: int, n_cores: int = 8,
                           m: int | None = None) -> "NpuQuantMatVec":
        return cls(packed, M, K, n_cores=n_cores, m=m)

    @classmethod
    def from_gguf_tensor(cls, t, expert_idx: int | None = None, n_cores: int = 8,
                         m: int | None = None) -> "NpuQuantMatVec":
        packed = repack_iq3_xxs_weight(t) if expert_idx is None else repack_iq3_xxs_per_expert(t, expert_idx)
        return cls(packed, int(t.shape[1]), int(t.shape[0]), n_cores=n_cores, m=m)
