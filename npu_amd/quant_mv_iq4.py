"""IQ4_XS dequant-matvec operator -- drop-in for the reference's ``npu/quant_mv_iq4.py``.

The reference expands every 136-byte superblock to 512 bytes of bf16 on the
host (``npu/quant_mv_iq4.py:174-203``) and runs a plain bf16 dot on the tile.
Here the raw 136-byte superblocks stay in HBM and are dequantised in registers
(``csrc/iq_decode.h``) with fp32 accumulation, so ``B_BYTES == RAW_B_BYTES``.
"""
from __future__ import annotations

import numpy as np

from npu_amd._dropin import QuantMatVec, check_type, raw_rows
from npu_amd.gguf_types import GGMLQuantizationType as QT

BLK = 256
RAW_B_BYTES = 136
B_BYTES = 136


def repack_iq4_xs_weight(t) -> np.ndarray:
    """Raw (M, K/256*136) bytes of a 2-D IQ4_XS tensor (reference :206-214)."""
    check_type(t, QT.IQ4_XS, "IQ4_XS")
    return raw_rows(t)


def repack_iq4_xs_per_expert(t, expert_idx: int) -> np.ndarray:
    """Raw bytes of one expert of a stacked IQ4_XS tensor (reference :217-231)."""
    check_type(t, QT.IQ4_XS, "IQ4_XS")
    return raw_rows(t, expert_idx)


class NpuIQ4MatVec(QuantMatVec):
    """``F.linear(x, W)`` with W as raw IQ4_XS superblocks (reference :262-361)."""

    QTYPE = QT.IQ4_XS
    PROFILE = "qmv_iq4"

    def __init__(self, packed_weight: np.ndarray, M: int, K: int, n_cores: int = 4, m: int | None = None):
        super().__init__(packed_weight, M, K, n_cores=n_cores, m=m)

    @classmethod
    def from_iq4_xs_bytes(cls, packed: np.ndarray, M: int, K: int, n_cores: int = 4,
                          m: int | None = None) -> "NpuIQ4MatVec":
        return cls(packed, M, K, n_cores=n_cores, m=m)

    @classmethod
    def from_gguf_tensor(cls, t, expert_idx: int | None = None, n_cores: int = 4,
                         m: int | None = None) -> "NpuIQ4MatVec":
        packed = repack_iq4_xs_weight(t) if expert_idx is None else repack_iq4_xs_per_expert(t, expert_idx)
        return cls(packed, int(t.shape[1]), int(t.shape[0]), n_cores=n_cores, m=m)
