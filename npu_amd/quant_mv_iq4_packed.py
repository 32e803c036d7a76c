"""Semi-compact IQ4_XS operator -- drop-in for the reference's ``npu/quant_mv_iq4_packed.py``.

The reference's "packed" format (288 B per superblock: fp32 group scales + int8
kvalues, ``npu/quant_mv_iq4_packed.py:181-206``) exists to avoid a slow scalar
nibble lookup on the AIE tile.  On gfx950 the raw 136-byte superblock is
decoded in registers with ``v_perm_b32`` table lookups, so the packed operator
shares the raw IQ4_XS kernel and ``B_BYTES`` is 136.
"""
from __future__ import annotations

import numpy as np

from npu_amd._dropin import check_type, raw_rows
from npu_amd.gguf_types import GGMLQuantizationType as QT
from npu_amd.quant_mv_iq4 import BLK, RAW_B_BYTES, NpuIQ4MatVec

B_BYTES = 136

__all__ = ["BLK", "RAW_B_BYTES", "B_BYTES", "NpuIQ4PackedMatVec", "repack_iq4_xs_packed_weight",
           "repack_iq4_xs_packed_per_expert"]


def repack_iq4_xs_packed_weight(t) -> np.ndarray:
    check_type(t, QT.IQ4_XS, "IQ4_XS")
    return raw_rows(t)


def repack_iq4_xs_packed_per_expert(t, expert_idx: int) -> np.ndarray:
    check_type(t, QT.IQ4_XS, "IQ4_XS")
    return raw_rows(t, expert_idx)


class NpuIQ4PackedMatVec(NpuIQ4MatVec):
    """Same contract as the reference (:265-364); raw IQ4_XS bytes in HBM."""

    PROFILE = "qmv_iq4_packed"

    @classmethod
    def from_iq4_xs_packed_bytes(cls, packed: np.ndarray, M: int, K: int, n_cores: int = 4,
                                 m: int | None = None) -> "NpuIQ4PackedMatVec":
        return cls(packed, M, K, n_cores=n_cores, m=m)

    @classmethod
    def from_gguf_tensor(cls, t, expert_idx: int | None = None, n_cores: int = 4,
                         m: int | None = None) -> "NpuIQ4PackedMatVec":
        packed = (repack_iq4_xs_packed_weight(t) if expert_idx is None
                  else repack_iq4_xs_packed_per_expert(t, expert_idx))
        return cls(packed, int(t.shape[1]), int(t.shape[0]), n_cores=n_cores, m=m)
