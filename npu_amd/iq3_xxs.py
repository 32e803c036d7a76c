"""IQ3_XXS tables and dequant -- drop-in for the reference's ``npu/iq3_xxs.py``.

``GRID`` (fp32 [256, 4]) and ``KSIGNS`` (int8 +1/-1 [128, 8]) are decoded from
the device header ``csrc/iq_tables.h`` (gguf-py 0.18.0's grid, as the
reference's ``npu/iq3_xxs_tables.h`` holds it) and the ksigns parity rule.
``dequant_block`` / ``dequant_rows`` run the gfx950 dequant kernel; there is no
CPU implementation in this package.
"""
from __future__ import annotations

import re
from pathlib import Path

import numpy as np
import torch

from npu_amd import ops
from npu_amd._dropin import device
from npu_amd.gguf_types import GGMLQuantizationType as QT


def _load_grid() -> np.ndarray:
    text = (Path(__file__).resolve().parent / "csrc" / "iq_tables.h").read_text()
    body = text.split("#define GM_IQ3XXS_GRID_INIT", 1)[1].split("#define", 1)[0]
    words = np.array([int(v, 16) for v in re.findall(r"0x([0-9a-f]{8})u", body)], dtype=np.uint32)
    lanes = (words[:, None] >> (8 * np.arange(4, dtype=np.uint32))[None, :]) & 0xFF
    return lanes.astype(np.float32)


def _build_ksigns() -> np.ndarray:
    i = np.arange(128)
    byte = i | ((np.array([bin(v).count("1") for v in i]) & 1) << 7)
    bits = (byte[:, None] >> np.arange(8)[None, :]) & 1
    return np.where(bits == 0, np.int8(1), np.int8(-1))


GRID: np.ndarray = _load_grid()          # (256, 4) fp32
KSIGNS: np.ndarray = _build_ksigns()     # (128, 8) int8

assert GRID.shape == (256, 4) and GRID.dtype == np.float32
assert KSIGNS.shape == (128, 8) and KSIGNS.dtype == np.int8


def dequant_rows(blocks_u8: np.ndarray) -> np.ndarray:
    """(..., n_blocks, 98) uint8 -> fp32 (..., n_blocks*256), on the GPU."""
    blocks_u8 = np.array(blocks_u8, copy=True, order="C")      # writable: torch.from_numpy shares it
    if blocks_u8.dtype != np.uint8 or blocks_u8.shape[-1] != 98:
        raise ValueError(f"need (..., n, 98) uint8, got {blocks_u8.shape}/{blocks_u8.dtype}")
    n = blocks_u8.size // 98
    out = ops.dequant(QT.IQ3_XXS, torch.from_numpy(blocks_u8.reshape(-1)).to(device()), n).cpu().numpy()
    return out.reshape(*blocks_u8.shape[:-2], blocks_u8.shape[-2] * 256)


def dequant_block(block_bytes) -> np.ndarray:
    """One 98-byte IQ3_XXS block -> fp32[256]."""
    if isinstance(block_bytes, (bytes, bytearray)):
        block = np.frombuffer(bytes(block_bytes), dtype=np.uint8)
    else:
        block = np.ascontiguousarray(block_bytes).view(np.uint8).reshape(-1)
    if block.shape != (98,):
        raise ValueError(f"expected 98-byte IQ3_XXS block, got {block.shape}")
    return dequant_rows(block.reshape(1, 98))
