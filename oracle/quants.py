"""GGUF IQ4_XS / IQ3_XXS superblock dequantisation -- test infrastructure (oracle).

CPU restatement (numpy) of the dequant arithmetic the reference runs through
gguf-py 0.18.0 ``gguf.quants.dequantize`` (reference call sites
``qwen/model.py:266`` for the CPU hot path, ``npu/iq3_xxs.py:150``,
``qwen/test_npu_experts.py:41-43``).  gguf-py is not vendored in the reference;
the formulas follow the reference's own host restatements of it:

* IQ4_XS, 136-byte superblock of 256 weights -- ``npu/quant_mv_iq4.py:174-203``
  (before its bf16 cast on :203)::

      d  = fp16 bytes[0:2]
      sh = u16  bytes[2:4]          (2 high scale bits per sub-block)
      sl = u8   bytes[4:8]          (4 low scale bits per sub-block)
      qs = u8   bytes[8:136]        (16 bytes per 32-weight sub-block)
      ls_s = ((sl[s//2] >> 4*(s%2)) & 15) | (((sh >> 2s) & 3) << 4)
      y[32s + j]      = d * (ls_s - 32) * kv[qs[16s + j] & 15]     j < 16
      y[32s + 16 + j] = d * (ls_s - 32) * kv[qs[16s + j] >> 4]

* IQ3_XXS, 98-byte superblock of 256 weights -- ``npu/iq3_xxs.py:4-15, 64-119``::

      d  = fp16 bytes[0:2]
      qs = u8   bytes[2:66]         (8 grid indices per sub-block)
      w  = u32  bytes[66:98]        (one word per 32-weight sub-block)
      db_s = d * (0.5 + (w_s >> 28)) * 0.5
      group g (0..3) of sub-block s: sign byte = ksigns[(w_s >> 7g) & 127]
      lanes 0-3 = grid[qs[8s + 2g]], lanes 4-7 = grid[qs[8s + 2g + 1]]
      y[32s + 8g + i] = db_s * grid_lane_i * (sign bit i ? -1 : +1)

Every dequantised value is an exact fp32 product (IQ4_XS: 11 + 6 + 7 significant
bits; IQ3_XXS: 11 + 5 + 6), so any evaluation order gives identical bits; the
GPU kernels are held to float equality with these functions.

Pinning: hand-derived known-answer superblocks (``tests/golden/iq_kat.npz``,
built element by element in pure Python by ``tests/golden/make_kat.py``),
field-isolation tests (one varying field at a time, expected values derived
from the layout description above), the table fixture, and brute-force
enumeration of every scale x nibble (IQ4_XS) and every grid x sign x scale
(IQ3_XXS) combination.
"""
from __future__ import annotations

import numpy as np

from oracle import tables

QK = 256
IQ4_XS_BYTES = 136
IQ3_XXS_BYTES = 98

# ggml type ids (GGMLQuantizationType) used on this path.
GGML_F32 = 0
GGML_IQ3_XXS = 18
GGML_IQ4_XS = 23

_KV = tables.kvalues_iq4nl().astype(np.float32)
_GRID = tables.iq3xxs_grid().astype(np.float32)
_SIGNS = tables.ksigns_pm1().astype(np.float32)


def _blocks(raw: np.ndarray, nbytes: int) -> np.ndarray:
    b = np.ascontiguousarray(raw).view(np.uint8).reshape(-1)
    if b.size % nbytes:
        raise ValueError(f"{b.size} bytes is not a whole number of {nbytes}-byte superblocks")
    return b.reshape(-1, nbytes)


def dequant_iq4_xs(raw: np.ndarray) -> np.ndarray:
    """uint8 bytes (n_sb*136) -> float32 [n_sb*256]."""
    b = _blocks(raw, IQ4_XS_BYTES)
    n = b.shape[0]
    d = np.ascontiguousarray(b[:, 0:2]).view(np.float16).astype(np.float32)      # [n,1]
    sh = np.ascontiguousarray(b[:, 2:4]).view(np.uint16).astype(np.int32)       # [n,1]
    sl = b[:, 4:8].astype(np.int32)                                             # [n,4]
    s = np.arange(8)
    low = (sl[:, s // 2] >> (4 * (s % 2))) & 15                                 # [n,8]
    high = (sh >> (2 * s)) & 3                                                  # [n,8]
    ls = (low | (high << 4)) - 32
    dl = d * ls.astype(np.float32)                                              # [n,8]
    qs = b[:, 8:136].reshape(n, 8, 16)
    lo = _KV[qs & 15]                                                           # [n,8,16]
    hi = _KV[qs >> 4]
    vals = np.concatenate([lo, hi], axis=2)                                     # [n,8,32]
    return (dl[:, :, None] * vals).reshape(-1)


def dequant_iq3_xxs(raw: np.ndarray) -> np.ndarray:
    """uint8 bytes (n_sb*98) -> float32 [n_sb*256]."""
    b = _blocks(raw, IQ3_XXS_BYTES)
    n = b.shape[0]
    d = np.ascontiguousarray(b[:, 0:2]).view(np.float16).astype(np.float32)      # [n,1]
    qs = b[:, 2:66].reshape(n, 8, 4, 2)
    w = np.ascontiguousarray(b[:, 66:98]).view(np.uint32)                        # [n,8]
    db = d * (np.float32(0.5) + (w >> 28).astype(np.float32)) * np.float32(0.5)  # [n,8]
    sidx = (w[:, :, None] >> (7 * np.arange(4, dtype=np.uint32))) & 127          # [n,8,4]
    signs = _SIGNS[sidx]                                                          # [n,8,4,8]
    mags = _GRID[qs].reshape(n, 8, 4, 8)                                          # [n,8,4,8]
    return (db[:, :, None, None] * (signs * mags)).reshape(-1)


def dequant(raw: np.ndarray, qtype: int) -> np.ndarray:
    if qtype == GGML_IQ4_XS:
        return dequant_iq4_xs(raw)
    if qtype == GGML_IQ3_XXS:
        return dequant_iq3_xxs(raw)
    if qtype == GGML_F32:
        return np.ascontiguousarray(raw).view(np.float32).reshape(-1).copy()
    raise ValueError(f"unsupported ggml type {qtype}")


def block_bytes(qtype: int) -> int:
    if qtype == GGML_IQ4_XS:
        return IQ4_XS_BYTES
    if qtype == GGML_IQ3_XXS:
        return IQ3_XXS_BYTES
    raise ValueError(f"unsupported ggml type {qtype}")


def dequant_matrix(raw: np.ndarray, qtype: int, M: int, K: int) -> np.ndarray:
    """Raw row-major [M, K/256 superblocks] bytes -> float32 [M, K] (torch Linear layout).
    Q8_0 / Q4_K / Q5_K / Q6_K rows go through ``oracle.kquants`` (its own restatement)."""
    if K % QK:
        raise ValueError(f"K={K} must be a multiple of {QK}")
    from oracle import kquants
    flat = np.ascontiguousarray(raw).view(np.uint8).reshape(-1)
    if int(qtype) in kquants.BLOCK:
        w, nb = kquants.BLOCK[int(qtype)]
        need = M * (K // w) * nb
        if flat.size != need:
            raise ValueError(f"{flat.size} bytes, expected {need} for M={M} K={K}")
        return kquants.dequant(flat, qtype).reshape(M, K)
    need = M * (K // QK) * block_bytes(qtype)
    if flat.size != need:
        raise ValueError(f"{flat.size} bytes, expected {need} for M={M} K={K}")
    return dequant(flat, qtype).reshape(M, K)
