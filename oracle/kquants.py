"""GGUF Q8_0 / Q4_K / Q5_K / Q6_K dequantisation -- test infrastructure (oracle).

The reference model's GGUF holds a few tensors outside IQ3_XXS / IQ4_XS: the Q5_K /
Q6_K routed-expert outliers of blk.1 / blk.34 (``qwen/forward.py:495-498``), and
other types among the shared-expert and dense tensors (``qwen/test_dequant.py:3-4``).
The reference dequantises them with gguf-py 0.18.0 ``gguf.quants.dequantize``
(``qwen/model.py:212, 266``; pinned at ``uv.lock:132-134``, not vendored).  This
module restates the ggml block formats that gguf-py decodes (little-endian; fp16
``d`` / ``dmin``; "sub-block" = 32 weights, "block" = what the type stores):

* Q8_0, 34 B per 32 weights: d, int8 q[32];  y = d * q.
* Q4_K, 144 B per 256: d, dmin, scales[12], qs[128].  Sub-block s (0..7) has a 6-bit
  scale sc_s and 6-bit min m_s packed in scales[12]:
      s < 4:  sc = scales[s] & 63,                        m = scales[s + 4] & 63
      s >= 4: sc = (scales[s + 4] & 15) | (scales[s - 4] >> 6) << 4,
              m  = (scales[s + 4] >> 4) | (scales[s] >> 6) << 4
  weights 64p .. 64p + 31 are the low nibbles of qs[32p .. 32p + 31] (sub-block 2p),
  64p + 32 .. 64p + 63 their high nibbles (sub-block 2p + 1):
      y = (d * sc_s) * q - (dmin * m_s)
* Q5_K, 176 B per 256: d, dmin, scales[12], qh[32], qs[128]; as Q4_K with a fifth bit:
  weight l (< 32) of sub-block s adds 16 when bit s of qh[l] is set.
* Q6_K, 210 B per 256: ql[128], qh[64], int8 scales[16], d.  Weight e (0..255) with
  n = e // 128, quarter = (e % 128) // 32, l = e % 32 has the 6-bit value
      low 4 bits: ql[64n + l + 32 (quarter & 1)], low nibble if quarter < 2 else high
      high 2 bits: bits 2 quarter .. 2 quarter + 1 of qh[32n + l]
  and y = (d * scales[e // 16]) * (value - 32).

Exactness: d * sc (11 + 6 or 8 bits) and its product with the quant (<= 24 bits in
all four formats) are exact in fp32, so each weight has at most one rounding (the
subtraction of the min term in Q4_K / Q5_K) and any evaluation order that keeps the
products exact -- numpy's, ggml's, an fma -- gives identical bits.

Parity: no reference vectors exist for these types (gguf-py and the model file are
absent), so agreement with gguf-py is unpinned beyond this restatement of the format.
``tests/test_oracle_kquants.py`` pins this implementation against an independent
per-weight packer (``pack_*``: chosen quants and scales -> bytes), closed forms and
exhaustive scale/min packings.
"""
from __future__ import annotations

import numpy as np

Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14
BLOCK = {Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}   # (weights, bytes)


def _f16(b: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(b).view(np.float16).astype(np.float32).reshape(-1)


def _blocks(raw: np.ndarray, qtype: int) -> np.ndarray:
    nb = BLOCK[qtype][1]
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    if raw.size % nb:
        raise ValueError(f"{raw.size} bytes is not a whole number of {nb}-byte blocks")
    return raw.reshape(-1, nb)


def dequant_q8_0(raw: np.ndarray) -> np.ndarray:
    b = _blocks(raw, Q8_0)
    d = _f16(b[:, 0:2])
    q = b[:, 2:34].view(np.int8).astype(np.float32)
    return (d[:, None] * q).reshape(-1)


def scale_min_k4(scales: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """[n, 12] packed bytes -> (sc, m), each [n, 8] (sub-block order)."""
    s = scales.astype(np.uint8)
    sc = np.empty(s.shape[:-1] + (8,), np.uint8)
    m = np.empty_like(sc)
    sc[..., :4] = s[..., 0:4] & 63
    m[..., :4] = s[..., 4:8] & 63
    sc[..., 4:] = (s[..., 8:12] & 15) | ((s[..., 0:4] >> 6) << 4)
    m[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
    return sc, m


def _k_affine(b: np.ndarray, q: np.ndarray) -> np.ndarray:
    """y = (d * sc) * q - (dmin * m) for q [n, 8, 32] in sub-block order."""
    d, dmin = _f16(b[:, 0:2]), _f16(b[:, 2:4])
    sc, m = scale_min_k4(b[:, 4:16])
    dsc = d[:, None] * sc.astype(np.float32)
    dm = dmin[:, None] * m.astype(np.float32)
    return (dsc[:, :, None] * q - dm[:, :, None]).reshape(-1)


def _nibbles_by_subblock(qs: np.ndarray) -> np.ndarray:
    """qs [n, 128] -> [n, 8, 32]: sub-block 2p = low nibbles of qs[32p:32p+32], 2p+1 = high."""
    q = qs.reshape(-1, 4, 32)
    return np.stack([q & 15, q >> 4], axis=2).reshape(-1, 8, 32)


def dequant_q4_k(raw: np.ndarray) -> np.ndarray:
    b = _blocks(raw, Q4_K)
    return _k_affine(b, _nibbles_by_subblock(b[:, 16:144]).astype(np.float32))


def dequant_q5_k(raw: np.ndarray) -> np.ndarray:
    b = _blocks(raw, Q5_K)
    lo = _nibbles_by_subblock(b[:, 48:176]).astype(np.int32)
    qh = b[:, 16:48].astype(np.int32)                                  # [n, 32]
    hi = np.stack([(qh >> s) & 1 for s in range(8)], axis=1)           # [n, 8, 32]
    return _k_affine(b, (lo + 16 * hi).astype(np.float32))


def dequant_q6_k(raw: np.ndarray) -> np.ndarray:
    b = _blocks(raw, Q6_K)
    ql = b[:, 0:128].reshape(-1, 2, 64).astype(np.int32)
    qh = b[:, 128:192].reshape(-1, 2, 32).astype(np.int32)
    sc = b[:, 192:208].view(np.int8).astype(np.float32)
    d = _f16(b[:, 208:210])
    q = np.empty((b.shape[0], 2, 4, 32), np.int32)                     # [n, half, quarter, l]
    for quarter in range(4):
        low = ql[:, :, 32 * (quarter & 1):32 * (quarter & 1) + 32]
        low = (low & 15) if quarter < 2 else (low >> 4)
        q[:, :, quarter, :] = low | (((qh >> (2 * quarter)) & 3) << 4)
    q = (q - 32).reshape(b.shape[0], 256).astype(np.float32)
    dsc = (d[:, None] * sc).repeat(16, axis=1)                          # scale of weight e: e // 16
    return (dsc * q).reshape(-1)


def dequant(raw: np.ndarray, qtype: int) -> np.ndarray:
    fn = {Q8_0: dequant_q8_0, Q4_K: dequant_q4_k, Q5_K: dequant_q5_k, Q6_K: dequant_q6_k}.get(int(qtype))
    if fn is None:
        raise ValueError(f"unsupported ggml type {qtype}")
    return fn(raw)


# ------------------------------------------------------------- packers
# Chosen per-weight quants and per-sub-block scales -> block bytes, written weight by
# weight from the layout description above (the inverse direction of the decoders).
def pack_q8_0(d: float, q: np.ndarray) -> np.ndarray:
    out = np.zeros(34, np.uint8)
    out[0:2] = np.array([d], np.float16).view(np.uint8)
    out[2:] = np.asarray(q, np.int8).view(np.uint8)
    return out


def pack_scale_min_k4(sc: list[int], m: list[int]) -> np.ndarray:
    out = np.zeros(12, np.uint8)
    for s in range(8):
        if s < 4:
            out[s] |= sc[s] & 63
            out[s + 4] |= m[s] & 63
        else:
            out[s + 4] |= (sc[s] & 15) | ((m[s] & 15) << 4)
            out[s - 4] |= (sc[s] >> 4) << 6
            out[s] |= (m[s] >> 4) << 6
    return out


def pack_q4_k(d: float, dmin: float, sc: list[int], m: list[int], q: np.ndarray, five: bool = False) -> np.ndarray:
    """q: 256 values (0..15, or 0..31 with five=True for Q5_K) in weight order."""
    nb = 176 if five else 144
    out = np.zeros(nb, np.uint8)
    out[0:2] = np.array([d], np.float16).view(np.uint8)
    out[2:4] = np.array([dmin], np.float16).view(np.uint8)
    out[4:16] = pack_scale_min_k4(sc, m)
    qs0 = 48 if five else 16
    for e in range(256):
        s, l = e // 32, e % 32
        p, hi = s // 2, s % 2
        v = int(q[e])
        out[qs0 + 32 * p + l] |= (v & 15) << (4 * hi)
        if five and v & 16:
            out[16 + l] |= 1 << s
    return out


def pack_q6_k(d: float, sc: list[int], q: np.ndarray) -> np.ndarray:
    """q: 256 values in -32..31 in weight order; sc: 16 int8 scales."""
    out = np.zeros(210, np.uint8)
    for e in range(256):
        n, quarter, l = e // 128, (e % 128) // 32, e % 32
        v = int(q[e]) + 32
        out[64 * n + l + 32 * (quarter & 1)] |= (v & 15) << (4 * (quarter >> 1))
        out[128 + 32 * n + l] |= (v >> 4) << (2 * quarter)
    out[192:208] = np.asarray(sc, np.int8).view(np.uint8)
    out[208:210] = np.array([d], np.float16).view(np.uint8)
    return out
