"""Known-answer superblocks for IQ4_XS and IQ3_XXS -> ``tests/golden/iq_kat.npz``.

The inputs are hand-built to isolate each field of the GGUF layouts (scale
nibbles and high bits, low vs high qs nibbles, grid indices, sign indices,
4-bit scales, subnormal / negative / zero d) plus a few random blocks.  The
expected outputs are computed here element by element in pure Python, with
Python floats (fp64, exact for these products), straight from the layout
descriptions in the reference (``npu/quant_mv_iq4.py:180-202``,
``npu/iq3_xxs.py:4-15, 64-90``) -- not from the vectorised oracle -- and
stored as float32 (exact, since every value fits in 24 significant bits).

The IQ3_XXS grid and kvalues come from ``ref_tables.npz`` (reference-held data).

    python tests/golden/make_kat.py
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
TABLES = np.load(HERE / "ref_tables.npz")
GRID = TABLES["iq3xxs_grid"].astype(int).tolist()          # [256][4]
KSIGNS_PM1 = TABLES["ksigns_pm1"].astype(int).tolist()     # [128][8]
KV = TABLES["kvalues_iq4nl"].astype(int).tolist()          # [16]


def f16(v: float) -> bytes:
    return struct.pack("<e", v)


def f16_val(b: bytes) -> float:
    return struct.unpack("<e", b)[0]


# ------------------------------------------------------------------ IQ4_XS
def iq4_block(d: float, scales_h: int, scales_l: list[int], qs: list[int]) -> bytes:
    assert len(scales_l) == 4 and len(qs) == 128
    return f16(d) + struct.pack("<H", scales_h) + bytes(scales_l) + bytes(qs)


def iq4_expected(blk: bytes) -> list[float]:
    d = f16_val(blk[0:2])
    sh = struct.unpack("<H", blk[2:4])[0]
    sl = list(blk[4:8])
    qs = list(blk[8:136])
    out = [0.0] * 256
    for s in range(8):
        low = (sl[s // 2] >> (4 * (s % 2))) & 15
        high = (sh >> (2 * s)) & 3
        ls = low | (high << 4)
        for j in range(16):
            q = qs[16 * s + j]
            out[32 * s + j] = d * (ls - 32) * KV[q & 15]
            out[32 * s + 16 + j] = d * (ls - 32) * KV[q >> 4]
    return out


def iq4_cases(rng: np.random.Generator) -> list[bytes]:
    cases = []
    # every nibble value in the low half and a different one in the high half, ls = 0 everywhere
    cases.append(iq4_block(1.0, 0, [0, 0, 0, 0], [(j % 16) | (((15 - j) % 16) << 4) for j in range(128)]))
    # each sub-block a distinct scale: ls_s = s (low nibbles only), qs nibble 8 (kv = 1)
    sl = [(0 | (1 << 4)), (2 | (3 << 4)), (4 | (5 << 4)), (6 | (7 << 4))]
    cases.append(iq4_block(0.5, 0, sl, [0x88] * 128))
    # high scale bits only: scales_h pattern 0b11_10_01_00_11_10_01_00
    cases.append(iq4_block(0.25, 0b1110010011100100, [0, 0, 0, 0], [0x98] * 128))
    # extremes ls = 63 (sl nibble 15, sh bits 3) and ls = 32 (zero scale)
    cases.append(iq4_block(1.0, 0xFFFF, [0xFF] * 4, [0xF0] * 128))
    cases.append(iq4_block(1.0, 0xAAAA, [0x00] * 4, [0x5A] * 128))
    # subnormal, negative and zero d
    cases.append(iq4_block(2.0 ** -24, 0x1234, [0x9C, 0x3E, 0x71, 0x05], list(range(128))))
    cases.append(iq4_block(-3.0e-3, 0x8421, [0x11, 0x22, 0x44, 0x88], list(range(255, 127, -1))))
    cases.append(iq4_block(0.0, 0xFFFF, [0xFF] * 4, [0xFF] * 128))
    # random blocks
    for _ in range(8):
        d = float(np.float16(abs(rng.standard_normal()) * 2e-3))
        cases.append(iq4_block(d, int(rng.integers(0, 65536)), rng.integers(0, 256, 4).tolist(),
                               rng.integers(0, 256, 128).tolist()))
    return cases


# ----------------------------------------------------------------- IQ3_XXS
def iq3_block(d: float, qs: list[int], words: list[int]) -> bytes:
    assert len(qs) == 64 and len(words) == 8
    return f16(d) + bytes(qs) + struct.pack("<8I", *words)


def iq3_expected(blk: bytes) -> list[float]:
    d = f16_val(blk[0:2])
    qs = list(blk[2:66])
    words = struct.unpack("<8I", blk[66:98])
    out = [0.0] * 256
    for s in range(8):
        w = words[s]
        db = d * (0.5 + (w >> 28)) * 0.5
        for g in range(4):
            signs = KSIGNS_PM1[(w >> (7 * g)) & 127]
            lanes = GRID[qs[8 * s + 2 * g]] + GRID[qs[8 * s + 2 * g + 1]]
            for i in range(8):
                out[32 * s + 8 * g + i] = db * signs[i] * lanes[i]
    return out


def iq3_word(sign_idx: list[int], scale: int) -> int:
    return sign_idx[0] | (sign_idx[1] << 7) | (sign_idx[2] << 14) | (sign_idx[3] << 21) | (scale << 28)


def iq3_cases(rng: np.random.Generator) -> list[bytes]:
    cases = []
    # every grid index once across 4 blocks, positive signs, scale 0
    for b in range(4):
        cases.append(iq3_block(1.0, list(range(64 * b, 64 * b + 64)), [iq3_word([0, 0, 0, 0], 0)] * 8))
    # every sign index once (128 = 8 sub-blocks x 4 groups x 4 blocks), grid index 0, all scales
    for b in range(4):
        words = [iq3_word([(32 * b + 4 * s + g) for g in range(4)], (4 * b + s) % 16) for s in range(8)]
        cases.append(iq3_block(0.75, [0] * 64, words))
    # scale 15 with the last grid point, subnormal / negative / zero d
    cases.append(iq3_block(1.0, [255] * 64, [iq3_word([127, 1, 64, 85], 15)] * 8))
    cases.append(iq3_block(2.0 ** -20, list(range(64)), [iq3_word([s, 2 * s, 3 * s, 4 * s], s) for s in range(8)]))
    cases.append(iq3_block(-1.5e-3, list(range(63, -1, -1)), [0xFFFFFFFF] * 8))
    cases.append(iq3_block(0.0, [17] * 64, [0x12345678] * 8))
    for _ in range(8):
        d = float(np.float16(abs(rng.standard_normal()) * 2e-3))
        cases.append(iq3_block(d, rng.integers(0, 256, 64).tolist(),
                               [int(v) for v in rng.integers(0, 2 ** 32, 8, dtype=np.uint64)]))
    return cases


def main() -> None:
    rng = np.random.Generator(np.random.PCG64(20261201))
    iq4 = iq4_cases(rng)
    iq3 = iq3_cases(rng)
    np.savez(
        HERE / "iq_kat.npz",
        iq4_blocks=np.frombuffer(b"".join(iq4), dtype=np.uint8).reshape(len(iq4), 136),
        iq4_expected=np.array([iq4_expected(b) for b in iq4], dtype=np.float32),
        iq3_blocks=np.frombuffer(b"".join(iq3), dtype=np.uint8).reshape(len(iq3), 98),
        iq3_expected=np.array([iq3_expected(b) for b in iq3], dtype=np.float32),
    )
    print(f"wrote {HERE / 'iq_kat.npz'}: {len(iq4)} IQ4_XS + {len(iq3)} IQ3_XXS blocks")


if __name__ == "__main__":
    main()
