"""Pin the oracle's IQ4_XS / IQ3_XXS dequant against known answers and closed forms."""
import struct
from pathlib import Path

import numpy as np
import pytest

from oracle import quants as Q
from oracle import tables

ROOT = Path(__file__).resolve().parents[1]
KAT = np.load(ROOT / "tests" / "golden" / "iq_kat.npz")
KV = tables.kvalues_iq4nl().astype(np.float64)
GRID = tables.iq3xxs_grid().astype(np.float64)


def test_kat_iq4_xs():
    got = Q.dequant_iq4_xs(KAT["iq4_blocks"]).reshape(-1, 256)
    assert np.array_equal(got, KAT["iq4_expected"])


def test_kat_iq3_xxs():
    got = Q.dequant_iq3_xxs(KAT["iq3_blocks"]).reshape(-1, 256)
    assert np.array_equal(got, KAT["iq3_expected"])


def _iq4(d, sh, sl, qs):
    return np.frombuffer(struct.pack("<e", d) + struct.pack("<H", sh) + bytes(sl) + bytes(qs), np.uint8)


def test_iq4_brute_force_scale_and_nibble():
    """Every 6-bit scale x every nibble, in both nibble positions and all 8 sub-blocks."""
    d = 0.125
    for ls in range(64):
        lo, hi = ls & 15, ls >> 4
        sl = [lo | (lo << 4)] * 4
        sh = sum(hi << (2 * s) for s in range(8))
        for n in range(16):
            other = (n + 5) % 16
            y = Q.dequant_iq4_xs(_iq4(d, sh, sl, [n | (other << 4)] * 128)).reshape(8, 32)
            assert np.all(y[:, :16] == d * (ls - 32) * KV[n])
            assert np.all(y[:, 16:] == d * (ls - 32) * KV[other])


def test_iq4_subblock_scale_isolation():
    """A scale nibble or high-bit pair changes exactly one sub-block."""
    base = dict(d=1.0, sh=0, sl=[0, 0, 0, 0], qs=[0x88] * 128)
    ref = Q.dequant_iq4_xs(_iq4(**base)).reshape(8, 32)
    for s in range(8):
        sl = [0, 0, 0, 0]
        sl[s // 2] = 1 << (4 * (s % 2))
        y = Q.dequant_iq4_xs(_iq4(1.0, 0, sl, [0x88] * 128)).reshape(8, 32)
        changed = np.nonzero(np.any(y != ref, axis=1))[0].tolist()
        assert changed == [s] and np.all(y[s] == -31.0)
        y = Q.dequant_iq4_xs(_iq4(1.0, 1 << (2 * s), [0] * 4, [0x88] * 128)).reshape(8, 32)
        changed = np.nonzero(np.any(y != ref, axis=1))[0].tolist()
        assert changed == [s] and np.all(y[s] == 16.0 - 32.0)


def test_iq4_qs_position():
    """qs byte j of sub-block s drives weights 32s+j (low nibble) and 32s+16+j (high)."""
    for s in (0, 3, 7):
        for j in (0, 7, 15):
            qs = [0x88] * 128
            qs[16 * s + j] = 0xF0          # low nibble 0 (-127), high nibble 15 (113)
            y = Q.dequant_iq4_xs(_iq4(1.0, 0x5555, [0] * 4, qs))   # high bits 01 -> ls 16 -> scale -16
            diff = np.nonzero(y != -16.0)[0].tolist()
            assert diff == [32 * s + j, 32 * s + 16 + j]
            assert y[32 * s + j] == -16.0 * -127 and y[32 * s + 16 + j] == -16.0 * 113


def _iq3(d, qs, words):
    return np.frombuffer(struct.pack("<e", d) + bytes(qs) + struct.pack("<8I", *words), np.uint8)


def test_iq3_brute_force_grid_sign_scale():
    """Every grid index x sign index x scale, against grid * sign * d * (0.5 + ls) / 2."""
    signs = tables.ksigns_pm1().astype(np.float64)
    for ls in range(16):
        for sidx in range(128):
            w = sidx | (sidx << 7) | (sidx << 14) | (sidx << 21) | (ls << 28)
            for g0 in range(0, 256, 64):
                qs = [(g0 + i) % 256 for i in range(64)]
                y = Q.dequant_iq3_xxs(_iq3(0.5, qs, [w] * 8)).reshape(8, 4, 8)
                db = 0.5 * (0.5 + ls) * 0.5
                q = np.array(qs).reshape(8, 4, 2)
                want = db * signs[sidx][None, None, :] * np.concatenate([GRID[q[..., 0]], GRID[q[..., 1]]], -1)
                assert np.array_equal(y, want.astype(np.float32))


def test_iq3_ksigns_parity_bit_drives_lane7():
    w_odd = 1       # one explicit sign bit -> parity bit set -> lanes 0 and 7 negative
    y = Q.dequant_iq3_xxs(_iq3(1.0, [0] * 64, [w_odd] * 8)).reshape(8, 32)
    assert y[0, 0] < 0 and y[0, 7] < 0 and np.all(y[0, 1:7] > 0) and np.all(y[0, 8:] > 0)


@pytest.mark.parametrize("qtype", [Q.GGML_IQ4_XS, Q.GGML_IQ3_XXS])
def test_dequant_is_exact_product(qtype):
    """Random blocks: each fp32 output equals the fp64 product of its fields."""
    from npu_amd import synth
    g = np.random.Generator(np.random.PCG64(7))
    blocks = synth.host_superblocks(g, qtype, 64)
    y = Q.dequant(blocks, qtype).astype(np.float64)
    assert np.all(np.isfinite(y))
    assert np.array_equal(y.astype(np.float32).astype(np.float64), y)


def test_dequant_matrix_layout():
    from npu_amd import synth
    g = np.random.Generator(np.random.PCG64(3))
    w = synth.host_quant_matrix(g, Q.GGML_IQ3_XXS, 4, 512)
    full = Q.dequant_matrix(w, Q.GGML_IQ3_XXS, 4, 512)
    for r in range(4):
        assert np.array_equal(full[r], Q.dequant_iq3_xxs(w[r]))
    with pytest.raises(ValueError):
        Q.dequant_matrix(w, Q.GGML_IQ3_XXS, 4, 500)
