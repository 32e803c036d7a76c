"""Codebooks: oracle tables and the device header against the reference-held data."""
import re
from pathlib import Path

import numpy as np

from oracle import tables

ROOT = Path(__file__).resolve().parents[1]
FIX = np.load(ROOT / "tests" / "golden" / "ref_tables.npz")


def test_oracle_grid_matches_reference_header():
    assert np.array_equal(tables.iq3xxs_grid(), FIX["iq3xxs_grid"])


def test_grid_codes_sorted_and_magnitudes():
    codes = np.asarray(tables.IQ3XXS_GRID_CODES)
    assert codes.size == 256
    assert np.all(np.diff(codes) > 0), "gguf-py's grid is a strictly increasing list of points"
    assert set(np.unique(FIX["iq3xxs_grid"]).tolist()) == set(tables.IQ3XXS_GRID_MAP)


def test_ksigns_matches_reference_and_parity():
    assert np.array_equal(tables.ksigns_pm1(), FIX["ksigns_pm1"])
    b = tables.ksigns_bytes()
    assert all(bin(int(v)).count("1") % 2 == 0 for v in b), "every ksigns byte has even popcount"
    assert np.array_equal(b & 0x7F, np.arange(128))


def test_kvalues_match_reference_literal():
    kv = tables.kvalues_iq4nl()
    assert np.array_equal(kv, FIX["kvalues_iq4nl"])
    assert np.all(np.diff(kv.astype(int)) > 0)


def test_device_header_tables_match_reference():
    text = (ROOT / "npu_amd" / "csrc" / "iq_tables.h").read_text()
    grid_txt = text.split("#define GM_IQ3XXS_GRID_INIT", 1)[1].split("#define", 1)[0]
    words = [int(v, 16) for v in re.findall(r"0x([0-9a-f]{8})u", grid_txt)]
    assert len(words) == 256
    grid = np.array([[(w >> (8 * j)) & 0xFF for j in range(4)] for w in words], dtype=np.uint8)
    assert np.array_equal(grid, FIX["iq3xxs_grid"])
    kv_txt = text.split("#define GM_IQ4NL_PACKED_INIT", 1)[1]
    kw = [int(v, 16) for v in re.findall(r"0x([0-9a-f]{8})u", kv_txt)][:4]
    kv = np.array([(w >> (8 * j)) & 0xFF for w in kw for j in range(4)], dtype=np.uint8).view(np.int8)
    assert np.array_equal(kv, FIX["kvalues_iq4nl"])
