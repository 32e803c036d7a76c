"""Extract the codebook tables that the reference repository itself holds into
small numeric fixtures.

Run in the build container only (it reads ``/root/reference``); its outputs are
committed so nothing at test time needs the reference tree:

    python tests/golden/make_table_fixtures.py

Sources (all reference-held data, parsed as text, nothing imported):

* ``npu/iq3_xxs_tables.h:5-262``   -- ``IQ3_XXS_GRID[256*4]`` (fp32 text, written
  by ``npu/quant_mv.py:52-71`` from gguf-py 0.18.0's ``IQ3_XXS.grid``).
* ``npu/iq3_xxs_tables.h:263-392`` -- ``IQ3_XXS_KSIGNS_FP[128*8]`` (+1/-1 text,
  from gguf-py's ``IQ2_XXS.ksigns``).
* ``npu/quant_mv_iq4.py:194-197`` and ``npu/quant_mv_iq4_packed.py:35-39`` --
  the ``kvalues_iq4nl`` literal (both copies must agree).

Output: ``tests/golden/ref_tables.npz`` with arrays
``iq3xxs_grid`` (uint8 [256,4]), ``ksigns_pm1`` (int8 [128,8]) and
``kvalues_iq4nl`` (int8 [16]).
"""
from __future__ import annotations

import re
from pathlib import Path

import numpy as np

REF = Path("/root/reference")
OUT = Path(__file__).with_name("ref_tables.npz")


def _c_array_body(text: str, name: str) -> list[float]:
    m = re.search(re.escape(name) + r"\s*\[[^\]]*\]\s*=\s*\{(.*?)\};", text, re.S)
    if m is None:
        raise ValueError(f"array {name} not found")
    vals = re.findall(r"[-+]?\d+\.\d+f", m.group(1))
    return [float(v[:-1]) for v in vals]


def _kvalues_literal(path: Path, anchor: str) -> list[int]:
    text = path.read_text()
    i = text.index(anchor)
    m = re.search(r"\[([-\d,\s]+)\]", text[i:])
    if m is None:
        raise ValueError(f"kvalues literal not found in {path}")
    return [int(v) for v in m.group(1).replace("\n", " ").split(",") if v.strip()]


def main() -> None:
    hdr = (REF / "npu" / "iq3_xxs_tables.h").read_text()
    grid = np.array(_c_array_body(hdr, "IQ3_XXS_GRID"), dtype=np.float64)
    ks = np.array(_c_array_body(hdr, "IQ3_XXS_KSIGNS_FP"), dtype=np.float64)
    if grid.size != 1024 or ks.size != 1024:
        raise ValueError(f"unexpected table sizes {grid.size} {ks.size}")
    if not np.all(grid == np.round(grid)) or grid.min() < 0 or grid.max() > 255:
        raise ValueError("grid entries are not small non-negative integers")
    if not np.all(np.abs(ks) == 1.0):
        raise ValueError("ksigns entries are not +-1")
    kv_a = _kvalues_literal(REF / "npu" / "quant_mv_iq4.py", "kvalues = np.array(")
    kv_b = _kvalues_literal(REF / "npu" / "quant_mv_iq4_packed.py", "_KVALUES = np.array(")
    if kv_a != kv_b or len(kv_a) != 16:
        raise ValueError(f"kvalues literals disagree: {kv_a} vs {kv_b}")
    np.savez(
        OUT,
        iq3xxs_grid=grid.reshape(256, 4).astype(np.uint8),
        ksigns_pm1=ks.reshape(128, 8).astype(np.int8),
        kvalues_iq4nl=np.array(kv_a, dtype=np.int8),
    )
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
