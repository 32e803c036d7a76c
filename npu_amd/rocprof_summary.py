"""Summaries of rocprofv3 output for the MoE-block kernels (the files under profiles/).

Reads a ``--kernel-trace --stats`` kernel-stats CSV and four ``--pmc`` counter CSVs
(FETCH_SIZE and WRITE_SIZE, KiB per dispatch, each for the workload and for a plain
copy kernel of known size) and writes

* ``hbm_traffic.json`` -- per kernel: rocprof average duration, counter means, the
  copy-calibrated HBM bytes per launch and the algorithmic bytes per launch;
* ``<name>.md`` -- the same as a table, with the commands that produced the inputs.

With ``--inst-pmc I.csv`` it instead tabulates, per kernel, rocprof durations and the
instruction counters of one ``--pmc`` pass (``SQ_WAVES``, ``SQ_INSTS_VALU``,
``SQ_INSTS_SALU``, ``SQ_INSTS_LDS``, ``SQ_INSTS_VMEM_RD``: device totals per dispatch),
with the VALU issue time they imply (``<name>.md``).

With ``--durations`` it tabulates the kernel-stats CSV alone (optionally per unit of
work, ``--per``).

With ``--trace T.csv`` it tabulates durations per kernel and launch shape (grid size)
from a kernel trace; ``--grid-pmc`` counter CSVs add, per shape, the copy-calibrated
HBM bytes (FETCH_SIZE / WRITE_SIZE) and instruction counts per wave.

With ``--prefill-pmc P.csv`` it instead summarises the prefill kernels: rocprof
durations and, from the counters ``MfmaUtil``, ``MfmaFlopsF16`` and ``MfmaFlopsBF16``
(one ``--pmc`` pass), each kernel's MFMA busy fraction and issued MFMA TFLOP/s
against the 2.5 PFLOP/s dense f16/bf16 peak (``<name>.md`` and ``prefill_mfma.json``).

Calibration: the copy kernel moves ``calib_bytes`` each way per launch, so
``scale = calib_bytes / (counter KiB * 1024)`` for each counter; a kernel's HBM bytes
per launch are ``FETCH * 1024 * scale_fetch + WRITE * 1024 * scale_write``.

    python -m npu_amd.rocprof_summary --stats S.csv --fetch F.csv --write W.csv \\
        --calib-fetch CF.csv --calib-write CW.csv --calib-bytes 268435456 --out profiles
"""
from __future__ import annotations

import argparse
import csv
import json
import statistics
from collections import defaultdict
from pathlib import Path

# Config-5 block shape (BASELINE configs 3 and 5).
D, FF, E, K = 2048, 512, 256, 8


def algorithmic_bytes(d: int = D, ff: int = FF, e: int = E, k: int = K) -> dict[str, int]:
    """Bytes each T = 1 decode kernel must move at least once (weights read, activations
    read once, outputs written once), for a block with IQ4_XS gate/up, IQ3_XXS down, the
    shared expert in the same formats, an RMSNorm weight and a shared scalar gate.  The
    router accumulators are 8 copies of e + 2 fp64 words (raw router dot products, the
    shared gate's, the sum of x^2) in runs of 4 x 64 + 16 words at e <= 256.
      k_dec_router1: router [e, d] bf16, shared scalar gate [d] bf16, x and the RMSNorm
        weight fp32; writes the 8 accumulator copies (copy 0 and zeros).
      k_dec_gateup1w: the k routed and the shared experts' gate and up rows, x and the
        RMSNorm weight (the limb row is built in LDS), the 8 accumulator copies; writes
        k + 1 SwiGLU rows [ff] fp32, the logits, the ids and weights and the shared gate.
      k_dec_down1: the k routed and the shared down rows, the k + 1 SwiGLU rows, the
        weights, the shared gate and x (residual); writes y [d].
      k_dec_down1 in a chain (k_dec_down1_next): also the next layer's router and shared
        gate [e + 1, d] bf16 (router_t) and RMSNorm weight, and one fp64 atomic per
        accumulator word per block of 8 rows (d / 8 blocks)."""
    iq4_row, iq3_row = d // 256 * 136, ff // 256 * 98
    acc = 8 * (e + 2) * 8                      # the words read; the runs are padded to whole lines
    down = (k + 1) * d * iq3_row + (k + 1) * ff * 4 + k * 4 + 4 + d * 4 + d * 4
    return {
        "k_dec_router1": e * d * 2 + d * 2 + d * 4 + d * 4 + acc,
        "k_dec_gateup1w": (k + 1) * 2 * ff * iq4_row + d * 4 + d * 4 + acc + (k + 1) * ff * 4 + e * 4
                          + 2 * k * 4 + 4,
        "k_dec_down1": down,
        "k_dec_down1_next": down + (e + 1) * d * 2 + d * 4 + d // 8 * (e + 2) * 8,
    }


def short(name: str) -> str:
    """Kernel name without return type, namespaces in parentheses and arguments."""
    base = name.replace("(anonymous namespace)::", "")
    if base.startswith("void "):
        base = base[5:]
    return base.split("(")[0].strip()


def family(name: str) -> str:
    return short(name).split("<")[0]


def counter_means(path: str) -> dict[str, float]:
    vals: dict[str, list[float]] = defaultdict(list)
    with open(path) as f:
        for r in csv.DictReader(f):
            vals[short(r["Kernel_Name"])].append(float(r["Counter_Value"]))
    return {k: statistics.fmean(v) for k, v in vals.items()}


def kernel_stats(path: str) -> dict[str, dict]:
    out = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            out[short(r["Name"])] = {"calls": int(r["Calls"]), "avg_us": float(r["AverageNs"]) / 1e3,
                                     "min_us": float(r["MinNs"]) / 1e3, "max_us": float(r["MaxNs"]) / 1e3}
    return out


MFMA_PEAK_TFLOPS = 2500.0      # dense f16 / bf16 MFMA, MI355X


def counter_table(path: str) -> dict[str, dict[str, float]]:
    """Per kernel instance and counter: mean over dispatches."""
    vals: dict[str, dict[str, list[float]]] = defaultdict(lambda: defaultdict(list))
    with open(path) as f:
        for r in csv.DictReader(f):
            vals[short(r["Kernel_Name"])][r["Counter_Name"]].append(float(r["Counter_Value"]))
    return {k: {c: statistics.fmean(v) for c, v in d.items()} for k, d in vals.items()}


def prefill_summary(a) -> None:
    stats = kernel_stats(a.stats)
    pmc = counter_table(a.prefill_pmc)
    kernels = {}
    for name, st in stats.items():
        if not (family(name).startswith(("k_pf_", "k_pfs_")) or family(name) == "k_dispatch"):
            continue
        c = pmc.get(name, {})
        flops = c.get("MfmaFlopsF16", 0.0) + c.get("MfmaFlopsBF16", 0.0)
        tflops = flops / (st["avg_us"] * 1e-6) / 1e12
        kernels[name] = {"calls": st["calls"], "rocprof_avg_us": st["avg_us"],
                         "mfma_util_pct": c.get("MfmaUtil"), "mfma_flops_per_launch": flops,
                         "mfma_TFLOPs_at_rocprof_avg": tflops, "frac_of_dense_peak": tflops / MFMA_PEAK_TFLOPS}
    out = Path(a.out)
    out.mkdir(parents=True, exist_ok=True)
    (out / "prefill_mfma.json").write_text(json.dumps({"peak_TFLOPs": MFMA_PEAK_TFLOPS, "kernels": kernels},
                                                      indent=1) + "\n")
    total = sum(k["rocprof_avg_us"] * k["calls"] for k in kernels.values())
    lines = [f"# {a.name}: prefill kernel durations and MFMA use", "", a.commands, "",
             "| kernel | calls | rocprof avg us | share of prefill time | MfmaUtil % | MFMA GFLOP/launch | "
             "MFMA TFLOP/s | of 2.5 PF dense |", "|---|---|---|---|---|---|---|---|"]
    for name, k in sorted(kernels.items(), key=lambda kv: -kv[1]["rocprof_avg_us"]):
        util = "-" if k["mfma_util_pct"] is None else f"{k['mfma_util_pct']:.1f}"
        lines.append(f"| {name[:60]} | {k['calls']} | {k['rocprof_avg_us']:.2f} | "
                     f"{k['rocprof_avg_us'] * k['calls'] / total:.3f} | {util} | "
                     f"{k['mfma_flops_per_launch'] / 1e9:.3f} | {k['mfma_TFLOPs_at_rocprof_avg']:.1f} | "
                     f"{k['frac_of_dense_peak']:.4f} |")
    (out / f"{a.name}.md").write_text("\n".join(lines) + "\n")
    print(json.dumps(kernels, indent=1))


def inst_summary(a) -> None:
    """Durations and instruction counters per kernel family of the decode chain.  A wave64
    VALU instruction occupies a 16-lane SIMD for 4 cycles, so the VALU issue time of a
    dispatch is at least VALU instructions x 4 / (SIMDs x clock)."""
    stats = kernel_stats(a.stats)
    pmc = counter_table(a.inst_pmc)
    lines = [f"# {a.name}: kernel durations and instruction counts", "", a.commands, "",
             "Counters are device totals per dispatch (mean over dispatches). VALU issue time = "
             f"SQ_INSTS_VALU x 4 cycles / ({a.simds} SIMDs x {a.sclk_ghz} GHz): the time the kernel needs "
             "if every SIMD issued a VALU instruction every 4 cycles.", "",
             "| kernel | calls | rocprof avg us | waves | VALU / wave | SALU / wave | LDS / wave | VMEM rd / wave | "
             "VALU issue us |", "|---|---|---|---|---|---|---|---|---|"]
    for name, st in sorted(stats.items(), key=lambda kv: -kv[1]["calls"] * kv[1]["avg_us"]):
        c = pmc.get(name)
        if not c or "SQ_WAVES" not in c or c["SQ_WAVES"] <= 0:
            continue
        w = c["SQ_WAVES"]
        valu_us = c.get("SQ_INSTS_VALU", 0.0) * 4 / (a.simds * a.sclk_ghz * 1e3)
        lines.append(f"| {name[:60]} | {st['calls']} | {st['avg_us']:.2f} | {w:.0f} | "
                     f"{c.get('SQ_INSTS_VALU', 0) / w:.0f} | {c.get('SQ_INSTS_SALU', 0) / w:.0f} | "
                     f"{c.get('SQ_INSTS_LDS', 0) / w:.0f} | {c.get('SQ_INSTS_VMEM_RD', 0) / w:.0f} | {valu_us:.2f} |")
    out = Path(a.out)
    out.mkdir(parents=True, exist_ok=True)
    (out / f"{a.name}.md").write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


def durations(a) -> None:
    """Durations per kernel from a ``--kernel-trace --stats`` kernel-stats CSV (kernels whose
    name contains ``--kernel`` only), with each kernel's total per unit of work when
    ``--per N`` gives the units the run timed (e.g. decode steps)."""
    stats = kernel_stats(a.stats)
    rows = [(n, st) for n, st in stats.items() if not a.kernel or a.kernel in n]
    rows.sort(key=lambda kv: -kv[1]["calls"] * kv[1]["avg_us"])
    head = "| kernel | calls | avg us | min us | max us |" + (" us per unit |" if a.per else "")
    lines = [f"# {a.name}: kernel durations", "", a.commands, "", head,
             "|---|---|---|---|---|" + ("---|" if a.per else "")]
    total = 0.0
    for n, st in rows:
        per = st["calls"] * st["avg_us"] / a.per if a.per else None
        total += per or 0.0
        lines.append(f"| {n[:70]} | {st['calls']} | {st['avg_us']:.2f} | {st['min_us']:.2f} | {st['max_us']:.2f} |"
                     + (f" {per:.1f} |" if per is not None else ""))
    if a.per:
        lines += ["", f"Sum over the listed kernels: {total:.1f} us per unit ({a.per} units)."]
    out = Path(a.out)
    out.mkdir(parents=True, exist_ok=True)
    (out / f"{a.name}.md").write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


def trace_by_grid(a) -> None:
    """Per kernel and launch shape (grid size): dispatches and duration statistics from a
    ``--kernel-trace`` CSV, for runs that launch one kernel at several sizes."""
    rows: dict[tuple[str, int], list[float]] = defaultdict(list)
    with open(a.trace) as f:
        for r in csv.DictReader(f):
            name = short(r["Kernel_Name"])
            if a.kernel and a.kernel not in name:
                continue
            grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
            rows[(name, grid)].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    pmc: dict[tuple[str, int], dict[str, list[float]]] = defaultdict(lambda: defaultdict(list))
    for path in a.grid_pmc:
        with open(path) as f:
            for r in csv.DictReader(f):
                name = short(r["Kernel_Name"])
                if a.kernel and a.kernel not in name:
                    continue
                pmc[(name, int(r["Grid_Size"]))][r["Counter_Name"]].append(float(r["Counter_Value"]))
    s_fetch = s_write = 1.0
    if a.calib_fetch and a.calib_write:
        s_fetch = a.calib_bytes / (counter_means(a.calib_fetch)[a.calib_kernel] * 1024)
        s_write = a.calib_bytes / (counter_means(a.calib_write)[a.calib_kernel] * 1024)
    algo = {}
    for kv in a.algo:
        key, b = kv.rsplit("=", 1)
        kern, grid = key.rsplit("@", 1)
        algo[(kern, int(grid))] = int(b)
    head = "| kernel | grid (work-items) | dispatches | avg us | median us | min us | max us |"
    rule = "|---|---|---|---|---|---|---|"
    if pmc:
        head += (" HBM bytes/dispatch | algorithmic bytes | traffic/algorithmic | waves | VALU / wave | SALU / wave |"
                 " LDS / wave | VMEM rd / wave |")
        rule += "---|---|---|---|---|---|---|---|"
    lines = [f"# {a.name}: kernel durations by launch shape", "", a.commands, ""]
    if pmc and a.calib_fetch:
        lines += [f"HBM bytes = FETCH_SIZE x 1024 x {s_fetch:.4f} + WRITE_SIZE x 1024 x {s_write:.4f} (the scales "
                  f"make a {a.calib_bytes} B {a.calib_kernel} read as that many bytes each way); instruction "
                  "counts are device totals per dispatch over SQ_WAVES.", ""]
    lines += [head, rule]

    def fmt(x, spec):
        return "-" if x is None else format(x, spec)
    for (name, grid), d in sorted(rows.items()):
        line = (f"| {name[:80]} | {grid} | {len(d)} | {statistics.fmean(d):.2f} | {statistics.median(d):.2f} | "
                f"{min(d):.2f} | {max(d):.2f} |")
        if pmc:
            c = {k: statistics.fmean(v) for k, v in pmc.get((name, grid), {}).items()}
            hbm = None
            if "FETCH_SIZE" in c:
                hbm = c["FETCH_SIZE"] * 1024 * s_fetch + c.get("WRITE_SIZE", 0.0) * 1024 * s_write
            alg = next((b for (k, g), b in algo.items() if g == grid and k in name), None)
            ratio = hbm / alg if hbm is not None and alg else None
            w = c.get("SQ_WAVES")
            per = (lambda key: c[key] / w if w and key in c else None)
            line += (f" {fmt(hbm, '.0f')} | {fmt(alg, 'd')} | {fmt(ratio, '.3f')} | {fmt(w, '.0f')} | "
                     f"{fmt(per('SQ_INSTS_VALU'), '.0f')} | {fmt(per('SQ_INSTS_SALU'), '.0f')} | "
                     f"{fmt(per('SQ_INSTS_LDS'), '.0f')} | {fmt(per('SQ_INSTS_VMEM_RD'), '.0f')} |")
        lines.append(line)
    out = Path(a.out)
    out.mkdir(parents=True, exist_ok=True)
    (out / f"{a.name}.md").write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--trace", help="kernel-trace CSV: durations per kernel and grid size (trace mode)")
    ap.add_argument("--kernel", default="", help="trace mode: only kernels whose name contains this")
    ap.add_argument("--grid-pmc", action="append", default=[],
                    help="trace mode: counter CSV whose means per kernel and grid size become columns "
                         "(FETCH_SIZE / WRITE_SIZE, SQ_WAVES / SQ_INSTS_*; repeatable)")
    ap.add_argument("--stats")
    ap.add_argument("--prefill-pmc", help="counter CSV of MfmaUtil/MfmaFlopsF16/MfmaFlopsBF16 (prefill mode)")
    ap.add_argument("--inst-pmc", help="counter CSV of SQ_WAVES/SQ_INSTS_* (instruction mode)")
    ap.add_argument("--simds", type=int, default=1024, help="SIMDs of the device (256 CUs x 4 on MI355X)")
    ap.add_argument("--sclk-ghz", type=float, default=2.4, help="shader clock for the VALU issue time")
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--calib-fetch")
    ap.add_argument("--calib-write")
    ap.add_argument("--calib-bytes", type=int, default=256 << 20)
    ap.add_argument("--calib-kernel", default="__amd_rocclr_copyBuffer")
    ap.add_argument("--out", default="profiles")
    ap.add_argument("--name", default="moe_decode_config5")
    ap.add_argument("--commands", default="", help="text describing the commands (markdown)")
    ap.add_argument("--algo", action="append", default=[],
                    help="KERNEL=BYTES: algorithmic bytes per launch of a kernel family (replaces the "
                         "T = 1 decode table; repeatable); in trace mode KERNEL@GRID=BYTES")
    ap.add_argument("--json", default="hbm_traffic.json", help="name of the JSON written to --out")
    ap.add_argument("--durations", action="store_true",
                    help="durations mode: the kernel-stats table of --stats (filter --kernel, units --per)")
    ap.add_argument("--per", type=float, default=0.0, help="durations mode: units of work the run timed")
    a = ap.parse_args()
    if a.trace:
        trace_by_grid(a)
        return
    if not a.stats:
        ap.error("--stats is required outside trace mode")
    if a.durations:
        durations(a)
        return
    if a.prefill_pmc:
        prefill_summary(a)
        return
    if a.inst_pmc:
        inst_summary(a)
        return
    if not (a.fetch and a.write and a.calib_fetch and a.calib_write):
        ap.error("decode mode needs --fetch, --write, --calib-fetch and --calib-write")

    stats = kernel_stats(a.stats)
    fetch, write = counter_means(a.fetch), counter_means(a.write)
    cf, cw = counter_means(a.calib_fetch)[a.calib_kernel], counter_means(a.calib_write)[a.calib_kernel]
    s_fetch, s_write = a.calib_bytes / (cf * 1024), a.calib_bytes / (cw * 1024)
    algo = dict((kv.split("=")[0], int(kv.split("=")[1])) for kv in a.algo) if a.algo else algorithmic_bytes()
    kernels = {}
    for name, st in stats.items():
        fam = family(name)
        if fam not in algo or name not in fetch:
            continue
        hbm = fetch[name] * 1024 * s_fetch + write.get(name, 0.0) * 1024 * s_write
        kernels[fam] = {
            "instance": name, "calls": st["calls"], "rocprof_avg_us": st["avg_us"],
            "fetch_kib": fetch[name], "write_kib": write.get(name, 0.0),
            "hbm_bytes_per_launch": round(hbm), "algorithmic_bytes_per_launch": algo[fam],
            "traffic_over_algorithmic": hbm / algo[fam],
            "algorithmic_GBps_at_rocprof_avg": algo[fam] / (st["avg_us"] * 1e-6) / 1e9,
        }
    out = Path(a.out)
    out.mkdir(parents=True, exist_ok=True)
    doc = {"calibration": {"kernel": a.calib_kernel, "bytes_each_way": a.calib_bytes, "fetch_kib": cf,
                           "write_kib": cw, "fetch_scale": s_fetch, "write_scale": s_write},
           "kernels": kernels}
    (out / a.json).write_text(json.dumps(doc, indent=1) + "\n")
    lines = [f"# {a.name}: kernel durations and HBM traffic", "", a.commands, "",
             f"Copy calibration ({a.calib_kernel}, {a.calib_bytes} B each way): FETCH_SIZE reads "
             f"{cf:.1f} KiB (scale {s_fetch:.4f}), WRITE_SIZE {cw:.1f} KiB (scale {s_write:.4f}).", "",
             "| kernel | calls | rocprof avg us | FETCH KiB | WRITE KiB | HBM bytes/launch | algorithmic bytes | "
             "traffic/algorithmic | algorithmic GB/s |", "|---|---|---|---|---|---|---|---|---|"]
    for fam, k in kernels.items():
        lines.append(f"| {k['instance']} | {k['calls']} | {k['rocprof_avg_us']:.2f} | {k['fetch_kib']:.1f} | "
                     f"{k['write_kib']:.1f} | {k['hbm_bytes_per_launch']} | {k['algorithmic_bytes_per_launch']} | "
                     f"{k['traffic_over_algorithmic']:.3f} | {k['algorithmic_GBps_at_rocprof_avg']:.1f} |")
    lines += ["", "All kernels (rocprof --stats):", "", "| kernel | calls | avg us | min us | max us |",
              "|---|---|---|---|---|"]
    for name, st in sorted(stats.items(), key=lambda kv: -kv[1]["calls"] * kv[1]["avg_us"])[:16]:
        lines.append(f"| {name[:90]} | {st['calls']} | {st['avg_us']:.2f} | {st['min_us']:.2f} | {st['max_us']:.2f} |")
    (out / f"{a.name}.md").write_text("\n".join(lines) + "\n")
    print(json.dumps(kernels, indent=1))


if __name__ == "__main__":
    main()
