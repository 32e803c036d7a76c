"""Per-block timeline of the decode kernels over a chain of config-5 blocks.

The profiling build (``python -m npu_amd.build --timeline`` -> libnpu_amd_tl.so)
has every decode kernel write, from thread 0 of each block, the chip-wide
100 MHz ``s_memrealtime`` counter at block entry, at two kernel-specific marks
and at the end, into the layer's own workspace (csrc/timeline.h).  This script
replays the config-5 chain (40 blocks, T = 1 or 8, hipGraph, as bench.py does)
and summarises, per kernel and relative to the start of each block's first
kernel: when blocks enter, reach each mark and end, and the gaps between the
last block of one kernel ending and the first block of the next entering.

    python -m npu_amd.build --timeline
    NPU_AMD_LIB=timeline python -m npu_amd.timeline [--layers 40] [--T 1] [--chain] [--out FILE]
"""
from __future__ import annotations

import argparse
import os
import statistics
import sys

os.environ.setdefault("NPU_AMD_LIB", "timeline")

TICK_US = 0.01            # s_memrealtime runs at 100 MHz
N_SLOTS, MAXB, REC = 8, 2560, 8
SEED = 20261201


def _layer_records(blk, T: int):
    """[slot] -> list of (entry, mark1, mark2, end, hwid, clock0, clock1) for the blocks that wrote one."""
    import torch
    from npu_amd import ops
    need = ops.moe_workspace_bytes(blk.struct, T)
    nbytes = N_SLOTS * MAXB * REC * 8
    raw = blk.workspace(T)[need - nbytes:need].view(torch.int64).view(N_SLOTS, MAXB, REC).cpu().numpy()
    out = []
    for s in range(N_SLOTS):
        rows = raw[s]
        out.append([tuple(int(v) for v in r[:8]) for r in rows if r[0] != 0])
    return out


def _zero_records(blk, T: int) -> None:
    from npu_amd import ops
    need = ops.moe_workspace_bytes(blk.struct, T)
    blk.workspace(T)[need - N_SLOTS * MAXB * REC * 8:need].zero_()


def run(n_layers: int, T: int, replays: int, chain: bool = False):
    import torch
    from npu_amd import _lib, synth
    if not _lib.LIB_PATH.name.endswith("_tl.so"):
        raise RuntimeError("set NPU_AMD_LIB=timeline (the timestamped build) before importing npu_amd")
    _lib.lib()
    dev = torch.device("cuda:0")
    layers = synth.device_config5_layers(n_layers, dev, SEED)
    D = layers[0].D
    x0 = torch.from_numpy(synth.host_input(SEED, T, D, rmsnorm=False)).to(dev)
    bufs = [x0.clone(), torch.empty_like(x0)]
    from npu_amd.moe import GpuMoeChain
    ch = GpuMoeChain(layers)

    def step():
        if chain:                                   # gm_moe_chain (bench.py's timed step)
            ch(bufs[0], residual=True, out=bufs[1])
        else:                                       # one gm_moe_forward per layer
            for i, blk in enumerate(layers):
                blk(bufs[i % 2], residual=True, out=bufs[(i + 1) % 2])
    step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(replays):
        g.replay()
    torch.cuda.synchronize()
    for blk in layers:
        _zero_records(blk, T)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    return [_layer_records(blk, T) for blk in layers]


def summarise(recs, names):
    """Per kernel slot: medians over the inner layers of block-level statistics (us)."""
    inner = recs[1:-1] if len(recs) > 2 else recs
    stats = {}
    gaps_in, gaps_between = {}, []
    for li, layer in enumerate(inner):
        # kernels in the order they ran (slot numbers do not follow the launch order)
        slots = sorted((s for s in range(N_SLOTS) if layer[s]), key=lambda s: min(r[0] for r in layer[s]))
        t0 = min(r[0] for r in layer[slots[0]])
        for s in slots:
            rs = layer[s]
            e = sorted(r[0] for r in rs)
            m1 = sorted(r[1] for r in rs if r[1] != 0)               # marks a kernel does not set stay 0
            m2 = sorted(r[2] for r in rs if r[2] != 0)
            en = sorted(r[3] for r in rs)
            m3 = sorted(r[7] for r in rs if r[7] != 0)
            d = {"blocks": len(rs), "entry_first": e[0] - t0, "entry_median": e[len(e) // 2] - t0,
                 "mark3_median": (m3[len(m3) // 2] - t0) if m3 else None, "mark3_last": (m3[-1] - t0) if m3 else None,
                 "entry_last": e[-1] - t0,
                 "mark1_median": (m1[len(m1) // 2] - t0) if m1 else None, "mark1_last": (m1[-1] - t0) if m1 else None,
                 "mark2_median": (m2[len(m2) // 2] - t0) if m2 else None, "mark2_last": (m2[-1] - t0) if m2 else None,
                 "end_median": en[len(en) // 2] - t0, "end_last": en[-1] - t0,
                 "block_median": sorted(r[3] - r[0] for r in rs)[len(rs) // 2],
                 "mhz": sorted((r[6] - r[5]) * 100.0 / max(r[3] - r[0], 1) for r in rs)[len(rs) // 2],
                 "xccs": len({r[4] >> 32 for r in rs})}
            for kk, v in d.items():
                stats.setdefault(s, {}).setdefault(kk, []).append(v)
        for a, b in zip(slots, slots[1:]):
            gaps_in.setdefault((a, b), []).append(min(r[0] for r in layer[b]) - max(r[3] for r in layer[a]))
        nxt = recs[li + 2] if len(recs) > 2 else None
        if nxt is not None:
            ns = sorted((s for s in range(N_SLOTS) if nxt[s]), key=lambda s: min(r[0] for r in nxt[s]))
            gaps_between.append(min(r[0] for r in nxt[ns[0]]) - max(r[3] for r in layer[slots[-1]]))
    med = lambda v: statistics.median(v) * TICK_US

    def pair(d, a, b):                                           # "median / last", "-" for an unset mark
        va, vb = [x for x in d[a] if x is not None], [x for x in d[b] if x is not None]
        return f"{med(va):.2f} / {med(vb):.2f}" if va and vb else "-"

    lines = ["| kernel | blocks | XCDs | entry first / median / last | mark 3 median / last | mark 1 median / last | "
             "mark 2 median / last | end median / last | block duration (median) | shader clock MHz (median) |",
             "|---|---|---|---|---|---|---|---|---|---|"]
    for s, d in stats.items():
        lines.append(
            f"| {names.get(s, s)} | {int(statistics.median(d['blocks']))} | {int(statistics.median(d['xccs']))} | "
            f"{med(d['entry_first']):.2f} / {med(d['entry_median']):.2f} / {med(d['entry_last']):.2f} | "
            f"{pair(d, 'mark3_median', 'mark3_last')} | {pair(d, 'mark1_median', 'mark1_last')} | "
            f"{pair(d, 'mark2_median', 'mark2_last')} | "
            f"{med(d['end_median']):.2f} / {med(d['end_last']):.2f} | {med(d['block_median']):.2f} | "
            f"{statistics.median(d['mhz']):.0f} |")
    lines.append("")
    for (a, b), v in gaps_in.items():
        lines.append(f"- gap {names.get(a, a)} last end -> {names.get(b, b)} first entry: {med(v):.2f} us (median)")
    if gaps_between:
        lines.append(f"- gap last kernel of block l -> first kernel of block l+1: {med(gaps_between):.2f} us (median)")
    first = lambda layer: min(r[0] for s in range(N_SLOTS) for r in layer[s])
    per_block = [first(nxt) - first(cur) for cur, nxt in zip(recs[1:-1], recs[2:])]
    if per_block:
        lines.append(f"- block period (first entry to next block's first entry): {med(per_block):.2f} us (median)")
    return "\n".join(lines)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--T", type=int, default=1)
    ap.add_argument("--replays", type=int, default=5)
    ap.add_argument("--out", default=None, help="also write the summary to this file")
    ap.add_argument("--chain", action="store_true", help="time gm_moe_chain instead of per-layer calls")
    ap.add_argument("--npz", default=None, help="also save every record (layer, kernel, block) to this .npz")
    args = ap.parse_args()
    recs = run(args.layers, args.T, args.replays, chain=args.chain)
    if args.npz:
        import numpy as np
        rows = [(li, s, *r) for li, layer in enumerate(recs) for s in range(N_SLOTS) for r in layer[s]]
        np.savez_compressed(args.npz, records=np.array(rows, dtype=np.int64),
                            columns=np.array(["layer", "kernel", "entry", "mark1", "mark2", "end", "hwid",
                                              "clock0", "clock1", "mark3"]))
    names = {0: "router (stage 1)", 1: "gate/up (stage 2)", 2: "down (stage 3)", 3: "combine (T > 1)",
             4: "router partials (T > 1)", 5: "routing (T > 1)", 6: "gate/up (T > 1)", 7: "down (T > 1)"}
    text = summarise(recs, names)
    print(text)
    if args.out:
        with open(args.out, "w") as f:
            f.write(text + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
