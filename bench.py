"""Benchmark of the MoE-block decode hot path on one MI355X.

Headline (BASELINE.json metric "MoE-block decode tokens/s; effective
quant-weight GB/s vs HBM peak (1 GPU)"), measured on BASELINE config 5 at
batch 1: one decode step = 40 chained MoE blocks (D=2048, FF=512, E=256,
top-8, IQ4_XS gate/up + IQ3_XXS down, quantised shared expert, bf16 router),
x_{l+1} = x_l + moe_l(rmsnorm(x_l)), captured once as a hipGraph and replayed;
~15.5 GB of seeded random expert weights stay resident in HBM and each step
feeds its output back as the next input, so routing changes step to step.
A single block (config 3) would fit in the 256 MB Infinity Cache when
replayed, so its per-block figures are reported from the chain.

Timed region: `--steps` graph replays between a synchronize and two HIP
events; inputs are resident in HBM before it starts.  One JSON line on stdout.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

HBM_PEAK_GBPS = 8000.0
D, FF, E, K_TOP, N_LAYERS = 2048, 512, 256, 8, 40
SEED = 20261201


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=N_LAYERS)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-layers", type=int, default=8, help="blocks in the bounded CPU sample")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the extra legs (B = 8, prefill, dense and quantised matvecs, full decode step)")
    ap.add_argument("--calib-copy", action="store_true", help="only run a plain 256 MiB copy (counter calibration)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only run the config-4 prefill measurement (8 layers), one JSON line")
    ap.add_argument("--batch8-only", action="store_true",
                    help="only run the config-5 batch-8 chain over --layers layers, one JSON line")
    ap.add_argument("--dense-only", action="store_true",
                    help="only run the dense bf16 projection matvec measurement, one JSON line")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the per-stage graphs the roofline is measured on (for rocprof)")
    ap.add_argument("--chain-only", action="store_true", help="only the B=1 chain (for rocprof)")
    ap.add_argument("--matvec-only", action="store_true", help="only BASELINE configs 1-2 (quantised matvec)")
    ap.add_argument("--eager", action="store_true", help="--matvec-only: eager launches instead of graph replays")
    ap.add_argument("--matvec-batched-only", action="store_true",
                    help="--matvec-only: only the batched launches (for counter passes)")
    ap.add_argument("--reps", type=int, default=10, help="--matvec-only: timed repetitions")
    ap.add_argument("--decode-step-only", action="store_true",
                    help="only the full decoder step (attention, Gated DeltaNet, MoE, lm_head), one JSON line")
    ap.add_argument("--quant-shapes", default=None,
                    help="comma-separated subset of the configs 1-2 shapes for --matvec-only")
    ap.add_argument("--dense-shapes", default="ssm_in,ssm_gate,ssm_out", help="projections for --dense-only")
    ap.add_argument("--dense-tokens", default="1,8", help="token counts for --dense-only")
    return ap.parse_args()


def build_layers(n_layers: int, device):
    from npu_amd import synth
    return synth.device_config5_layers(n_layers, device, SEED)


def unique_experts(blk, T: int) -> int:
    """Distinct experts the last call routed to (grouping table word 0)."""
    import torch
    from npu_amd import ops
    ws = blk.workspace(T)
    lay = ops.moe_workspace_offsets(blk.struct, T)
    # the grouping table sits right after the weights array; its word 0 is n_unique
    grp_off = lay["weights"] + ((T * blk.k * 4 + 255) // 256) * 256
    return int(ws[grp_off:grp_off + 4].view(torch.int32).item())


def run_chain(layers, T: int, steps: int, warmup: int, seed: int):
    """Capture decode steps through gm_moe_chain (all layers in one call: at T = 1 one router
    launch, then gate/up and down per layer, each down kernel computing the next layer's
    router dot products) and time `steps` of them.  The graph holds two steps, the first
    from bufs[0] to bufs[1] and the second back, so every step's output is the next step's
    input and routing changes step to step; a step is half a replay."""
    import torch
    from npu_amd import synth
    from npu_amd.moe import GpuMoeChain
    dev = layers[0].gate.device
    x0 = torch.from_numpy(synth.host_input(seed, T, D, rmsnorm=False)).to(dev)
    bufs = [x0.clone(), torch.empty_like(x0)]
    chain = GpuMoeChain(layers)
    chain(bufs[0], residual=True, out=bufs[1])   # eager pass: workspaces, attributes
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        chain(bufs[0], residual=True, out=bufs[1])
        chain(bufs[1], residual=True, out=bufs[0])
    reps, wreps = (steps + 1) // 2, (warmup + 1) // 2
    for _ in range(wreps):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / (2 * reps)
    n_unique = [unique_experts(blk, T) for blk in layers]
    finite = bool(torch.isfinite(bufs[0]).all())
    return ms, n_unique, finite


def check_chain(layers):
    """The headline workload's own output: one eager gm_moe_chain call from the timed input
    against the same layers run one gm_moe_forward at a time.  Reports whether the chain ran
    the accumulator-linked kernels, whether the top-k ids agree at every layer, and the
    output's rel error (the logits are the same dot products added in another order)."""
    import torch
    from npu_amd import synth
    from npu_amd.moe import GpuMoeChain
    dev = layers[0].gate.device
    x0 = torch.from_numpy(synth.host_input(SEED, 1, D, rmsnorm=False)).to(dev)
    ch = GpuMoeChain(layers)
    y = ch(x0, residual=True)
    torch.cuda.synchronize()
    ids_c = [blk.stages(1)["topk_ids"].clone() for blk in layers]
    x = x0
    same = True
    for blk, ic in zip(layers, ids_c):
        x = blk(x, residual=True)
        same = same and bool(torch.equal(blk.stages(1)["topk_ids"], ic))
    torch.cuda.synchronize()
    rel = float((y.double() - x.double()).abs().max() / x.double().abs().max())
    return {"fused_path": ch.fused(1), "ids_equal_every_layer": same, "rel_vs_per_layer": rel,
            "finite": bool(torch.isfinite(y).all())}


def time_stages(layers, T: int, reps: int = 20):
    """Average launch period of each decode stage kernel: one hipGraph per stage holding
    that stage's launch for every layer (distinct weights), replayed `reps` times between
    two HIP events on the replay stream.  Back-to-back dependent launches of one kernel,
    so the period is the kernel's duration plus the ~1 us dependent-dispatch gap (the
    rocprof duration of the same kernel is the lower bound)."""
    import torch
    from npu_amd import synth
    dev = layers[0].gate.device
    x = torch.from_numpy(synth.host_input(SEED + 1, T, D, rmsnorm=False)).to(dev)
    y = torch.empty_like(x)
    for blk in layers:                       # routing state in every workspace
        blk(x, residual=True, out=y)
    torch.cuda.synchronize()
    out = {}
    for stage, name in ((1, "router_shared_us"), (2, "gateup_us"), (3, "down_us")):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for blk in layers:
                blk(x, residual=True, out=y, stage=stage)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        out[name] = e0.elapsed_time(e1) * 1e3 / (reps * len(layers))
    return out


def time_stage_launches(layers, T: int, stage: int = 2, batches: int = 10):
    """Average launch duration of one decode stage's kernel, measured with HIP events on the
    launch stream: each batch holds that stage's launch for every layer (distinct weights),
    enqueued eagerly behind a spin kernel (torch.cuda._sleep) so that the host is ahead of
    the GPU and the launches run back to back; two events bracket the batch, and the
    duration is the batch time over its launches.  The first batch is a warm-up.  The
    layers' workspaces are prepared by stage 1 alone (stage 2 reads only its results), so
    every launch of the stage's kernel in a run of `bench.py --roofline-only` is a timed
    one: rocprofv3's average duration for the kernel over that run covers the same
    launches (the graph period of time_stages also holds the dependent-dispatch gap, and
    under tracing its launches stretch)."""
    import torch
    from npu_amd import synth
    dev = layers[0].gate.device
    x = torch.from_numpy(synth.host_input(SEED + 1, T, D, rmsnorm=False)).to(dev)
    y = torch.empty_like(x)
    for blk in layers:
        blk(x, residual=True, out=y, stage=1)
    torch.cuda.synchronize()
    periods = []
    for _ in range(batches + 1):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(20_000_000)
        e0.record()
        for blk in layers:
            blk(x, residual=True, out=y, stage=stage)
        e1.record()
        torch.cuda.synchronize()
        periods.append(e0.elapsed_time(e1) * 1e3 / len(layers))
    timed = periods[1:]
    return sum(timed) / len(timed)


def roofline(layers, launch_us: float, graph_period_us: float | None = None):
    """The dominant kernel, k_dec_gateup1w (top-k, routed and shared gate/up, SwiGLU, T = 1):
    its algorithmic bytes per launch (npu_amd.rocprof_summary.algorithmic_bytes: the k
    routed and the shared experts' raw gate and up rows, x and the RMSNorm weight, the
    router accumulators, the logits and the k + 1 SwiGLU rows it writes) over its average
    launch duration from time_stage_launches."""
    from npu_amd.rocprof_summary import algorithmic_bytes
    b = layers[0]
    n = algorithmic_bytes(D, FF, E, K_TOP)["k_dec_gateup1w"]
    assert b.gate[0].numel() == FF * (D // 256 * 136) and b.down[0].numel() == D * (FF // 256 * 98)
    gbps = n / (launch_us * 1e-6) / 1e9
    return {"bound": "hbm", "kernel": "k_dec_gateup1w (top-k + routed and shared gate/up + SwiGLU, T=1)",
            "achieved": gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": gbps / HBM_PEAK_GBPS,
            "traffic": traffic_bytes("k_dec_gateup1w"), "bytes_per_launch": n, "avg_launch_us": launch_us,
            "graph_period_us": graph_period_us}


def run_prefill(layers, T: int = 512, n_blocks: int = 8, reps: int = 5, samples: dict | None = None):
    """BASELINE config 4 on the chain's first `n_blocks` layers (distinct weights, so the
    ~250 MB of experts one block touches does not stay in the Infinity Cache): a per-expert
    router bias ~ N(0,1) skews the routing, inputs are N(0,1) [T, D].  Reports the mean
    block time, the weight bytes of the distinct experts read per block (effective GB/s),
    and the MFMA utilisation of the block's flops against the dense bf16 peak."""
    import torch
    from npu_amd import _lib as L
    from npu_amd import synth
    dev = layers[0].gate.device
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED + 4)
    blocks = layers[:n_blocks]
    saved = [(b.router_bias, b.struct.router_bias) for b in blocks]
    try:
        for b in blocks:
            b.router_bias = torch.randn(E, generator=gen, device=dev, dtype=torch.float32)
            b.struct.router_bias = L.ptr(b.router_bias)
        if samples is not None:                     # the CPU baseline's config-4 leg runs layer 0 with its bias
            samples["prefill_bias"] = blocks[0].router_bias.cpu()
        x = torch.from_numpy(synth.host_input(SEED + 5, T, D, rmsnorm=False)).to(dev)
        y = torch.empty_like(x)
        for b in blocks:
            b(x, out=y)
        torch.cuda.synchronize()
        n_unique = []
        for b in blocks:
            b(x, out=y)
            ids = b.stages(T)["topk_ids"]
            n_unique.append(int(torch.unique(ids).numel()))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            for b in blocks:
                b(x, out=y)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * n_blocks)
        finite = bool(torch.isfinite(y).all())
    finally:
        for b, (t, p) in zip(blocks, saved):
            b.router_bias, b.struct.router_bias = t, p
    b0 = blocks[0]
    per_expert = b0.gate[0].numel() + b0.up[0].numel() + b0.down[0].numel()
    fixed = (sum(t.numel() for t in (b0.gate_sh, b0.up_sh, b0.down_sh)) + b0.router.numel() * 2
             + b0.sh_gate_inp.numel() * 2)
    wbytes = sum(n * per_expert + fixed for n in n_unique) / len(n_unique)
    flops = 2.0 * T * (K_TOP + 1) * 3 * FF * D + 2.0 * T * E * D
    return {"workload": f"config4: prefill T={T}, router bias ~ N(0,1), mean over {n_blocks} distinct layers",
            "block_us": us, "tokens_per_s": T / (us * 1e-6),
            "mean_unique_experts": sum(n_unique) / len(n_unique), "weight_bytes_per_block": wbytes,
            "effective_weight_GBps": wbytes / (us * 1e-6) / 1e9,
            "hbm_frac": wbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS,
            "flops_per_block": flops, "TFLOPs": flops / (us * 1e-6) / 1e12,
            "mfma_util_vs_bf16_dense_peak": flops / (us * 1e-6) / 2.5e15, "finite": finite}


def kquant_shared_layers(layers, seed: int = SEED + 6):
    """The same blocks with the shared expert as the reference model's GGUF stores it: Q6_K
    gate, Q8_0 up and Q6_K down (seeded random blocks, transcoded once on the device to I8
    rows), beside the IQ routed experts (the same device tensors, not copied)."""
    import numpy as np
    import torch
    from npu_amd import _lib as L
    from npu_amd import ops, synth
    from npu_amd.gguf_types import GGMLQuantizationType as QT
    from npu_amd.moe import GpuMoeBlock
    g = np.random.default_rng(seed)
    dev = layers[0].gate.device
    out = []
    for b in layers:
        def i8(q, M, K, per):
            raw = synth.host_kquant_blocks(g, q, M * K // per)
            return ops.transcode_i8(int(q), torch.from_numpy(raw.reshape(-1)).to(dev)).view(M, K // 32 * 48)
        out.append(GpuMoeBlock(gate=b.gate, up=b.up, down=b.down, router=b.router, q_gate=b.q_gate,
                               q_down=b.q_down, D=b.D, FF=b.FF, E=b.E, k=b.k,
                               gate_sh=i8(QT.Q6_K, b.FF, b.D, 256), up_sh=i8(QT.Q8_0, b.FF, b.D, 32),
                               down_sh=i8(QT.Q6_K, b.D, b.FF, 256), q_gate_sh=L.GM_QTYPE_I8,
                               q_down_sh=L.GM_QTYPE_I8, sh_gate_inp=b.sh_gate_inp, norm_w=b.norm_w,
                               norm_eps=b.norm_eps, device=dev))
    return out


def run_decode_step(moe_layers, n_prefill: int = 64, steps: int = 20, seed: int = SEED + 50):
    """The whole decoder for one token (qwen/forward.py:834-893 at T = 1) through
    npu_amd.qwen_core.forward: the reference model's 40 layers (Gated DeltaNet in 30, gated
    attention in every fourth, Qwen3.6-35B-A3B shapes: D 2048, 16 q / 2 kv heads of 256,
    RoPE 64; 16 K / 32 V heads of 128 with a conv of 4), each followed by its MoE block
    (the chain's config-5 blocks, RMSNorm weight 1), the output norm and a 248,320 x 2048
    lm_head.  Seeded device weights: the core projections bf16 N(0, 0.02), embedding
    N(0, 1).  `n_prefill` tokens are decoded first to fill the KV caches and the recurrent
    states; then one decode step at position `n_prefill` is captured in a hipGraph and
    replayed `steps` times (each replay rewrites cache row `n_prefill` and advances the
    recurrent states), timed between HIP events on the replay stream.  Eager steps (one
    C-ABI call per core layer and MoE block, host launch included) are timed beside it."""
    import torch
    from npu_amd import qwen_core as QN
    dev = moe_layers[0].gate.device
    n_layer = len(moe_layers)
    cfg = QN.Config(n_layer=n_layer, is_attention=[(i + 1) % 4 == 0 for i in range(n_layer)])
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def w(*shape, std=0.02):
        return (torch.randn(*shape, generator=g, device=dev) * std).to(torch.bfloat16).float()

    def v(n, base=1.0, std=0.1):
        return base + torch.randn(n, generator=g, device=dev) * std
    D, Dh, Hq, Hkv = cfg.d_model, cfg.head_dim, cfg.n_head, cfg.n_head_kv
    Hk, Hv, S = cfg.ssm_n_k_heads, cfg.ssm_n_v_heads, cfg.ssm_d_state
    C = 2 * Hk * S + Hv * S
    layers = []
    for i in range(n_layer):
        if cfg.is_attention[i]:
            core = QN.AttnLayer(i=i, attn_norm=v(D), post_norm=torch.ones(D, device=dev), wq=w(2 * Hq * Dh, D),
                                wk=w(Hkv * Dh, D), wv=w(Hkv * Dh, D), wo=w(D, Hq * Dh), q_norm=v(Dh), k_norm=v(Dh))
            core.gpu = QN.GpuAttn(core, cfg)
        else:
            core = QN.SSMLayer(i=i, attn_norm=v(D), post_norm=torch.ones(D, device=dev), w_in=w(C, D),
                               w_gate=w(Hv * S, D), conv1d=v(C * cfg.ssm_d_conv, 0.0, 0.5).view(C, -1),
                               a=-torch.rand(Hv, generator=g, device=dev), alpha=w(Hv, D, std=0.05),
                               beta=w(Hv, D, std=0.05), dt_bias=v(Hv, 0.0, 0.5), ssm_norm=v(S), w_out=w(D, Hv * S))
            core.gpu = QN.GpuSsm(core, cfg)
        for name in [f for f in ("wq", "wk", "wv", "wo", "w_in", "w_gate", "w_out") if hasattr(core, f)]:
            setattr(core, name, None)                  # the bf16 device copies are what runs
        layers.append((core, moe_layers[i]))
    V = cfg.vocab_size
    max_pos = n_prefill + 8
    cos, sin = QN.build_partial_rope_cache(cfg.rope_dim, max_pos, cfg.rope_theta, device=dev)
    model = QN.Model(cfg=cfg, token_embd=torch.randn(V, D, generator=g, device=dev), output_norm=v(D),
                     lm_head=w(V, D), layers=layers, rope_cos=cos, rope_sin=sin)
    kv, st = None, None
    tok = 17
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for pos in range(n_prefill):                        # eager decode steps
        logits, kv, st = QN.forward(model, [tok], start_pos=pos, kv_caches=kv, ssm_states=st)
        tok = (tok * 31 + pos) % V
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / n_prefill
    kv_len = [c.length if c is not None else None for c in kv]
    tok_dev = torch.tensor([tok], dtype=torch.long, device=dev)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        logits, _, _ = QN.forward(model, tok_dev, start_pos=n_prefill, kv_caches=kv, ssm_states=st)
    for c, n in zip(kv, kv_len):                        # the replays rewrite row n_prefill
        if c is not None:
            c.length = n
    gr.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        gr.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    core_bytes = sum((l[0].gpu.wqkv.numel() + l[0].gpu.wo.numel()) * 2 if isinstance(l[0], QN.AttnLayer) else
                     (l[0].gpu.w_in.numel() + l[0].gpu.w_gate.numel() + l[0].gpu.w_out.numel()) * 2
                     for l in layers)
    moe_bytes = sum(b.weight_bytes_per_token() for b in moe_layers)
    head = V * D * 2
    total = core_bytes + moe_bytes + head
    return {"workload": f"full decode step: {n_layer} layers ({sum(cfg.is_attention)} gated attention, "
                        f"{n_layer - sum(cfg.is_attention)} Gated DeltaNet) + MoE blocks + lm_head {V} x {D}, "
                        f"position {n_prefill}, hipGraph replay",
            "ms_per_token": ms, "tokens_per_s": 1e3 / ms, "eager_ms_per_token": eager_ms,
            "weight_bytes_per_token": total, "core_weight_bytes": core_bytes, "moe_weight_bytes": moe_bytes,
            "lm_head_bytes": head, "effective_weight_GBps": total / (ms * 1e-3) / 1e9,
            "hbm_frac": total / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
            "finite": bool(torch.isfinite(logits).all())}


DENSE_SHAPES = (("ssm_in", 8192, 2048), ("ssm_gate", 4096, 2048), ("ssm_out", 2048, 4096))
# on request only (--dense-shapes lm_head): the output projection, 1 GB, 2 distinct copies
DENSE_EXTRA = (("lm_head", 248_320, 2048),)


def run_dense_mv(dev, n_layers: int = 30, reps: int = 20, shapes=None, tokens=(1, 8)):
    """The dense bf16 projections NpuMatVec serves (qwen/forward.py:827-831): the Gated
    DeltaNet layer's w_in 8192x2048, w_gate 4096x2048 and w_out 2048x4096
    (qwen/test_npu_ssm.py), bf16 weights N(0, 0.02) for `n_layers` distinct layers
    (1.9 GB, beyond the Infinity Cache), fp32 x.  Per shape and token count, one hipGraph
    holds that projection's gm_matvec for every layer; the replay period per launch
    gives the effective weight GB/s (weight bytes / time; x and y are < 0.5% of them).
    torch's bf16 F.linear (x rounded to bf16) on the same weights is timed the same way
    for scale."""
    import torch
    from npu_amd import _lib as L
    from npu_amd.gguf_types import GGMLQuantizationType as QT
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED + 30)
    todo = [sh for sh in DENSE_SHAPES + DENSE_EXTRA if (shapes is None and sh in DENSE_SHAPES)
            or (shapes is not None and sh[0] in shapes)]
    nl = {name: (2 if M * K * 2 > (1 << 29) else n_layers) for name, M, K in todo}     # >= 2 GB per shape
    Ws = {name: [(torch.randn(M, K, generator=gen, device=dev) * 0.02).to(torch.bfloat16) for _ in range(nl[name])]
          for name, M, K in todo}
    lib = L.lib()

    def period_us(fn, launches):
        fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (reps * launches)

    out = {"workload": f"SSM projections (qwen/test_npu_ssm.py shapes), bf16 weights, {n_layers} distinct layers",
           "shapes": {}}
    for name, M, K in todo:
        wbytes = M * K * 2
        for T in tokens:
            x = torch.randn(T, K, generator=gen, device=dev)
            y = torch.empty(T, M, device=dev)
            xb = x.to(torch.bfloat16)

            def ours():
                s = L.stream_ptr()
                for W in Ws[name]:
                    L.check(lib.gm_matvec(int(QT.BF16), L.ptr(W), M, K, L.ptr(x), T, L.ptr(y), s), "gm_matvec")

            def torch_linear():
                for W in Ws[name]:
                    torch.nn.functional.linear(xb, W)

            us = period_us(ours, nl[name])
            ref = x.double() @ Ws[name][-1].double().T
            rel = float((y.double() - ref).abs().max() / ref.abs().max())
            tus = period_us(torch_linear, nl[name])
            gbps = (wbytes + T * (K + M) * 4) / (us * 1e-6) / 1e9
            out["shapes"][f"{name}_T{T}"] = {
                "M": M, "K": K, "T": T, "us_per_launch": us, "weight_GBps": wbytes / (us * 1e-6) / 1e9,
                "algorithmic_GBps": gbps, "hbm_frac": gbps / HBM_PEAK_GBPS, "rel_err_vs_f64": rel,
                "torch_bf16_linear_us": tus}
    return out


QUANT_MV_SHAPES = (("config1_iq4xs_512x2048", 23, 512, 2048), ("config2_iq3xxs_2048x512", 18, 2048, 512),
                   ("config2_iq3xxs_512x2048", 18, 512, 2048))


def run_quant_mv(dev, reps: int = 10, batch: int = 64, total_mb: int = 330, samples: dict | None = None,
                 shapes=None, graph: bool = True, per_call_leg: bool = True):
    """BASELINE configs 1 and 2: one y = W x with W a raw IQ4_XS [512 x 2048] or IQ3_XXS
    [2048 x 512] / [512 x 2048] matrix (the reference's NpuIQ4MatVec / NpuQuantMatVec
    call, npu/quant_mv.py:419-463), fp32 x ~ N(0, 1), seeded device-generated
    superblocks.  Enough distinct matrices for ~330 MB (beyond the 256 MB Infinity Cache)
    are resident; one hipGraph holds one gm_matvec per matrix (the back-to-back calls of
    the configs), replayed `reps` times: period per call.  Batched variant: `batch`
    consecutive matrices are one [batch M x K] raw matrix, so one launch computes their
    products with the same x.  Algorithmic bytes per call: W + x + y.  ``graph=False``
    times the same launches eagerly (for counter collection, which serialises every
    dispatch anyway); ``per_call_leg=False`` skips the per-call launches (a few batched
    launches are all a counter pass needs)."""
    import torch
    from npu_amd import _lib as L
    from npu_amd import ops, synth
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED + 40)
    lib = L.lib()
    out = {}
    for name, qt, M, K in QUANT_MV_SHAPES:
        if shapes is not None and name not in shapes:
            continue
        rb = (K // 256) * (136 if qt == 23 else 98)
        n = max(batch, (total_mb << 20) // (M * rb) // batch * batch)
        W = synth.device_quant_matrix(gen, qt, M, K, n, dev)                  # [n, M, rb] uint8
        x = torch.randn(K, generator=gen, device=dev)
        y = torch.empty(n, M, device=dev)
        yb = torch.empty(n // batch, batch * M, device=dev)

        def per_call():
            s = L.stream_ptr()
            for i in range(n):
                L.check(lib.gm_matvec(qt, L.ptr(W[i]), M, K, L.ptr(x), 1, L.ptr(y[i]), s), "gm_matvec")

        def batched():
            s = L.stream_ptr()
            for j in range(n // batch):
                L.check(lib.gm_matvec(qt, L.ptr(W[j * batch]), batch * M, K, L.ptr(x), 1, L.ptr(yb[j]), s),
                        "gm_matvec")

        def period_us(fn, launches):
            fn()
            torch.cuda.synchronize()
            run = fn
            if graph:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    fn()
                g.replay()
                torch.cuda.synchronize()
                run = g.replay
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                run()
            e1.record()
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) * 1e3 / (reps * launches)

        us = period_us(per_call, n) if per_call_leg else float("nan")
        ub = period_us(batched, n // batch)
        # the last matrix against its device dequant (gm_dequant_f32, exact) in float64
        Wd = ops.dequant(qt, W[n - 1].reshape(-1)).view(M, K).double()
        ref = Wd @ x.double()
        y_last = y[n - 1] if per_call_leg else yb.view(n, M)[n - 1]
        rel = float((y_last.double() - ref).abs().max() / ref.abs().max())
        same = bool(torch.equal(yb.view(n, M), y)) if per_call_leg else None
        if samples is not None:                     # the CPU baseline's leg: the last matrix and x
            samples.setdefault("quant_mv", {})[name] = (qt, M, K, W[n - 1].cpu().numpy(), x.cpu().numpy())
        algo = M * rb + K * 4 + M * 4
        out[name] = {"M": M, "K": K, "distinct_matrices": n, "resident_MB": n * M * rb / 2**20,
                     "algorithmic_bytes_per_call": algo,
                     "graph_us_per_call": us, "graph_GBps": algo / (us * 1e-6) / 1e9,
                     "graph_frac": algo / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS,
                     "batched_matrices_per_launch": batch, "batched_us_per_launch": ub,
                     "batched_GBps": batch * algo / (ub * 1e-6) / 1e9,
                     "batched_frac": batch * algo / (ub * 1e-6) / 1e9 / HBM_PEAK_GBPS,
                     "rel_err_vs_f64": rel, "batched_equals_per_call": same}
        del W, y, yb
    return out


def _median_ms(fn, runs: int = 5, warmup: int = 2) -> tuple[float, int]:
    """Median wall time of ``fn`` in ms over ``runs`` timed calls after ``warmup`` untimed
    ones (time.perf_counter_ns), and the number of timed calls."""
    import statistics
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter_ns()
        fn()
        times.append((time.perf_counter_ns() - t0) * 1e-6)
    return statistics.median(times), runs


def _host_layers(layers):
    import numpy as np
    from npu_amd import synth
    from oracle import moe as OM
    out = []
    for blk in layers:
        h = synth.HostMoeLayer(
            D=D, FF=FF, E=E, k=K_TOP, q_gate=blk.q_gate, q_down=blk.q_down,
            gate=blk.gate.cpu().numpy(), up=blk.up.cpu().numpy(), down=blk.down.cpu().numpy(),
            router=blk.router.cpu().numpy().view(np.uint16), gate_sh=blk.gate_sh.cpu().numpy(),
            up_sh=blk.up_sh.cpu().numpy(), down_sh=blk.down_sh.cpu().numpy(),
            sh_gate_inp=blk.sh_gate_inp.cpu().numpy().view(np.uint16), norm_w=blk.norm_w.cpu().numpy())
        out.append(OM.OracleLayer(h))
    return out


def _pre_dequant(hosts, x0, T_residual=True):
    """Per layer, the experts one pass from x0 routes to (and the shared expert), dequantised."""
    import torch
    from oracle import moe as OM
    pre, y = [], x0
    for L in hosts:
        st = {}
        y_next = OM.block_forward(y, L, residual=T_residual, stages=st)
        d = {int(e): L.dequant_one(int(e)) for e in torch.unique(st["topk_ids"]).tolist()}
        d["shared"] = L.shared_weights()
        pre.append(d)
        y = y_next
    return pre


def cpu_baseline(layers, n_sample: int, budget_s: float = 12.0, prefill_bias=None, quant_mv=None):
    """The reference's CPU path, restated by the oracle (a port of qwen/forward.py:moe_forward's
    CPU branch, 652-663, and of the dequant + F.linear of the quantised operators), timed on
    this host's cores beside the GPU figures.  Headline (config 5, B = 1): the first
    `n_sample` blocks of the chain run back to back (each output feeding the next block) for
    about `budget_s` seconds, the median per-block time scaled to the 40-block step, with
    per-call dequant of every picked expert as dequant_one does, and again with those experts
    dequantised up front (the CPU's best case).  ``configs`` holds the other BASELINE configs,
    each the median of 5 runs after 2 warm-ups in both variants: 1 and 2 (one quantised
    matvec, dequant + F.linear), 3 (one block at T = 1), 4 (one block at T = 512 with the
    bench's router bias) and 5 at B = 8 (4 chained blocks)."""
    import statistics
    import numpy as np
    import torch
    import torch.nn.functional as F
    from npu_amd import synth
    from oracle import moe as OM
    from oracle import quants as Q

    threads = cpu_share()
    torch.set_num_threads(threads)
    hosts = _host_layers(layers[:n_sample])
    x0 = torch.from_numpy(synth.host_input(SEED, 1, D, rmsnorm=False))
    for _ in range(2):                                      # two untimed warm-up passes over the sample
        y = x0
        for L in hosts:
            y = OM.block_forward(y, L, residual=True)

    def passes(pre, budget):
        times, t_start = [], time.perf_counter()
        while not times or (time.perf_counter() - t_start < budget and len(times) < 200):
            y = x0                                         # same inputs each pass -> same routing
            t0 = time.perf_counter()
            for i, L in enumerate(hosts):
                y = OM.block_forward(y, L, residual=True, pre_dequant=None if pre is None else pre[i])
            times.append((time.perf_counter() - t0) / len(hosts))
        return times, time.perf_counter() - t_start

    t_call, wall_call = passes(None, budget_s)
    t_pre, wall_pre = passes(_pre_dequant(hosts, x0), budget_s / 4)
    per_block = statistics.median(t_call)
    per_block_pre = statistics.median(t_pre)
    blk_bytes = layers[0].weight_bytes_per_token()          # k experts + shared + router + shared gate
    configs = {"config3_block_T1": {
        "per_call_dequant_ms": per_block * 1e3, "pre_dequantised_ms": per_block_pre * 1e3,
        "effective_weight_GBps": blk_bytes / per_block / 1e9,
        "sample": f"the headline sample's per-block median ({len(t_call)} passes of {n_sample} blocks)"}}

    # configs 1 and 2: one quantised matvec, dequant + F.linear (and F.linear on the fp32 matrix)
    if quant_mv is not None:
        for name, (qt, M, K, raw, x) in quant_mv.items():
            x_t = torch.from_numpy(x)
            def per_call():
                F.linear(x_t, torch.from_numpy(Q.dequant_matrix(raw, qt, M, K)))
            Wf = torch.from_numpy(Q.dequant_matrix(raw, qt, M, K))
            ms_call, n = _median_ms(per_call, runs=21)
            ms_pre, _ = _median_ms(lambda: F.linear(x_t, Wf), runs=21)
            algo = raw.size + 4 * (K + M)
            configs[name] = {"per_call_dequant_ms": ms_call, "pre_dequantised_ms": ms_pre,
                             "effective_GBps": algo / (ms_call * 1e-3) / 1e9, "runs": n,
                             "sample": "one matrix of the GPU leg's set, its x"}

    # config 4: one block at T = 512, router bias ~ N(0, 1) (the GPU leg's first layer and bias)
    if prefill_bias is not None:
        L0 = hosts[0]
        L4 = OM.OracleLayer(L0.h)
        L4.bias = prefill_bias.float().cpu()
        xp = torch.from_numpy(synth.host_input(SEED + 5, 512, D, rmsnorm=False))
        st = {}
        OM.block_forward(xp, L4, stages=st)
        uniq = torch.unique(st["topk_ids"]).tolist()
        ms_call, n = _median_ms(lambda: OM.block_forward(xp, L4))
        pre4 = {int(e): L4.dequant_one(int(e)) for e in uniq}
        pre4["shared"] = L4.shared_weights()
        ms_pre, _ = _median_ms(lambda: OM.block_forward(xp, L4, pre_dequant=pre4))
        per_exp = layers[0].gate[0].numel() + layers[0].up[0].numel() + layers[0].down[0].numel()
        wb = len(uniq) * per_exp + blk_bytes - K_TOP * per_exp
        configs["config4_prefill_T512"] = {
            "per_call_dequant_ms": ms_call, "pre_dequantised_ms": ms_pre, "tokens_per_s": 512 / (ms_call * 1e-3),
            "pre_dequantised_tokens_per_s": 512 / (ms_pre * 1e-3), "unique_experts": len(uniq),
            "effective_weight_GBps": wb / (ms_call * 1e-3) / 1e9, "runs": n,
            "sample": "layer 0 with the GPU leg's router bias, x = N(0, 1) [512, 2048]"}

    # config 5 at B = 8: 4 chained blocks, per-block median scaled to the 40-block step
    h8 = hosts[:4]
    x8 = torch.from_numpy(synth.host_input(SEED + 8, 8, D, rmsnorm=False))

    def chain8(pre=None):
        y = x8
        for i, L in enumerate(h8):
            y = OM.block_forward(y, L, residual=True, pre_dequant=None if pre is None else pre[i])
    ms_call, n = _median_ms(chain8)
    pre8 = _pre_dequant(h8, x8)
    ms_pre, _ = _median_ms(lambda: chain8(pre8))
    step_ms = ms_call / len(h8) * N_LAYERS
    configs["config5_b8"] = {"per_call_dequant_step_ms": step_ms, "tokens_per_s": 8 / (step_ms * 1e-3),
                             "pre_dequantised_step_ms": ms_pre / len(h8) * N_LAYERS,
                             "pre_dequantised_tokens_per_s": 8 / (ms_pre / len(h8) * N_LAYERS * 1e-3),
                             "runs": n, "sample": f"{len(h8)} chained config-5 blocks, B = 8, x {N_LAYERS} / {len(h8)}"}
    return {
        "value": 1.0 / (per_block * N_LAYERS), "unit": "tokens/s", "cores": threads, "kind": "port",
        "sample": (f"oracle restatement of moe_forward, B=1: {n_sample} chained config-5 blocks x {len(t_call)} "
                   f"passes ({wall_call:.1f} s), median per-block time x {N_LAYERS} blocks; per-call dequant "
                   f"of each picked expert (numpy) + torch fp32 F.linear, {threads} threads"),
        "block_ms": per_block * 1e3,
        "pre_dequantised_block_ms": per_block_pre * 1e3,
        "pre_dequantised_tokens_per_s": 1.0 / (per_block_pre * N_LAYERS),
        "cpu": cpu_model(), "os_cpu_count": os.cpu_count(), "warmup_passes": 2,
        "configs": configs,
    }


def cpu_model() -> str:
    """The host CPU's model name from /proc/cpuinfo (the architecture where it has none)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_share() -> int:
    """Threads for the CPU baseline: every core this process may run on.  A GPU host's job
    scheduler may pin the process to a share of the host (then OMP_NUM_THREADS says how
    many cores that share holds); without either, all of os.cpu_count()."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS", "")
    return min(n, int(omp)) if omp.isdigit() and int(omp) > 0 else n


def traffic_bytes(kernel: str):
    """HBM bytes per launch of `kernel` from the committed counter summary
    (profiles/hbm_traffic.json: FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the
    same counters read on a plain copy kernel of known size); None if absent."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            return json.load(f)["kernels"][kernel]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def calib_copy() -> None:
    import torch
    n = 256 << 20
    a = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    b = torch.empty_like(a)
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"calib_copy_bytes": n, "launches": 5}))


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (got --gpus {args.gpus}); "
              "multi-GPU expert parallelism is a design note, not built", file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU available", file=sys.stderr)
        return 1
    if args.calib_copy:
        calib_copy()
        return 0
    from npu_amd import _lib
    _lib.lib()
    dev = torch.device("cuda:0")

    if args.prefill_only:
        layers = build_layers(8, dev)
        torch.cuda.synchronize()
        out = {"prefill": run_prefill(layers)}
        out["prefill_kquant_shared"] = run_prefill(kquant_shared_layers(layers))
        print(json.dumps(out))
        return 0
    if args.dense_only:
        print(json.dumps({"dense_mv": run_dense_mv(dev, shapes=args.dense_shapes.split(","),
                                                   tokens=[int(t) for t in args.dense_tokens.split(",")])}))
        return 0
    if args.matvec_only:
        shapes = None if args.quant_shapes is None else args.quant_shapes.split(",")
        print(json.dumps({"quant_mv": run_quant_mv(dev, reps=args.reps, shapes=shapes, graph=not args.eager,
                                                   per_call_leg=not args.matvec_batched_only)}))
        return 0
    if args.decode_step_only:
        layers = build_layers(args.layers, dev)
        torch.cuda.synchronize()
        print(json.dumps({"decode_step": run_decode_step(layers)}))
        return 0
    if args.roofline_only:
        layers = build_layers(args.layers, dev)
        torch.cuda.synchronize()
        launch_us = time_stage_launches(layers, 1)
        print(json.dumps({"roofline": roofline(layers, launch_us)}))
        return 0
    if args.chain_only:
        layers = build_layers(args.layers, dev)
        torch.cuda.synchronize()
        ms1, _, ok1 = run_chain(layers, 1, args.steps, args.warmup, SEED)
        print(json.dumps({"ms_per_step": ms1, "block_us": ms1 * 1e3 / args.layers, "finite": ok1}))
        return 0
    if args.batch8_only:
        layers = build_layers(args.layers, dev)
        torch.cuda.synchronize()
        ms8, nu8, ok8 = run_chain(layers, 8, args.steps, args.warmup, SEED + 8)
        print(json.dumps({"batch8": {"layers": args.layers, "ms_per_step": ms8, "tokens_per_s": 8e3 / ms8,
                                     "mean_unique_experts_per_layer": sum(nu8) / len(nu8), "finite": ok8}}))
        return 0
    log(f"building {args.layers} layers of seeded synthetic weights on {torch.cuda.get_device_name(0)}")
    t0 = time.time()
    layers = build_layers(args.layers, dev)
    torch.cuda.synchronize()
    weight_gb = sum(sum(t.numel() * t.element_size() for t in (b.gate, b.up, b.down, b.router, b.gate_sh,
                                                              b.up_sh, b.down_sh, b.sh_gate_inp))
                    for b in layers) / 1e9
    log(f"built {weight_gb:.2f} GB resident in {time.time() - t0:.1f} s")

    per_expert = layers[0].gate[0].numel() + layers[0].up[0].numel() + layers[0].down[0].numel()
    fixed = (sum(t.numel() for t in (layers[0].gate_sh, layers[0].up_sh, layers[0].down_sh))
             + layers[0].router.numel() * 2 + layers[0].sh_gate_inp.numel() * 2)

    log(f"B=1 chain: warmup {args.warmup}, steps {args.steps}")
    ms1, nu1, ok1 = run_chain(layers, 1, args.steps, args.warmup, SEED)
    bytes1 = sum(n * per_expert + fixed for n in nu1)
    tok_s = 1e3 / ms1
    eff_gbps = bytes1 / (ms1 * 1e-3) / 1e9
    log(f"B=1: {ms1 * 1e3:.1f} us/step, {tok_s:.1f} tok/s, {eff_gbps:.1f} GB/s effective, finite={ok1}")

    chain_ok = check_chain(layers)
    log(f"40-layer chain vs per-layer gm_moe_forward: {chain_ok}")
    stages = time_stages(layers, 1)
    log(f"stages (us): {stages}")

    extra, samples = {}, {}
    if not args.no_extra:
        ms8, nu8, ok8 = run_chain(layers, 8, max(20, args.steps // 4), max(2, args.warmup // 4), SEED + 8)
        bytes8 = sum(n * per_expert + fixed for n in nu8)
        extra["batch8"] = {"ms_per_step": ms8, "tokens_per_s": 8e3 / ms8,
                           "effective_weight_GBps": bytes8 / (ms8 * 1e-3) / 1e9,
                           "mean_unique_experts_per_layer": sum(nu8) / len(nu8), "finite": ok8}
        log(f"B=8: {extra['batch8']}")
        extra["prefill"] = run_prefill(layers, samples=samples)
        log(f"prefill: {extra['prefill']}")
        extra["prefill_kquant_shared"] = run_prefill(kquant_shared_layers(layers[:8]))
        extra["prefill_kquant_shared"]["workload"] = ("config4 with the shared expert as the real GGUF holds it "
                                                      "(Q6_K gate, Q8_0 up, Q6_K down as I8 rows), 8 layers")
        log(f"prefill, K-quant shared expert: {extra['prefill_kquant_shared']}")
        extra["dense_mv"] = run_dense_mv(dev)
        log(f"dense bf16 matvec: {extra['dense_mv']}")
        extra["quant_mv"] = run_quant_mv(dev, samples=samples)
        log(f"quant matvec (configs 1-2): {extra['quant_mv']}")
        extra["decode_step"] = run_decode_step(layers)
        log(f"full decode step: {extra['decode_step']}")

    cpu = None
    if not args.no_cpu_baseline:
        log(f"CPU baseline: {args.cpu_layers} blocks of the oracle")
        cpu = cpu_baseline(layers, args.cpu_layers, prefill_bias=samples.get("prefill_bias"),
                           quant_mv=samples.get("quant_mv"))
        log(f"CPU: {cpu}")

    out = {
        "metric": "MoE-block decode tokens/s; effective quant-weight GB/s vs HBM peak (1 GPU)",
        "value": tok_s, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms1, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seeded, torch GPU generator; BASELINE config 5 distributions)",
        "config": {"workload": "config5: 40 chained MoE blocks, decode T=1 batch 1, hipGraph replay",
                   "D": D, "FF": FF, "experts": E, "top_k": K_TOP, "layers": args.layers,
                   "gate_up": "IQ4_XS", "down": "IQ3_XXS", "shared_expert": "IQ4_XS/IQ3_XXS",
                   "router": "bf16", "resident_weight_GB": round(weight_gb, 3)},
        "effective_weight_GBps": eff_gbps,
        "effective_weight_frac_of_peak": eff_gbps / HBM_PEAK_GBPS,
        "block_us": ms1 * 1e3 / args.layers,
        "weight_bytes_per_step": bytes1,
        "roofline": roofline(layers, time_stage_launches(layers, 1), stages["gateup_us"]),
        "stage_us": stages,
        "cpu_baseline": cpu,
        "finite": ok1,
        "chain_check": chain_ok,
    }
    out.update(extra)
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
