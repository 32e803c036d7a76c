"""BASELINE config 5 as a chain: four config-3 blocks in one hipGraph, against the oracle.

Each block is D=2048, FF=512, E=256, top-8, IQ4_XS gate/up, IQ3_XXS down, with the
shared expert, an RMSNorm weight != 1 and the residual add of qwen/forward.py:880-884
(x_{l+1} = x_l + moe_l(rms_norm(x_l))).  The four launches sequences are captured once
with two ping-pong activation buffers, exactly as bench.py's run_chain times them, and
the graph is replayed several times with eager work on the same workspaces in between.
Oracle: oracle.moe.block_forward layer by layer (= oracle.moe.chain_forward), a
restatement of qwen/forward.py:563-665.  Bar: every layer's top-k ids equal (all inputs
are near-tie free, asserted), the chain output within rel 1e-3 (fp32-accumulate decode),
every replay bit-identical to the first.
"""
import pytest
import torch

from npu_amd import synth
from npu_amd.moe import GpuMoeBlock, GpuMoeChain
from oracle import moe as OM

pytestmark = pytest.mark.gpu
N_LAYERS = 4


@pytest.fixture(scope="module")
def chain(gpu):
    hosts = [synth.host_moe_layer(200 + i, norm=True) for i in range(N_LAYERS)]
    return hosts, [GpuMoeBlock.from_host(h, device=gpu) for h in hosts]


def _oracle_chain(hosts, x0, k):
    """Per-layer top-k ids and the chain output; asserts every layer's input is near-tie free
    and that the k-th and (k+1)-th softmax probabilities differ in fp32 (the reference takes
    the top-k of the probabilities, which underflow to equal zeros when logits spread by
    more than ~100)."""
    ids, x = [], x0
    for li, h in enumerate(hosts):
        ol = OM.OracleLayer(h)
        margin = OM.topk_margin(OM.router_logits64(x, ol), k)
        assert bool((margin > 1e-5).all()), f"layer {li}: near-tie input, choose another seed"
        st = {}
        x = OM.block_forward(x, ol, residual=True, stages=st)
        pv = torch.topk(st["ffn_moe_probs"], k + 1, dim=-1).values
        assert bool((pv[:, k - 1] > pv[:, k]).all()), f"layer {li}: k-th probability ties (underflow)"
        ids.append(st["topk_ids"])
    return ids, x


@pytest.mark.parametrize("T", [1, 8])
def test_config5_chain_graph(gpu, chain, T):
    hosts, blocks = chain
    print(f"chain case T={T} layers={N_LAYERS}", flush=True)
    x0 = torch.from_numpy(synth.host_input(300 + T, T, hosts[0].D, rmsnorm=False))
    ids_ref, y_ref = _oracle_chain(hosts, x0, hosts[0].k)

    bufs = [x0.to(gpu).clone(), torch.empty_like(x0, device=gpu)]
    for i, blk in enumerate(blocks):                      # eager pass: workspaces sized before capture
        blk(bufs[i % 2], residual=True, out=bufs[(i + 1) % 2])
    torch.cuda.synchronize()
    y_eager = bufs[N_LAYERS % 2].clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i, blk in enumerate(blocks):
            blk(bufs[i % 2], residual=True, out=bufs[(i + 1) % 2])
    first = None
    for rep in range(3):
        bufs[0].copy_(x0.to(gpu))
        g.replay()
        torch.cuda.synchronize()
        y = bufs[N_LAYERS % 2].clone()
        ids = [blk.stages(T)["topk_ids"].cpu().long() for blk in blocks]
        for li in range(N_LAYERS):
            assert torch.equal(ids[li], ids_ref[li]), f"replay {rep}: layer {li} top-k ids differ"
        rel = OM.rel_err(y.cpu(), y_ref)
        assert rel <= 1e-3, f"replay {rep}: chain rel {rel:.3e}"
        if first is None:
            first = y
            assert torch.equal(y, y_eager), "graph replay differs from the eager chain"
        else:
            assert torch.equal(y, first), f"replay {rep} differs from replay 0"
        # eager work on the same workspaces between replays
        blocks[0](torch.randn_like(x0).to(gpu), residual=True)
        torch.cuda.synchronize()


# gm_moe_chain: the same chains through the library's chain entry point.  At T = 1 each
# layer's down kernel computes the next layer's router dot products (fp64 accumulators),
# so this checks the routing of layers 1.. computed that way against the oracle.
CHAIN_VARIANTS = {                                        # name: (seed base, layer arguments)
    "config5": (400, dict(norm=True)),
    "f32_router_bias": (410, dict(norm=True, router_f32=True, bias=True)),
    "no_norm_no_shared": (420, dict(shared=False, layers=2)),   # without RMSNorm activations grow fast
    "ungated_shared": (430, dict(norm=True, ungated=True)),
    "e512": (440, dict(norm=True, E=512)),                 # 8 accumulator words per lane
    "d1280": (450, dict(norm=True, D=1280)),               # D not a multiple of 512
}


@pytest.fixture(scope="module", params=sorted(CHAIN_VARIANTS))
def variant_chain(request, gpu):
    seed, kw = CHAIN_VARIANTS[request.param]
    kw = dict(kw)
    ungated = kw.pop("ungated", False)
    hosts = []
    for i in range(kw.pop("layers", N_LAYERS)):
        h = synth.host_moe_layer(seed + i, **kw)
        if ungated:
            h.sh_gate_inp = None
        hosts.append(h)
    return request.param, hosts, [GpuMoeBlock.from_host(h, device=gpu) for h in hosts]


@pytest.mark.parametrize("T", [1, 3, 8])
def test_gm_moe_chain(gpu, variant_chain, T):
    name, hosts, blocks = variant_chain
    n = len(hosts)
    print(f"gm_moe_chain case {name} T={T} layers={n}", flush=True)
    x0 = torch.from_numpy(synth.host_input(500 + T, T, hosts[0].D, rmsnorm=hosts[0].norm_w is None))
    if hosts[0].norm_w is None:
        x0 = x0 * 0.01           # without RMSNorm the block amplifies ~x^2: keeps layer 1's logits spread ~10
    ids_ref, y_ref = _oracle_chain(hosts, x0, hosts[0].k)
    ch = GpuMoeChain(blocks)
    assert ch.mode(T) == (1 if T == 1 else 2), f"{name}: the chain took path {ch.mode(T)}"
    xd = x0.to(gpu)
    y_eager = ch(xd, residual=True)
    torch.cuda.synchronize()
    for li in range(n):
        st = blocks[li].stages(T)
        ids = st["topk_ids"].cpu().long()
        if not torch.equal(ids, ids_ref[li]):
            lg = st["ffn_moe_logits"].cpu()
            print(f"layer {li}: ids {ids.tolist()} vs {ids_ref[li].tolist()}; logits[0,:8] {lg[0, :8].tolist()}")
        assert torch.equal(ids, ids_ref[li]), f"layer {li} top-k ids differ"
    rel = OM.rel_err(y_eager.cpu(), y_ref)
    assert rel <= 1e-3, f"chain rel {rel:.3e}"
    # the per-layer entry point computes the same function
    bufs = [xd.clone(), torch.empty_like(xd)]
    for i, blk in enumerate(blocks):
        blk(bufs[i % 2], residual=True, out=bufs[(i + 1) % 2])
    torch.cuda.synchronize()
    rel_pl = OM.rel_err(y_eager.cpu(), bufs[n % 2].cpu())
    assert rel_pl <= 1e-5, f"chain vs per-layer gm_moe_forward rel {rel_pl:.3e}"
    # captured once, replayed with other work on the workspaces in between: bit-identical
    out = torch.empty_like(xd)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ch(xd, residual=True, out=out)
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y_eager), f"replay {rep} differs from the eager chain"
        blocks[0](torch.randn_like(xd), residual=True)
        torch.cuda.synchronize()


def test_config5_headline_chain_40_layers(gpu):
    """The bench's headline workload itself: bench.py's 40 config-5 layers (same seed, same
    input) through one gm_moe_chain call (the accumulator-linked kernels, asserted), against
    (a) the same 40 layers run one gm_moe_forward at a time: top-k ids equal at every layer,
    output rel <= 1e-5 (the chain's logits are the same dot products added in another order);
    (b) the oracle, layer by layer from the device weights (experts fetched as routed): ids
    equal at every layer (every layer's input asserted near-tie free) and output rel <= 1e-3."""
    import bench
    print("headline chain case: 40 config-5 layers, T=1", flush=True)
    layers = synth.device_config5_layers(bench.N_LAYERS, gpu, bench.SEED)
    x0 = torch.from_numpy(synth.host_input(bench.SEED, 1, bench.D, rmsnorm=False))
    ch = GpuMoeChain(layers)
    assert ch.fused(1)
    y_chain = ch(x0.to(gpu), residual=True)
    torch.cuda.synchronize()
    ids_chain = [blk.stages(1)["topk_ids"].cpu().long().clone() for blk in layers]
    x = x0.to(gpu)
    ids_pl = []
    for blk in layers:
        x = blk(x, residual=True)
        ids_pl.append(blk.stages(1)["topk_ids"].cpu().long().clone())
    torch.cuda.synchronize()
    for li in range(len(layers)):
        assert torch.equal(ids_chain[li], ids_pl[li]), f"layer {li}: chain and per-layer ids differ"
    rel_pl = OM.rel_err(y_chain.cpu(), x.cpu())
    assert rel_pl <= 1e-5, f"chain vs per-layer rel {rel_pl:.3e}"
    hosts = [synth.host_view(blk) for blk in layers]
    ids_ref, y_ref = _oracle_chain(hosts, x0, 8)
    for li in range(len(layers)):
        assert torch.equal(ids_chain[li], ids_ref[li]), f"layer {li}: ids differ from the oracle"
    rel = OM.rel_err(y_chain.cpu(), y_ref)
    print(f"headline chain: rel vs per-layer {rel_pl:.2e}, vs oracle {rel:.2e}", flush=True)
    assert rel <= 1e-3, f"chain vs oracle rel {rel:.3e}"
    del layers, hosts
    torch.cuda.empty_cache()


def test_gm_moe_chain_shared_workspace_t8(gpu, chain):
    """gm_moe_chain allows one workspace for every layer.  At T = 8 the layers then cannot
    be linked (a combine kernel would write the next layer's router inputs over the partial
    rows it reads), so each layer runs as gm_moe_forward: the output equals the per-layer
    calls bit for bit, and the linked chain (distinct workspaces) to fp32 rounding."""
    from npu_amd import ops
    hosts, blocks = chain
    T, n = 8, len(blocks)
    print(f"gm_moe_chain case shared workspace T={T} layers={n}", flush=True)
    xd = torch.from_numpy(synth.host_input(610, T, hosts[0].D, rmsnorm=False)).to(gpu)
    ws = torch.zeros(ops.moe_workspace_bytes(blocks[0].struct, T), dtype=torch.uint8, device=gpu)
    y, buf = torch.empty_like(xd), torch.empty_like(xd)
    ops.moe_chain_raw([b.struct for b in blocks], xd, y, buf, [ws] * n, residual=True)
    bufs = [xd.clone(), torch.empty_like(xd)]
    for i, blk in enumerate(blocks):
        blk(bufs[i % 2], residual=True, out=bufs[(i + 1) % 2])
    ch = GpuMoeChain(blocks)
    assert ch.mode(T) == 2
    y_linked = ch(xd, residual=True)
    torch.cuda.synchronize()
    assert torch.equal(y, bufs[n % 2]), "shared-workspace chain differs from the per-layer calls"
    rel = OM.rel_err(y_linked.cpu(), y.cpu())
    assert rel <= 1e-5, f"linked chain vs per-layer rel {rel:.3e}"
