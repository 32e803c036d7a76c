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
from npu_amd.moe import GpuMoeBlock
from oracle import moe as OM

pytestmark = pytest.mark.gpu
N_LAYERS = 4


@pytest.fixture(scope="module")
def chain(gpu):
    hosts = [synth.host_moe_layer(200 + i, norm=True) for i in range(N_LAYERS)]
    return hosts, [GpuMoeBlock.from_host(h, device=gpu) for h in hosts]


def _oracle_chain(hosts, x0, k):
    """Per-layer top-k ids and the chain output; asserts every layer's input is near-tie free."""
    ids, x = [], x0
    for li, h in enumerate(hosts):
        ol = OM.OracleLayer(h)
        margin = OM.topk_margin(OM.router_logits64(x, ol), k)
        assert bool((margin > 1e-5).all()), f"layer {li}: near-tie input, choose another seed"
        st = {}
        x = OM.block_forward(x, ol, residual=True, stages=st)
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
