"""GPU parity of the MoE block prefill path (T > 8: grouped MFMA GEMMs).

Oracle: oracle.moe.block_forward, the restatement of qwen/forward.py:563-665
(the reference runs prefill through the same CPU loop).  Bar: top-k ids
identical for every token whose k-th/(k+1)-th logit margin is clear of fp32
rounding, rel <= 1e-2 over those tokens (activations and h are rounded to bf16
before the MFMA products), bit-identical repeats (fixed-order combine).
"""
import numpy as np
import pytest
import torch

from npu_amd import synth
from npu_amd.gguf_types import GGMLQuantizationType as QT
from npu_amd.moe import GpuMoeBlock
from oracle import moe as OM

pytestmark = pytest.mark.gpu
REL_TOL = 1e-2


def _check(gpu, h, T, residual=False, seed=5, rmsnorm_input=True, logits_atol=None, x_scale=1.0):
    print(f"prefill case D={h.D} FF={h.FF} E={h.E} k={h.k} T={T} q=({h.q_gate},{h.q_down}) "
          f"shared={h.gate_sh is not None} residual={residual}", flush=True)
    ol = OM.OracleLayer(h)
    x = torch.from_numpy(synth.host_input(seed, T, h.D, rmsnorm=rmsnorm_input)) * x_scale
    blk = GpuMoeBlock.from_host(h, device=gpu)
    y = blk(x.to(gpu), residual=residual)
    y2 = blk(x.to(gpu), residual=residual)
    st_gpu = {k: v.clone().cpu() for k, v in blk.stages(T).items()}
    y, y2 = y.cpu(), y2.cpu()
    st = {}
    ref = OM.block_forward(x, ol, residual=residual, stages=st)
    margin = OM.topk_margin(OM.router_logits64(x, ol), h.k)
    clear = margin > 1e-5
    assert int(clear.sum()) >= T - 2, "too many near-ties for a meaningful check"
    assert torch.equal(st_gpu["topk_ids"].long()[clear], st["topk_ids"][clear]), "top-k ids differ"
    assert torch.allclose(st_gpu["ffn_moe_weights_norm"][clear], st["ffn_moe_weights_norm"][clear], rtol=1e-5,
                          atol=1e-7)
    assert torch.isfinite(y).all()
    rel = float((y[clear] - ref[clear]).abs().max() / ref[clear].abs().max())
    assert rel <= REL_TOL, rel
    assert torch.equal(y, y2), "repeat calls must be bit-identical"
    if logits_atol is not None:
        assert torch.allclose(st_gpu["ffn_moe_logits"], st["ffn_moe_logits"], rtol=0, atol=logits_atol)
        if h.sh_gate_inp is not None:
            assert torch.allclose(st_gpu["shared_expert_gate_sigmoid"], st["shared_expert_gate_sigmoid"], rtol=1e-5)
    return rel, st


def test_config4_prefill(gpu):
    """T=512, D=2048, FF=512, E=256, top-8, per-expert router bias ~ N(0,1)."""
    h = synth.host_moe_layer(40, q_gate=QT.IQ4_XS, q_down=QT.IQ3_XXS, bias=True)
    rel, st = _check(gpu, h, 512, seed=7, rmsnorm_input=False)
    counts = torch.bincount(st["topk_ids"].flatten(), minlength=h.E)
    assert int(counts.max()) > 64, "the skew must give experts more than one 64-token segment"


@pytest.mark.parametrize("q_gate,q_down", [(QT.IQ4_XS, QT.IQ3_XXS), (QT.IQ3_XXS, QT.IQ4_XS),
                                           (QT.IQ4_XS, QT.IQ4_XS), (QT.IQ3_XXS, QT.IQ3_XXS)])
@pytest.mark.parametrize("T", [9, 64, 130])
@pytest.mark.parametrize("shared", [True, False])
def test_small_prefill(gpu, q_gate, q_down, T, shared):
    h = synth.host_moe_layer(60 + T, D=512, FF=256, E=16, k=4, q_gate=q_gate, q_down=q_down, shared=shared,
                             bias=True)
    _check(gpu, h, T, seed=T)


@pytest.mark.parametrize("T", [16, 200])
def test_prefill_norm_and_residual(gpu, T):
    h = synth.host_moe_layer(70 + T, D=1024, FF=512, E=64, k=8, norm=True, bias=True)
    _check(gpu, h, T, residual=True, rmsnorm_input=False)


def test_prefill_model_assignment(gpu):
    """The reference model's assignment (IQ3_XXS gate/up, IQ4_XS down), E=128, T=96."""
    h = synth.host_moe_layer(80, D=2048, FF=512, E=128, k=8, q_gate=QT.IQ3_XXS, q_down=QT.IQ4_XS)
    _check(gpu, h, 96, seed=3)


def test_prefill_stage_outputs(gpu):
    h = synth.host_moe_layer(81, D=512, FF=256, E=32, k=4, bias=True)
    T = 40
    x = torch.from_numpy(synth.host_input(4, T, h.D))
    blk = GpuMoeBlock.from_host(h, device=gpu)
    blk(x.to(gpu))
    got = {k: v.cpu() for k, v in blk.stages(T).items()}
    st = {}
    OM.block_forward(x, OM.OracleLayer(h), stages=st)
    assert torch.allclose(got["ffn_moe_logits"], st["ffn_moe_logits"], rtol=0, atol=2e-5)
    assert torch.equal(got["topk_ids"].long(), st["topk_ids"])
    assert torch.allclose(got["shared_expert_gate_sigmoid"], st["shared_expert_gate_sigmoid"], rtol=1e-5)


@pytest.mark.parametrize("T", [1, 3, 8])
def test_prefill_path_at_decode_sizes(gpu, T):
    """gm_moe_prefill at T <= 8 against the oracle, and against the decode kernels."""
    h = synth.host_moe_layer(90 + T, q_gate=QT.IQ4_XS, q_down=QT.IQ3_XXS)
    ol = OM.OracleLayer(h)
    x = torch.from_numpy(synth.host_input(T, T, h.D))
    blk = GpuMoeBlock.from_host(h, device=gpu)
    yp = blk(x.to(gpu), path="prefill").cpu()
    yd = blk(x.to(gpu), path="decode").cpu()
    ref = OM.block_forward(x, ol)
    margin = OM.topk_margin(OM.router_logits64(x, ol), h.k)
    assert bool((margin > 1e-5).all()), "near-tie token: choose another seed"
    assert OM.rel_err(yp, ref) <= REL_TOL
    assert OM.rel_err(yd, ref) <= 1e-3
    assert OM.rel_err(yp, yd) <= REL_TOL


@pytest.mark.parametrize("D,FF,E,k,T", [(256, 256, 512, 8, 40), (4096, 256, 16, 4, 20), (256, 1024, 8, 2, 24),
                                        (2304, 256, 64, 4, 20), (2304, 256, 320, 8, 24), (8192, 256, 16, 4, 12),
                                        (8192, 256, 260, 8, 9)])
def test_prefill_size_limits(gpu, D, FF, E, k, T):
    """Prefill at the limits it accepts: E = 512 (dispatch histogram width, 8-per-lane top-k),
    D = 4096, FF = 1024 (the 4-superblock h tile of the down kernel); D = 2304 (nine
    256-wide router ranges) and D = 8192 (sixteen 512-wide ranges, the prep kernel's
    two-pass branch for D > 4096), each with E <= 256 and E > 256."""
    h = synth.host_moe_layer(110 + k, D=D, FF=FF, E=E, k=k, bias=True)
    _check(gpu, h, T, seed=k)


@pytest.mark.parametrize("D,E,k,T", [(2048, 256, 8, 64), (2048, 256, 8, 300), (2304, 64, 4, 40), (8192, 16, 4, 12)])
def test_prefill_fp32_router(gpu, D, E, k, T):
    """Router and shared gate in fp32 with values bf16 cannot hold (GGUF F32 tensors; the
    reference reads both in fp32, qwen/forward.py:41-47): the prefill router GEMM splits
    each fp32 weight into three bf16 pieces and accumulates all nine piece products, so
    the logits keep fp32 accuracy.  512- and 256-wide K ranges, D up to 8192."""
    h = synth.host_moe_layer(130 + T, D=D, FF=256, E=E, k=k, router_f32=True, bias=True)
    assert not np.array_equal(synth.from_bf16(synth.to_bf16(h.router)), h.router)
    _check(gpu, h, T, seed=T, logits_atol=2e-5)


@pytest.mark.parametrize("D,E,k,T", [(1024, 64, 8, 40), (8192, 16, 4, 12)])
@pytest.mark.parametrize("x_scale", [1e6, 3e-8])
def test_prefill_input_scale(gpu, D, E, k, T, x_scale):
    """Inputs far outside f16's range and no RMSNorm weight (the way the drop-in builds its
    blocks): x 1e6 would overflow f16 (65504) and x 3e-8 would fall into f16 subnormals
    if the gate/up operand were f16(x) itself.  The operand is f16(x 2^s) with a
    per-token power of two, undone exactly after the products; D = 8192 takes the prep
    kernel's two-pass branch.  The router and shared gate (fp32) are divided by the
    same factor so that the logits keep their usual size: at logits of 1e6 every
    softmax probability but the largest underflows to an exact 0, and torch.topk
    orders such ties arbitrarily."""
    h = synth.host_moe_layer(150 + k, D=D, FF=256, E=E, k=k, bias=True)
    h.router = (synth.as_f32(h.router) / x_scale).astype(np.float32)
    h.sh_gate_inp = (synth.as_f32(h.sh_gate_inp) / x_scale).astype(np.float32)
    _check(gpu, h, T, seed=k, rmsnorm_input=False, x_scale=x_scale)


def test_prefill_rejects_wide_ff(gpu):
    """FF > 1024 is outside the prefill kernels' h tile: a clear error, nothing launched."""
    h = synth.host_moe_layer(120, D=256, FF=2048, E=4, k=2)
    blk = GpuMoeBlock.from_host(h, device=gpu)
    x = torch.from_numpy(synth.host_input(1, 12, h.D)).to(gpu)
    with pytest.raises(ValueError, match="FF"):
        blk(x, path="prefill")


def _kquant_blocks(rng, qtype, n):
    """Random blocks of a K-quant / Q8_0 type with finite fp16 d (and dmin)."""
    from oracle import kquants as KQ
    w, nb = KQ.BLOCK[qtype]
    b = rng.integers(0, 256, (n, nb), dtype=np.uint8)
    d = (rng.standard_normal(n) * 1e-2).astype(np.float16).view(np.uint8).reshape(n, 2)
    if qtype == KQ.Q6_K:
        b[:, 208:210] = d
    else:
        b[:, 0:2] = d
        if qtype != KQ.Q8_0:
            b[:, 2:4] = (np.abs(rng.standard_normal(n)) * 1e-2).astype(np.float16).view(np.uint8).reshape(n, 2)
    return b


@pytest.mark.parametrize("T,D,FF,E,k", [(12, 512, 256, 16, 4), (130, 1024, 512, 64, 8), (512, 2048, 512, 256, 8)])
def test_prefill_kquant_shared_expert(gpu, T, D, FF, E, k):
    """IQ routed experts beside a Q6_K / Q8_0 shared expert (as the real model's GGUF holds
    it; transcoded once to I8 rows) at T > 8.  The routed experts stay on the prefill GEMMs
    and the shared expert runs as two f16 MFMA GEMMs of its own:
    (a) with an all-zero I8 shared expert the output equals the same layer without one, bit
    for bit (the routed part is the same computation, so a run of the tokens as decode
    chunks, which rounds the routed part differently, fails this);
    (b) with the K-quant shared expert, the output minus that layer's output equals
    sigmoid(xn . g_sh) times the fp64 shared expert within 5e-3 of the shared term's maximum
    (f16 weights and activations, bf16 SwiGLU rows, as the routed prefill experts);
    (c) the oracle's routed part plus that shared term matches within the prefill bar."""
    import torch.nn.functional as F
    from npu_amd import _lib as L, ops
    from oracle import kquants as KQ
    print(f"prefill kquant-shared case T={T} D={D} FF={FF} E={E} k={k}", flush=True)
    rng = np.random.default_rng(T + D)
    h = synth.host_moe_layer(90 + T, D=D, FF=FF, E=E, k=k, shared=False)
    raw = {"gate": (_kquant_blocks(rng, KQ.Q6_K, FF * D // 256), KQ.Q6_K, (FF, D)),
           "up": (_kquant_blocks(rng, KQ.Q8_0, FF * D // 32), KQ.Q8_0, (FF, D)),
           "down": (_kquant_blocks(rng, KQ.Q6_K, D * FF // 256), KQ.Q6_K, (D, FF))}
    i8 = {n: ops.transcode_i8(int(q), torch.from_numpy(b.reshape(-1)).to(gpu)).view(shp[0], shp[1] // 32 * 48)
          for n, (b, q, shp) in raw.items()}
    g_sh = torch.from_numpy((rng.standard_normal(D) * 0.02).astype(np.float32)).to(torch.bfloat16)  # bf16 router kept
    common = dict(gate=h.gate, up=h.up, down=h.down, router=h.router, q_gate=h.q_gate, q_down=h.q_down,
                  D=D, FF=FF, E=E, k=k, device=gpu)
    blk = GpuMoeBlock(**common, gate_sh=i8["gate"], up_sh=i8["up"], down_sh=i8["down"], q_gate_sh=L.GM_QTYPE_I8,
                      q_down_sh=L.GM_QTYPE_I8, sh_gate_inp=g_sh)
    blk_r = GpuMoeBlock(**common)
    zero = {n: torch.zeros_like(t) for n, t in i8.items()}
    blk_0 = GpuMoeBlock(**common, gate_sh=zero["gate"], up_sh=zero["up"], down_sh=zero["down"],
                        q_gate_sh=L.GM_QTYPE_I8, q_down_sh=L.GM_QTYPE_I8, sh_gate_inp=g_sh)
    x = torch.from_numpy(synth.host_input(31 + T, T, D))
    y = blk(x.to(gpu)).cpu().double()
    y_r = blk_r(x.to(gpu)).cpu().double()
    assert torch.equal(blk_0(x.to(gpu)).cpu().double(), y_r), "zero shared expert: routed part must be unchanged"
    assert torch.equal(blk(x.to(gpu)).cpu().double(), y), "repeat calls must be bit-identical"
    xs = x.double()
    gs, us, ds = (torch.from_numpy(KQ.dequant(b, q).reshape(shp)).double() for b, q, shp in raw.values())
    sh = (F.silu(xs @ gs.T) * (xs @ us.T)) @ ds.T
    sg = torch.sigmoid(xs @ g_sh.double())
    shared = sg[:, None] * sh
    err = float((y - y_r - shared).abs().max() / shared.abs().max())
    assert err <= 5e-3, f"shared GEMMs beside the routed GEMMs: {err:.3e}"
    ol = OM.OracleLayer(h)
    margin = OM.topk_margin(OM.router_logits64(x, ol), k)
    clear = margin > 1e-5
    assert int(clear.sum()) >= T - 2
    ref = OM.block_forward(x, ol).double() + shared
    rel = float((y[clear] - ref[clear]).abs().max() / ref[clear].abs().max())
    assert rel <= REL_TOL, rel
