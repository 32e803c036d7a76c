"""GPU parity of the drop-in operators (reference npu/*.py and qwen/forward.py names)."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from npu_amd import iq3_xxs, mlp, mv, quant_mv, quant_mv_iq4, quant_mv_iq4_packed, qwen_moe, synth
from npu_amd.gguf_types import GGMLQuantizationType as QT, QuantTensor
from oracle import moe as OM
from oracle import quants as Q

pytestmark = pytest.mark.gpu


def _stack(qtype, E, M, K, seed):
    g = np.random.Generator(np.random.PCG64(seed))
    return QuantTensor("t", qtype, (K, M, E), synth.host_quant_matrix(g, qtype, M, K, E))


@pytest.mark.parametrize("cls,qtype,M,K", [
    (quant_mv.NpuQuantMatVec, QT.IQ3_XXS, 512, 2048),
    (quant_mv_iq4.NpuIQ4MatVec, QT.IQ4_XS, 2048, 512),
    (quant_mv_iq4_packed.NpuIQ4PackedMatVec, QT.IQ4_XS, 2048, 512),
])
def test_quant_operators_from_gguf_tensor(gpu, cls, qtype, M, K):
    t = _stack(qtype, 4, M, K, 3)
    op = cls.from_gguf_tensor(t, expert_idx=2)
    x = torch.randn(K, generator=torch.Generator().manual_seed(0)) * 0.05   # qwen/test_npu_experts.py:68
    y = op(x)                                  # CPU in, CPU out (reference behaviour)
    assert y.shape == (M,) and y.device.type == "cpu"
    ref = F.linear(x, torch.from_numpy(Q.dequant_matrix(t.data[2], qtype, M, K)))
    assert OM.cos(y, ref) >= 0.999999 and OM.rel_err(y, ref) <= 1e-3
    y2 = op(x.reshape(1, 1, K).to(gpu))       # GPU in, GPU out; batched shape kept
    assert y2.is_cuda and y2.shape == (1, 1, M)
    assert torch.equal(y2.cpu().reshape(-1), y)
    with pytest.raises(AssertionError):
        op(torch.zeros(K + 1))


def test_npu_matvec_and_concat(gpu):
    g = torch.Generator().manual_seed(1)
    Ws = [torch.randn(r, 2048, generator=g) * 0.02 for r in (256, 64, 32)]
    x = torch.randn(2048, generator=g)
    y = mv.NpuMatVec(Ws[0])(x)
    ref = F.linear(x, Ws[0].to(torch.bfloat16).float())
    assert OM.rel_err(y, ref) <= 1e-5
    op = mv.NpuConcatMatVec(tuple(Ws))
    yc = op(x)
    refc = F.linear(x, torch.cat(Ws).to(torch.bfloat16).float())
    assert op.out_splits == (256, 64, 32) and OM.rel_err(yc, refc) <= 1e-5


@pytest.mark.parametrize("shape", [(1, 256), (1,), (3,), (2, 13)])
@pytest.mark.parametrize("out_f,in_f", [(576, 576), (1536, 576), (576, 1536), (300, 2048)])
def test_npu_linear(gpu, shape, out_f, in_f):
    """NpuLinear (npu/linear.py:147-244) against float64 F.linear of the bf16 weight and
    the fp32 input, at the reference self-test's shape (576 x 576, x [1, 256, 576]) and
    SmolLM2's projection shapes; one token runs the VALU matvec, more the MFMA kernel."""
    from npu_amd.linear import NpuLinear
    g = torch.Generator().manual_seed(out_f + in_f + len(shape))
    W = torch.randn(out_f, in_f, generator=g, dtype=torch.bfloat16)
    x = torch.randn(*shape, in_f, generator=g)
    lin = NpuLinear(W)
    y = lin(x)
    assert y.dtype == torch.float32 and y.shape == (*shape, out_f) and not y.is_cuda
    ref = F.linear(x.double(), W.double())
    assert OM.rel_err(y.double(), ref) <= 1e-5
    # the reference self-test's own bar (npu/linear.py:258-262), bf16 input
    xb = x.to(torch.bfloat16)
    assert float((lin(xb) - F.linear(xb.float(), W.float())).abs().max()) < 5e-2
    yd = lin(x.to(gpu))
    assert yd.is_cuda and torch.equal(yd.cpu(), y)


@pytest.mark.parametrize("stacked", [False, True])
def test_npu_fused_mlp(gpu, stacked):
    g = torch.Generator().manual_seed(2)
    hidden, ffn = 2048, 512
    wg, wu, wd = (torch.randn(ffn, hidden, generator=g) * 0.02, torch.randn(ffn, hidden, generator=g) * 0.02,
                  torch.randn(hidden, ffn, generator=g) * 0.02)
    x = torch.randn(hidden, generator=g)
    op = mlp.NpuFusedMLP(torch.cat([wg, wu]), wd) if stacked else mlp.NpuFusedMLP(wg, wd, w_up=wu)
    y = op(x)
    b = lambda w: w.to(torch.bfloat16).float()
    ref = F.linear(F.silu(F.linear(x, b(wg))) * F.linear(x, b(wu)), b(wd))
    assert OM.rel_err(y, ref) <= 1e-4
    assert torch.equal(op(x), y), "repeat determinism (qwen/test_npu_shexp_fused.py:73-74)"


def test_iq3_xxs_module(gpu):
    g = np.random.Generator(np.random.PCG64(4))
    blocks = synth.host_superblocks(g, QT.IQ3_XXS, 16)
    assert np.array_equal(iq3_xxs.dequant_rows(blocks), Q.dequant_iq3_xxs(blocks))
    assert np.array_equal(iq3_xxs.dequant_block(blocks[3].tobytes()), Q.dequant_iq3_xxs(blocks[3]))


@pytest.mark.parametrize("T", [1, 4])
def test_qwen_moe_forward_dropin(gpu, T):
    hs = [synth.host_moe_layer(40 + i, D=2048, FF=512, E=64, k=8) for i in range(2)]
    ts = qwen_moe.SyntheticTensorStore(hs)
    layers = [qwen_moe.MoELayer.load(ts, i) for i in range(2)]
    qwen_moe.enable_npu(layers, ops=("router", "experts", "experts_packed_down"))
    assert "router" in layers[0].npu and "expert_tensors" in layers[0].npu
    x = torch.from_numpy(synth.host_input(9, T, 2048)).reshape(1, T, 2048)
    for i, L in enumerate(layers):
        y = qwen_moe.moe_forward(x, L, ts.cfg)
        assert y.shape == x.shape and y.device.type == "cpu"
        ref = OM.moe_forward(x, OM.OracleLayer(hs[i]))
        assert OM.rel_err(y, ref) <= 1e-3
    # dequant_one mirrors MoELayer.dequant_one (qwen/forward.py:480-491)
    g, u, d = layers[0].dequant_one(5)
    assert torch.equal(g, torch.from_numpy(Q.dequant_matrix(hs[0].gate[5], hs[0].q_gate, 512, 2048)))
    assert d.shape == (2048, 512)


@pytest.mark.parametrize("T", [1, 12])
def test_qwen_moe_forward_from_gguf_file(gpu, tmp_path, T):
    """The MoE drop-in fed from a GGUF file read by npu_amd.gguf_file (the reference reads
    its model through gguf-py's GGUFReader + TensorStore, qwen/model.py:164-277): raw
    expert superblocks mapped from the file straight to HBM, router / shared gate from F32
    tensors holding values bf16 cannot represent (kept in fp32 on the device: top-k ids
    equal to the oracle's, which reads them in fp32 as the reference does)."""
    from npu_amd import gguf_file
    hs = [synth.host_moe_layer(60 + i, D=1024, FF=256, E=32, k=4, q_gate=q, q_down=d, router_f32=True)
          for i, (q, d) in enumerate([(QT.IQ4_XS, QT.IQ3_XXS), (QT.IQ3_XXS, QT.IQ4_XS)])]
    path = tmp_path / "moe.gguf"
    synth.write_gguf_model(path, hs)
    ts = gguf_file.TensorStore(path)
    assert ts.cfg.n_layer == 2 and ts.cfg.n_expert_used == 4
    layers = [qwen_moe.MoELayer.load(ts, i) for i in range(2)]
    x = torch.from_numpy(synth.host_input(11, T, 1024)).reshape(1, T, 1024)
    for i, L in enumerate(layers):
        y = qwen_moe.moe_forward(x, L, ts.cfg)
        ol, st = OM.OracleLayer(hs[i]), {}
        ref = OM.moe_forward(x, ol, stages=st)
        assert OM.rel_err(y, ref) <= (1e-3 if T <= 8 else 1e-2), OM.rel_err(y, ref)
        assert bool((OM.topk_margin(OM.router_logits64(x.reshape(T, 1024), ol), 4) > 1e-5).all())
        blk = L.npu["moe_block"]
        assert blk.q_router == QT.F32
        assert torch.equal(blk.stages(T)["topk_ids"].cpu().long(), st["topk_ids"]), f"layer {i}: ids differ"
    g = ts.get_expert("blk.1.ffn_gate_exps.weight", 3)
    assert np.array_equal(g, Q.dequant_matrix(hs[1].gate[3], hs[1].q_gate, 256, 1024))


@pytest.mark.parametrize("T", [1, 10])
def test_qwen_moe_forward_kquant_layers(gpu, tmp_path, T):
    """A model file whose second layer holds Q5_K gate/up and Q6_K down experts, as the
    reference model's blk.1 / blk.34 outliers (qwen/forward.py:495-498): the drop-in runs
    every layer on the device (the K-quant experts transcoded once to I8 rows), where
    the reference keeps a per-expert CPU dequant + F.linear for them.  Bar: 1e-3, except
    the IQ layer at T > 8 (the prefill GEMMs, 1e-2)."""
    from npu_amd import gguf_file
    hs = [synth.host_moe_layer(70, D=1024, FF=256, E=32, k=4, q_gate=QT.IQ3_XXS, q_down=QT.IQ4_XS),
          synth.host_moe_layer(71, D=1024, FF=256, E=32, k=4, q_gate=QT.Q5_K, q_down=QT.Q6_K)]
    path = tmp_path / "moe_kq.gguf"
    synth.write_gguf_model(path, hs)
    ts = gguf_file.TensorStore(path)
    layers = [qwen_moe.MoELayer.load(ts, i) for i in range(2)]
    qwen_moe.enable_npu(layers, ops=("router", "experts"))
    x = torch.from_numpy(synth.host_input(13, T, 1024)).reshape(1, T, 1024)
    for i, L in enumerate(layers):
        y = qwen_moe.moe_forward(x, L, ts.cfg)
        ref = OM.moe_forward(x, OM.OracleLayer(hs[i]))
        bar = 1e-2 if (i == 0 and T > 8) else 1e-3
        assert OM.rel_err(y, ref) <= bar, (i, OM.rel_err(y, ref))



def test_enable_npu_attention_and_ssm_cores(gpu):
    """enable_npu over a model's (core, moe) pairs (qwen/forward.py:775, 813-831): an attention
    core gets ``wo`` (attn_o) and ``wqkv`` (attn_qkv, split (8192, 512, 512)), a Gated
    DeltaNet core ``w_in`` / ``w_gate`` / ``w_out`` (ssm), at the shapes of
    qwen/test_npu_{attn_o,attn_qkv,ssm}.py; each output against float64 F.linear of the bf16
    weight (the operators stage weights in bf16, as the reference does) at rel <= 1e-5.  Ops
    that are not asked for leave their keys absent, and a core of the other kind is left alone."""
    from types import SimpleNamespace

    g = torch.Generator().manual_seed(11)

    def w(*shape):
        return torch.randn(*shape, generator=g) * 0.02

    attn = SimpleNamespace(wq=w(8192, 2048), wk=w(512, 2048), wv=w(512, 2048), wo=w(2048, 4096), npu=None)
    ssm = SimpleNamespace(w_in=w(8192, 2048), w_gate=w(4096, 2048), w_out=w(2048, 4096), npu=None)
    hs = [synth.host_moe_layer(70 + i, D=2048, FF=256, E=16, k=4) for i in range(2)]
    ts = qwen_moe.SyntheticTensorStore(hs)
    model = SimpleNamespace(layers=[(ssm, qwen_moe.MoELayer.load(ts, 0)), (attn, qwen_moe.MoELayer.load(ts, 1))])
    qwen_moe.enable_npu(model, ops=("router", "attn_o", "attn_qkv", "ssm"))
    assert set(attn.npu) == {"wo", "wqkv"} and set(ssm.npu) == {"w_in", "w_gate", "w_out"}
    assert all("moe_block" in moe.npu and "router" in moe.npu for _, moe in model.layers)

    def ref(x, W):
        return (x.double() @ W.to(torch.bfloat16).double().T).float()

    x = torch.randn(2048, generator=g) * 0.05               # post-norm hidden state scale
    xo = torch.randn(4096, generator=g) * 0.05
    checks = [("attn_o", attn.npu["wo"](xo), ref(xo, attn.wo)),
              ("attn_qkv", attn.npu["wqkv"](x), ref(x, torch.cat([attn.wq, attn.wk, attn.wv]))),
              ("ssm_in", ssm.npu["w_in"](x), ref(x, ssm.w_in)),
              ("ssm_gate", ssm.npu["w_gate"](x), ref(x, ssm.w_gate)),
              ("ssm_out", ssm.npu["w_out"](xo), ref(xo, ssm.w_out))]
    for name, y, yr in checks:
        assert y.shape == yr.shape, name
        assert OM.rel_err(y, yr) <= 1e-5, f"{name}: rel {OM.rel_err(y, yr):.3e}"
    assert attn.npu["wqkv"].out_splits == (8192, 512, 512)
    q, k, v = attn.npu["wqkv"](x).split((8192, 512, 512))
    assert OM.rel_err(k, ref(x, attn.wk)) <= 1e-5 and OM.rel_err(v, ref(x, attn.wv)) <= 1e-5
    # only what is asked for
    attn2 = SimpleNamespace(wq=attn.wq, wk=attn.wk, wv=attn.wv, wo=attn.wo, npu=None)
    ssm2 = SimpleNamespace(w_in=ssm.w_in, w_gate=ssm.w_gate, w_out=ssm.w_out, npu=None)
    qwen_moe.enable_npu(SimpleNamespace(layers=[(attn2, qwen_moe.MoELayer.load(ts, 0)),
                                                (ssm2, qwen_moe.MoELayer.load(ts, 1))]), ops=("attn_o",))
    assert set(attn2.npu) == {"wo"} and ssm2.npu is None
