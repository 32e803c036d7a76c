"""GPU parity of the core layers and the decoder loop (gm_attn_decode, gm_ssm_decode,
npu_amd.qwen_core.forward) against the oracle restatement of qwen/forward.py:133-239,
292-431 and 834-893.

Weights of the large projections are bf16 values (the device stages them as bf16, as
the reference's NPU operators do), so the oracle's fp32 products use the same numbers;
everything else is fp32.  Bar: rel = max|y - ref| / max|ref| <= 1e-4 per layer and
step (fp32 throughout, sums in another order), <= 2e-3 for the logits of the decoder
with MoE blocks (fp32-accumulate decode MoE, 1e-3 per block).  The attention runs past
the 64-position chunk of its split softmax; the SSM state is compared after every step.
The decoder's llama.cpp parity stays unpinned (no model file or llama.cpp here).
"""
import numpy as np
import pytest
import torch

from npu_amd import qwen_core as QN, qwen_moe, synth
from oracle import moe as OM
from oracle import qwen_core as QC

pytestmark = pytest.mark.gpu


def _bf(t):
    return t.to(torch.bfloat16).float()


def _cfgs(small: bool):
    if small:
        return (QC.CoreCfg(d_model=512, n_head=4, n_head_kv=2, head_dim=128, rope_dim=32, rope_theta=1e6,
                           ssm_d_inner=256, ssm_d_state=64, ssm_n_k_heads=2, ssm_n_v_heads=4),
                QN.Config(d_model=512, n_head=4, n_head_kv=2, head_dim=128, rope_dim=32, rope_theta=1e6,
                          ssm_d_inner=256, ssm_d_state=64, ssm_n_k_heads=2, ssm_n_v_heads=4))
    return QC.CoreCfg(), QN.Config()


def _attn_weights(cfg, seed):
    g = torch.Generator().manual_seed(seed)
    D, Hq, Hkv, Dh = cfg.d_model, cfg.n_head, cfg.n_head_kv, cfg.head_dim

    def w(*s, sc=0.02):
        return torch.randn(*s, generator=g) * sc
    return dict(attn_norm=1 + w(D, sc=0.1), post_norm=1 + w(D, sc=0.1), wq=_bf(w(2 * Hq * Dh, D)),
                wk=_bf(w(Hkv * Dh, D)), wv=_bf(w(Hkv * Dh, D)), wo=_bf(w(D, Hq * Dh)), q_norm=1 + w(Dh, sc=0.1),
                k_norm=1 + w(Dh, sc=0.1))


def _ssm_weights(cfg, seed):
    g = torch.Generator().manual_seed(seed)
    D, Hv, Hk, S = cfg.d_model, cfg.ssm_n_v_heads, cfg.ssm_n_k_heads, cfg.ssm_d_state
    C = 2 * Hk * S + Hv * S

    def w(*s, sc=0.02):
        return torch.randn(*s, generator=g) * sc
    return dict(attn_norm=1 + w(D, sc=0.1), post_norm=1 + w(D, sc=0.1), w_in=_bf(w(C, D)), w_gate=_bf(w(Hv * S, D)),
                conv1d=w(C, cfg.ssm_d_conv, sc=0.5), a=-torch.rand(Hv, generator=g) * 2,
                alpha=w(Hv, D, sc=0.05), beta=w(Hv, D, sc=0.05), dt_bias=w(Hv, sc=0.5),
                ssm_norm=1 + w(S, sc=0.1), w_out=_bf(w(D, Hv * S)))


def _rel(a, b):
    return float((a.double().cpu() - b.double().cpu()).abs().max() / b.double().cpu().abs().max())


@pytest.mark.parametrize("small", [True, False])
def test_attention_decode_steps(gpu, small):
    ocfg, ncfg = _cfgs(small)
    print(f"attention decode case small={small}", flush=True)
    W = _attn_weights(ocfg, 1)
    OL = QC.AttnW(**W)
    NL = QN.AttnLayer(i=0, **W)
    steps = 70                                            # past one 64-position chunk of the split softmax
    cos, sin = QC.build_partial_rope_cache(ocfg.rope_dim, 96, ocfg.rope_theta)
    xs = torch.randn(1, steps, ocfg.d_model, generator=torch.Generator().manual_seed(2))
    ocache, ncache = None, None
    for t in range(steps):
        yo, ocache = QC.attn_forward(xs[:, t:t + 1], OL, ocfg, cos, sin, ocache, t)
        yn, ncache = QN.attn_forward(xs[:, t:t + 1].to(gpu), NL, ncfg, cos, sin, ncache, t)
        assert _rel(yn, yo) <= 1e-4, f"step {t}: rel {_rel(yn, yo):.2e}"
    rep = ocfg.n_head // ocfg.n_head_kv
    assert _rel(ncache.k[:steps], ocache[0][0, :, ::rep]) <= 1e-5
    assert torch.equal(ncache.v[:steps].cpu(), ocache[1][0, :, ::rep]) or _rel(ncache.v[:steps], ocache[1][0, :, ::rep]) <= 1e-6
    # residual flag and a prefill of several tokens (one decode step per token, causal)
    x5 = torch.randn(1, 5, ocfg.d_model, generator=torch.Generator().manual_seed(3))
    yo5, _ = QC.attn_forward(x5, OL, ocfg, cos, sin, None, 0)
    yn5, c5 = QN.attn_forward(x5.to(gpu), NL, ncfg, cos, sin, None, 0, residual=True)
    assert c5.length == 5
    assert _rel(yn5 - x5.to(gpu), yo5) <= 1e-4


@pytest.mark.parametrize("small", [True, False])
def test_ssm_decode_steps(gpu, small):
    ocfg, ncfg = _cfgs(small)
    print(f"ssm decode case small={small}", flush=True)
    W = _ssm_weights(ocfg, 4)
    OL = QC.SSMW(**W)
    NL = QN.SSMLayer(i=0, **W)
    xs = torch.randn(1, 12, ocfg.d_model, generator=torch.Generator().manual_seed(5))
    ost, nst = None, None
    for t in range(12):
        yo, ost = QC.ssm_forward(xs[:, t:t + 1], OL, ocfg, ost)
        yn, nst = QN.ssm_forward(xs[:, t:t + 1].to(gpu), NL, ncfg, nst)
        assert _rel(yn, yo) <= 1e-4, f"step {t}: rel {_rel(yn, yo):.2e}"
        assert _rel(nst[0], ost[0]) <= 1e-5, f"step {t}: conv state"
        assert _rel(nst[1], ost[1]) <= 1e-4, f"step {t}: recurrent state rel {_rel(nst[1], ost[1]):.2e}"
    # the reference's state tuple hands over (host tensors in, device tensors out) and the
    # residual flag
    x1 = torch.randn(1, 3, ocfg.d_model, generator=torch.Generator().manual_seed(6))
    yo, ost2 = QC.ssm_forward(x1, OL, ocfg, ost)
    yn, nst2 = QN.ssm_forward(x1.to(gpu), NL, ncfg, tuple(t.cpu() for t in nst), residual=True)
    assert _rel(yn - x1.to(gpu), yo) <= 1e-4 and _rel(nst2[1], ost2[1]) <= 1e-4


def test_attention_long_context(gpu):
    """600 decode steps (10 chunks of the split softmax: the combine's unrolled 8-chunk body and
    its remainder) against the oracle, checked every 50 steps and at the end."""
    ocfg, ncfg = _cfgs(True)
    print("attention long-context case: 600 steps", flush=True)
    W = _attn_weights(ocfg, 21)
    OL, NL = QC.AttnW(**W), QN.AttnLayer(i=0, **W)
    steps = 600
    cos, sin = QC.build_partial_rope_cache(ocfg.rope_dim, steps + 8, ocfg.rope_theta)
    xs = torch.randn(1, steps, ocfg.d_model, generator=torch.Generator().manual_seed(22))
    ocache, ncache = None, None
    for t in range(steps):
        yo, ocache = QC.attn_forward(xs[:, t:t + 1], OL, ocfg, cos, sin, ocache, t)
        yn, ncache = QN.attn_forward(xs[:, t:t + 1].to(gpu), NL, ncfg, cos, sin, ncache, t)
        if t % 50 == 49 or t == steps - 1:
            assert _rel(yn, yo) <= 1e-4, f"step {t}: rel {_rel(yn, yo):.2e}"


def test_core_layers_general_paths(gpu):
    """The shapes the launch merges leave on their own kernels: a rope_dim above 64 whose half
    is no power of two (k_attn_prep before the partials) and d_state 256 (the recurrence in
    32-column blocks, then the gated norm), step by step against the oracle."""
    print("core general-path case: rope_dim 96, d_state 256", flush=True)
    kw = dict(d_model=512, n_head=4, n_head_kv=2, head_dim=128, rope_dim=96, rope_theta=1e6,
              ssm_d_inner=1024, ssm_d_state=256, ssm_n_k_heads=2, ssm_n_v_heads=4)
    ocfg, ncfg = QC.CoreCfg(**kw), QN.Config(**kw)
    W = _attn_weights(ocfg, 11)
    OL, NL = QC.AttnW(**W), QN.AttnLayer(i=0, **W)
    steps = 66                                            # past one 64-position chunk
    cos, sin = QC.build_partial_rope_cache(ocfg.rope_dim, 80, ocfg.rope_theta)
    xs = torch.randn(1, steps, ocfg.d_model, generator=torch.Generator().manual_seed(12))
    ocache, ncache = None, None
    for t in range(steps):
        yo, ocache = QC.attn_forward(xs[:, t:t + 1], OL, ocfg, cos, sin, ocache, t)
        yn, ncache = QN.attn_forward(xs[:, t:t + 1].to(gpu), NL, ncfg, cos, sin, ncache, t)
        assert _rel(yn, yo) <= 1e-4, f"attention step {t}: rel {_rel(yn, yo):.2e}"
    W = _ssm_weights(ocfg, 13)
    OS, NS = QC.SSMW(**W), QN.SSMLayer(i=0, **W)
    xs = torch.randn(1, 6, ocfg.d_model, generator=torch.Generator().manual_seed(14))
    ost, nst = None, None
    for t in range(6):
        yo, ost = QC.ssm_forward(xs[:, t:t + 1], OS, ocfg, ost)
        yn, nst = QN.ssm_forward(xs[:, t:t + 1].to(gpu), NS, ncfg, nst)
        assert _rel(yn, yo) <= 1e-4, f"ssm step {t}: rel {_rel(yn, yo):.2e}"
        assert _rel(nst[1], ost[1]) <= 1e-4, f"ssm step {t}: recurrent state rel {_rel(nst[1], ost[1]):.2e}"


def test_decoder_forward_prefill_and_decode(gpu):
    """A 4-layer model (three Gated DeltaNet layers and one attention layer, the reference
    model's pattern; D = 512, MoE E = 16, k = 4, FF = 256; vocab 1000): a 5-token prompt,
    then 3 decode steps, logits against the oracle decoder at every call."""
    print("decoder case: 4 layers, prompt 5, 3 steps", flush=True)
    ocfg, ncfg = _cfgs(True)
    n_layer = 4
    ncfg.n_layer, ncfg.is_attention = n_layer, [(i + 1) % 4 == 0 for i in range(n_layer)]
    ncfg.n_expert, ncfg.n_expert_used, ncfg.d_expert_ff = 16, 4, 256
    hs = [synth.host_moe_layer(600 + i, D=512, FF=256, E=16, k=4) for i in range(n_layer)]
    ts = qwen_moe.SyntheticTensorStore(hs)
    g = torch.Generator().manual_seed(7)
    V = 1000
    emb = torch.randn(V, 512, generator=g)
    onorm = 1 + 0.1 * torch.randn(512, generator=g)
    lm_head = _bf(torch.randn(V, 512, generator=g) * 0.05)
    cores_o, cores_n = [], []
    for i in range(n_layer):
        if ncfg.is_attention[i]:
            W = _attn_weights(ocfg, 20 + i)
            cores_o.append(QC.AttnW(**W))
            cores_n.append(QN.AttnLayer(i=i, **W))
        else:
            W = _ssm_weights(ocfg, 20 + i)
            cores_o.append(QC.SSMW(**W))
            cores_n.append(QN.SSMLayer(i=i, **W))
    cos, sin = QC.build_partial_rope_cache(ocfg.rope_dim, 64, ocfg.rope_theta)
    model = QN.Model(cfg=ncfg, token_embd=emb, output_norm=onorm, lm_head=lm_head,
                     layers=[(cores_n[i], qwen_moe.MoELayer.load(ts, i)) for i in range(n_layer)],
                     rope_cos=cos, rope_sin=sin)
    olayers = [(cores_o[i], OM.OracleLayer(hs[i])) for i in range(n_layer)]
    prompt = [3, 141, 59, 265, 358]
    lo, oc = QC.decoder_forward(prompt, emb, olayers, onorm, lm_head, ocfg, cos, sin)
    ln, kv, st = QN.forward(model, prompt)
    assert ln.shape == (5, V)
    assert _rel(ln, lo) <= 2e-3, f"prompt logits rel {_rel(ln, lo):.2e}"
    pos = len(prompt)
    for step, tok in enumerate([int(lo[-1].argmax()), 7, 999]):
        lo, oc = QC.decoder_forward([tok], emb, olayers, onorm, lm_head, ocfg, cos, sin, oc, pos)
        ln, kv, st = QN.forward(model, [tok], start_pos=pos, kv_caches=kv, ssm_states=st)
        assert _rel(ln, lo) <= 2e-3, f"decode step {step}: logits rel {_rel(ln, lo):.2e}"
        pos += 1


@pytest.mark.parametrize("router_f32,E,bias", [(False, 64, False), (True, 512, True)])
def test_decoder_linked_moe_router(gpu, router_f32, E, bias):
    """Decode steps with every core layer linked to its MoE block (gm_attn_decode_moe /
    gm_ssm_decode_moe form the block's router inputs, gm_moe_forward_acc runs it without the
    router launch) against the same steps unlinked (gm_attn_decode / gm_ssm_decode, then
    gm_moe_forward): top-k ids equal at every layer and step, logits rel <= 1e-5 (the same
    router dot products added in another order), and both against the oracle decoder at
    2e-3.  4 layers (three Gated DeltaNet, one attention), D = 512, MoE k = 8, FF = 512 (a
    block that fits the T = 1 accumulator kernels) with a bf16 router and E = 64, or an fp32
    router with a bias and E = 512 (two accumulator positions per thread); a 3-token prompt,
    then 3 steps."""
    print(f"decoder case: linked MoE router, router_f32={router_f32} E={E} bias={bias}", flush=True)
    ocfg, ncfg = _cfgs(True)
    n_layer = 4
    ncfg.n_layer, ncfg.is_attention = n_layer, [(i + 1) % 4 == 0 for i in range(n_layer)]
    ncfg.n_expert, ncfg.n_expert_used, ncfg.d_expert_ff = E, 8, 512
    hs = [synth.host_moe_layer(700 + i, D=512, FF=512, E=E, k=8, router_f32=router_f32, bias=bias)
          for i in range(n_layer)]
    ts = qwen_moe.SyntheticTensorStore(hs)
    g = torch.Generator().manual_seed(11)
    V = 1000
    emb = torch.randn(V, 512, generator=g)
    onorm = 1 + 0.1 * torch.randn(512, generator=g)
    lm_head = _bf(torch.randn(V, 512, generator=g) * 0.05)
    cores_o, cores_n = [], []
    for i in range(n_layer):
        if ncfg.is_attention[i]:
            W = _attn_weights(ocfg, 40 + i)
            cores_o.append(QC.AttnW(**W))
            cores_n.append(QN.AttnLayer(i=i, **W))
        else:
            W = _ssm_weights(ocfg, 40 + i)
            cores_o.append(QC.SSMW(**W))
            cores_n.append(QN.SSMLayer(i=i, **W))
    cos, sin = QC.build_partial_rope_cache(ocfg.rope_dim, 64, ocfg.rope_theta)
    moes = [qwen_moe.MoELayer.load(ts, i) for i in range(n_layer)]
    model = QN.Model(cfg=ncfg, token_embd=emb, output_norm=onorm, lm_head=lm_head,
                     layers=[(cores_n[i], moes[i]) for i in range(n_layer)], rope_cos=cos, rope_sin=sin)
    olayers = [(cores_o[i], OM.OracleLayer(hs[i])) for i in range(n_layer)]

    def ids():
        return [m.npu["moe_block"].stages(1)["topk_ids"].cpu().clone() for m in moes]
    prompt = [5, 77, 901]
    lo, oc = QC.decoder_forward(prompt, emb, olayers, onorm, lm_head, ocfg, cos, sin)
    _, kv_u, st_u = QN.forward(model, prompt, link_moe=False)
    _, kv_l, st_l = QN.forward(model, prompt, link_moe=True)      # T = 3: never linked
    assert all(model.gpu[("moe", i)][2] for i in range(n_layer)), "a MoE block does not fit the linked path"
    pos = len(prompt)
    for step, tok in enumerate([int(lo[-1].argmax()), 3, 512]):
        lo, oc = QC.decoder_forward([tok], emb, olayers, onorm, lm_head, ocfg, cos, sin, oc, pos)
        lu, kv_u, st_u = QN.forward(model, [tok], start_pos=pos, kv_caches=kv_u, ssm_states=st_u, link_moe=False)
        ids_u = ids()
        ll, kv_l, st_l = QN.forward(model, [tok], start_pos=pos, kv_caches=kv_l, ssm_states=st_l, link_moe=True)
        ids_l = ids()
        for li in range(n_layer):
            assert torch.equal(ids_l[li], ids_u[li]), f"step {step} layer {li}: linked ids differ"
        assert _rel(ll, lu) <= 1e-5, f"step {step}: linked vs unlinked logits rel {_rel(ll, lu):.2e}"
        assert _rel(ll, lo) <= 2e-3, f"step {step}: linked logits vs oracle rel {_rel(ll, lo):.2e}"
        pos += 1
