"""The core-layer oracle (oracle/qwen_core.py: qwen/forward.py:64-97, 133-239, 292-431)
against what the mathematics fixes, not against a second copy of the same formulas.

* RoPE: the cos/sin tables against angles pos * theta^(-2i/rd) in float64; the
  rotation against explicit 2x2 rotations of the pairs (i, i + rd/2) (an interleaved
  pairing (2i, 2i+1), a swapped sign or a wrong frequency order fails); norm kept;
  position 0 the identity; rotations compose by adding positions; lanes past rd pass.
* Attention: with one cached position the softmax is 1, so the output is
  wo (v_{h // rep} * sigmoid(gate)) (a wrong GQA mapping -- tiling instead of
  repeating -- or a missing gate fails); two positions with equal keys give the mean
  of their values; a causal prefill of T tokens equals T one-token decodes.
* Gated DeltaNet: the conv against its definition with one-hot kernels; with decay 1
  and beta = 1 a zero state becomes k v^T and the output v (k . q) (a sign error in
  d = v - S^T k, or S q instead of S^T q, fails); with beta = 0 the state is only
  decayed by exp(g); a prefill of T tokens equals T one-token steps; the L2 norm
  gives unit vectors.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import qwen_core as QC
from oracle.moe import rms_norm


def _g(seed):
    return torch.Generator().manual_seed(seed)


def test_rope_tables_and_rotation():
    rd, theta, P = 16, 10_000.0, 40
    cos, sin = QC.build_partial_rope_cache(rd, P, theta)
    i = np.arange(rd // 2)
    ang = np.arange(P)[:, None] * theta ** (-2.0 * i / rd)[None, :]
    assert np.allclose(cos.numpy(), np.cos(np.concatenate([ang, ang], 1)), atol=2e-6)
    assert np.allclose(sin.numpy(), np.sin(np.concatenate([ang, ang], 1)), atol=2e-6)
    Dh = 24
    x = torch.randn(1, 3, 2, Dh, generator=_g(1))
    pos = torch.tensor([0, 5, 31])
    y = QC.apply_partial_rope(x, cos[pos], sin[pos], rd)
    # explicit rotation of pair (j, j + rd/2) by the angle of position p
    for t, p in enumerate(pos.tolist()):
        for j in range(rd // 2):
            a = p * theta ** (-2.0 * j / rd)
            c, s = math.cos(a), math.sin(a)
            x1, x2 = x[0, t, :, j].double(), x[0, t, :, j + rd // 2].double()
            assert torch.allclose(y[0, t, :, j].double(), c * x1 - s * x2, atol=1e-5)
            assert torch.allclose(y[0, t, :, j + rd // 2].double(), s * x1 + c * x2, atol=1e-5)
    assert torch.equal(y[..., rd:], x[..., rd:])
    assert torch.allclose(y[:, 0], x[:, 0], atol=0)                      # position 0: cos 1, sin 0
    assert torch.allclose(y.norm(dim=-1), x.norm(dim=-1), rtol=1e-5)
    # rotations compose: rope(rope(x, a), b) = rope(x, a + b)
    a, b = 7, 11
    ya = QC.apply_partial_rope(x[:, :1], cos[a:a + 1], sin[a:a + 1], rd)
    yab = QC.apply_partial_rope(ya, cos[b:b + 1], sin[b:b + 1], rd)
    y2 = QC.apply_partial_rope(x[:, :1], cos[a + b:a + b + 1], sin[a + b:a + b + 1], rd)
    assert torch.allclose(yab, y2, atol=1e-5)


def _attn(cfg, seed, scale=0.1):
    g = _g(seed)
    D, Hq, Hkv, Dh = cfg.d_model, cfg.n_head, cfg.n_head_kv, cfg.head_dim

    def w(*s):
        return torch.randn(*s, generator=g) * scale
    return QC.AttnW(attn_norm=1 + w(D), post_norm=1 + w(D), wq=w(2 * Hq * Dh, D), wk=w(Hkv * Dh, D),
                    wv=w(Hkv * Dh, D), wo=w(D, Hq * Dh), q_norm=1 + w(Dh), k_norm=1 + w(Dh))


CFG_A = QC.CoreCfg(d_model=64, n_head=4, n_head_kv=2, head_dim=16, rope_dim=8, rope_theta=1000.0)


def test_attention_single_position_closed_form():
    cfg, L = CFG_A, _attn(CFG_A, 2)
    cos, sin = QC.build_partial_rope_cache(cfg.rope_dim, 8, cfg.rope_theta)
    x = torch.randn(1, 1, cfg.d_model, generator=_g(3))
    y, (k, v) = QC.attn_forward(x, L, cfg, cos, sin, None, 0)
    h = rms_norm(x, L.attn_norm, cfg.rms_eps).reshape(-1).double()
    vv = (L.wv.double() @ h).view(cfg.n_head_kv, cfg.head_dim)
    gate = (L.wq.double() @ h).view(cfg.n_head, 2, cfg.head_dim)[:, 1]
    rep = cfg.n_head // cfg.n_head_kv
    o = torch.stack([vv[hq // rep] for hq in range(cfg.n_head)]) * torch.sigmoid(gate)
    want = L.wo.double() @ o.reshape(-1)
    assert torch.allclose(y.reshape(-1).double(), want, rtol=1e-5, atol=1e-6)
    assert k.shape == (1, 1, cfg.n_head, cfg.head_dim)


def test_attention_equal_keys_mean_of_values_and_causal_prefill():
    cfg, L = CFG_A, _attn(CFG_A, 4)
    cos, sin = QC.build_partial_rope_cache(cfg.rope_dim, 16, cfg.rope_theta)
    x = torch.randn(1, 5, cfg.d_model, generator=_g(5))
    y_pf, cache_pf = QC.attn_forward(x, L, cfg, cos, sin, None, 0)
    cache, ys = None, []
    for t in range(5):
        y_t, cache = QC.attn_forward(x[:, t:t + 1], L, cfg, cos, sin, cache, t)
        ys.append(y_t)
    assert torch.allclose(torch.cat(ys, 1), y_pf, rtol=1e-5, atol=1e-6)
    assert torch.allclose(cache[0], cache_pf[0]) and torch.allclose(cache[1], cache_pf[1])
    # a cache of two positions with the same key: the softmax is 1/2 each, so the
    # attention output is the mean of the two values
    cache2 = (cache[0][:, :1].repeat(1, 2, 1, 1), cache[1][:, :2])
    x1 = torch.randn(1, 1, cfg.d_model, generator=_g(6))
    L0 = QC.AttnW(**{**L.__dict__, "wk": torch.zeros_like(L.wk)})        # the new token's key is 0 ...
    cache3 = (torch.zeros_like(cache2[0]), cache2[1])                     # ... as are the cached ones
    y3, _ = QC.attn_forward(x1, L0, cfg, cos, sin, cache3, 2)
    h = rms_norm(x1, L.attn_norm, cfg.rms_eps).reshape(-1).double()
    v_new = (L.wv.double() @ h).view(cfg.n_head_kv, cfg.head_dim)
    rep = cfg.n_head // cfg.n_head_kv
    vs = torch.stack([cache3[1][0, 0].double(), cache3[1][0, 1].double(),
                      torch.stack([v_new[hq // rep] for hq in range(cfg.n_head)])])
    gate = (L.wq.double() @ h).view(cfg.n_head, 2, cfg.head_dim)[:, 1]
    want = L.wo.double() @ (vs.mean(0) * torch.sigmoid(gate)).reshape(-1)
    assert torch.allclose(y3.reshape(-1).double(), want, rtol=1e-5, atol=1e-6)


CFG_S = QC.CoreCfg(d_model=64, ssm_d_conv=4, ssm_d_inner=32, ssm_d_state=8, ssm_n_k_heads=2, ssm_n_v_heads=4)


def _ssm(cfg, seed, *, a=None, beta_bias=None):
    g = _g(seed)
    D, Hv, Hk, S = cfg.d_model, cfg.ssm_n_v_heads, cfg.ssm_n_k_heads, cfg.ssm_d_state
    C = 2 * Hk * S + Hv * S

    def w(*s, sc=0.2):
        return torch.randn(*s, generator=g) * sc
    return QC.SSMW(attn_norm=1 + w(D, sc=0.1), post_norm=1 + w(D, sc=0.1), w_in=w(C, D), w_gate=w(Hv * S, D),
                   conv1d=w(C, cfg.ssm_d_conv, sc=0.5), a=(-torch.rand(Hv, generator=g) if a is None else a),
                   alpha=w(Hv, D, sc=0.05), beta=w(Hv, D, sc=0.05), dt_bias=w(Hv, sc=0.5),
                   ssm_norm=1 + w(S, sc=0.1), w_out=w(D, Hv * S))


def test_ssm_conv_one_hot_and_l2():
    cfg = CFG_S
    L = _ssm(cfg, 7)
    C = L.conv1d.shape[0]
    x = torch.randn(1, 3, cfg.d_model, generator=_g(8))
    h = rms_norm(x, L.attn_norm, cfg.rms_eps)
    mixed = F.linear(h, L.w_in)[0]                                       # [3, C]
    # kernel [0, 0, 0, 1]: the conv passes the current input
    L1 = QC.SSMW(**{**L.__dict__, "conv1d": torch.tensor([0., 0., 0., 1.]).repeat(C, 1)})
    _, (cs, _) = QC.ssm_forward(x, L1, cfg, None)
    assert torch.allclose(cs[0], mixed[-3:].T, atol=1e-6)                # state: the last 3 inputs
    # kernel [1, 0, 0, 0] over a zero state: step t sees input t - 3
    L2 = QC.SSMW(**{**L.__dict__, "conv1d": torch.tensor([1., 0., 0., 0.]).repeat(C, 1)})
    st = (torch.randn(1, C, 3, generator=_g(9)), torch.zeros(1, cfg.ssm_n_v_heads, 8, 8))
    _, (cs2, _) = QC.ssm_forward(x[:, :1], L2, cfg, st)
    assert torch.equal(cs2[0, :, :2], st[0][0, :, 1:]) and torch.allclose(cs2[0, :, 2], mixed[0], atol=1e-6)
    v = torch.randn(5, 8, generator=_g(10))
    assert torch.allclose(QC.l2_norm(v, 1e-6).norm(dim=-1), torch.ones(5), atol=1e-6)


def _conv_qkv(x, L, cfg, state=None):
    """The recurrence's q, k, v and the step's g / beta for one token, restated from the
    definitions (conv over [state, input], SiLU, L2 norm, tiling, scale)."""
    Hv, Hk, S = cfg.ssm_n_v_heads, cfg.ssm_n_k_heads, cfg.ssm_d_state
    C = 2 * Hk * S + Hv * S
    h = rms_norm(x, L.attn_norm, cfg.rms_eps)[0, 0].double()
    mixed = L.w_in.double() @ h
    cs = torch.zeros(C, 3, dtype=torch.float64) if state is None else state.double()
    cin = torch.cat([cs, mixed[:, None]], 1)
    conv = F.silu((cin * L.conv1d.double()).sum(1))
    q = conv[:Hk * S].view(Hk, S)
    k = conv[Hk * S:2 * Hk * S].view(Hk, S)
    q, k = q / q.norm(dim=-1, keepdim=True), k / k.norm(dim=-1, keepdim=True)
    rep = Hv // Hk
    q = torch.cat([q] * rep) / math.sqrt(S)                               # tile: head i uses K head i % Hk
    k = torch.cat([k] * rep)
    v = conv[2 * Hk * S:].view(Hv, S)
    return q, k, v


def test_delta_rule_closed_forms():
    cfg = CFG_S
    Hv, S = cfg.ssm_n_v_heads, cfg.ssm_d_state
    # decay 1 (a = 0) and beta = 1 (huge beta logits): a zero state becomes k v^T
    L = _ssm(cfg, 11, a=torch.zeros(Hv))
    L = QC.SSMW(**{**L.__dict__, "beta": torch.zeros_like(L.beta), "alpha": torch.zeros_like(L.alpha)})
    Lb = QC.SSMW(**{**L.__dict__, "beta": torch.zeros_like(L.beta)})
    x = torch.randn(1, 1, cfg.d_model, generator=_g(12))
    # beta = sigmoid(0) = 1/2 here; use the closed form with beta 1/2: S = k (v/2)^T, o = (v/2)(k . q)
    _, (_, Sn) = QC.ssm_forward(x, Lb, cfg, None)
    q, k, v = _conv_qkv(x, Lb, cfg)
    want = torch.einsum("hk,hv->hkv", k, v * 0.5)
    assert torch.allclose(Sn[0].double(), want, atol=1e-6)
    # the output before the gated norm is o = S^T q = (v/2) (k . q): check through the norm
    o = (v * 0.5) * (k * q).sum(-1, keepdim=True)
    h = rms_norm(x, L.attn_norm, cfg.rms_eps)[0, 0].double()
    z = L.w_gate.double() @ h
    on = (o / torch.sqrt(o.pow(2).mean(-1, keepdim=True) + cfg.rms_eps)) * L.ssm_norm.double()
    want_y = L.w_out.double() @ (on.reshape(-1) * F.silu(z))
    y, _ = QC.ssm_forward(x, Lb, cfg, None)
    assert torch.allclose(y.reshape(-1).double(), want_y, rtol=1e-4, atol=1e-5)
    # beta = 0 (logits -100): the state is only decayed by exp(g)
    L0 = QC.SSMW(**{**L.__dict__, "beta": torch.zeros_like(L.beta), "a": -torch.rand(Hv, generator=_g(13))})
    L0.beta[:, 0] = -1e4 / (x.abs().max() + 1)                           # a large negative logit ...
    S0 = torch.randn(1, Hv, S, S, generator=_g(14))
    st = (torch.zeros(1, L0.w_in.shape[0], 3), S0)
    hx = rms_norm(x, L0.attn_norm, cfg.rms_eps)[0, 0]
    bl = F.linear(hx, L0.beta)
    if bool((torch.sigmoid(bl) == 0).all()):                              # ... when it underflows to 0
        _, (_, S1) = QC.ssm_forward(x, L0, cfg, st)
        gdec = F.softplus(F.linear(hx, L0.alpha) + L0.dt_bias) * L0.a
        assert torch.allclose(S1[0], S0[0] * torch.exp(gdec)[:, None, None], rtol=1e-6)


def test_ssm_prefill_equals_steps():
    cfg = CFG_S
    L = _ssm(cfg, 15)
    x = torch.randn(1, 6, cfg.d_model, generator=_g(16))
    y_pf, (c_pf, S_pf) = QC.ssm_forward(x, L, cfg, None)
    st, ys = None, []
    for t in range(6):
        y_t, st = QC.ssm_forward(x[:, t:t + 1], L, cfg, st)
        ys.append(y_t)
    assert torch.allclose(torch.cat(ys, 1), y_pf, rtol=1e-5, atol=1e-6)
    assert torch.allclose(st[0], c_pf, atol=2e-6) and torch.allclose(st[1], S_pf, atol=2e-6)   # batched GEMM rounding
