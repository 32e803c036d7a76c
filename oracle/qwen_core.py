"""CPU restatement of the reference's attention and Gated DeltaNet layers and its
decoder step -- test infrastructure (oracle), never the product path.

Follows BojanFaletic/NPU ``qwen/forward.py`` in torch fp32, step by step:

* ``build_partial_rope_cache`` / ``apply_partial_rope``: :64-97 (cos/sin tables of
  ``[max_pos, rope_dim]``; the first ``rope_dim`` lanes of a head rotate as halves
  ``(x1, x2) -> (x1 cos - x2 sin, x2 cos + x1 sin)``, the rest pass through);
* ``attn_forward``: :133-239 (RMSNorm, gated Q with ``[q_h | gate_h]`` interleaved per
  head, per-head Q/K RMSNorm, partial RoPE at ``start_pos``, GQA by repeating each KV
  head, the KV cache concatenated along time, fp32 softmax with a causal mask for
  T > 1, output times ``sigmoid(gate)``, ``wo``);
* ``ssm_forward``: :292-431 (RMSNorm, ``w_in`` / ``w_gate`` projections, alpha/beta
  with ``softplus(alpha + dt_bias) * a`` and ``sigmoid(beta)``, the depthwise causal
  conv1d of kernel 4 over ``[conv_state, x]`` with SiLU, per-head L2 normalisation of q
  and k, K heads tiled onto V heads, q scaled by ``1/sqrt(Sk)``, the delta-rule
  recurrence ``S = S exp(g); d = (v - S^T k) beta; S += k d^T; o = S^T q``, the gated
  RMSNorm ``rmsnorm(o, ssm_norm) * silu(z)``, ``w_out``);
* ``decoder_forward``: :834-893 for the core layers and the MoE glue
  (``x = x + core(x); x = x + moe(rms_norm(x, post_norm))``), then the output norm and
  ``lm_head``.

Pinning (``tests/test_oracle_core.py``): RoPE against rotation matrices built from
its definition (angles theta^(-2i/rd) pos, norm preserved, position 0 the identity,
rotations compose by adding positions, pass-through lanes untouched); attention
against closed forms (one cached position returns v, equal keys return the mean of
v, GQA head mapping, causal prefill equals token-by-token decode); the delta rule
against closed forms (decay 1 and beta 0 keep the state, a zero state with beta 1
stores k v^T and returns v (k . q), orthonormal keys with decay 1 accumulate a
sum, exp(g) scales the state) and a prefill loop equal to token-by-token decode; the
conv against its definition with a one-hot kernel.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from oracle.moe import rms_norm


# ------------------------------------------------------------------ RoPE
def build_partial_rope_cache(rope_dim: int, max_pos: int, theta: float):
    """(cos, sin) tables [max_pos, rope_dim] in fp32 (qwen/forward.py:64-78)."""
    inv = 1.0 / (theta ** (torch.arange(0, rope_dim, 2, dtype=torch.float32) / rope_dim))
    ang = torch.outer(torch.arange(max_pos, dtype=torch.float32), inv)
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos(), ang.sin()


def apply_partial_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, rope_dim: int) -> torch.Tensor:
    """x [B, T, H, Dh], cos / sin [T, rope_dim] (qwen/forward.py:81-97)."""
    half = rope_dim // 2
    xr, xp = x[..., :rope_dim], x[..., rope_dim:]
    rot = torch.cat([-xr[..., half:], xr[..., :half]], dim=-1)
    c, s = cos[None, :, None, :], sin[None, :, None, :]
    return torch.cat([xr * c + rot * s, xp], dim=-1)


# ------------------------------------------------------------ layers
@dataclass
class CoreCfg:
    """The Config fields the core layers read (qwen/model.py:32-59)."""

    d_model: int = 2048
    n_head: int = 16
    n_head_kv: int = 2
    head_dim: int = 256
    rope_dim: int = 64
    rope_theta: float = 10_000_000.0
    rms_eps: float = 1e-6
    ssm_d_conv: int = 4
    ssm_d_inner: int = 4096
    ssm_d_state: int = 128
    ssm_n_k_heads: int = 16
    ssm_n_v_heads: int = 32


@dataclass
class AttnW:
    """AttnLayer's tensors (qwen/forward.py:104-130), fp32."""

    attn_norm: torch.Tensor
    post_norm: torch.Tensor
    wq: torch.Tensor      # [2 Hq Dh, D]
    wk: torch.Tensor      # [Hkv Dh, D]
    wv: torch.Tensor
    wo: torch.Tensor      # [D, Hq Dh]
    q_norm: torch.Tensor  # [Dh]
    k_norm: torch.Tensor


@dataclass
class SSMW:
    """SSMLayer's tensors (qwen/forward.py:246-284), fp32."""

    attn_norm: torch.Tensor
    post_norm: torch.Tensor
    w_in: torch.Tensor    # [conv_ch, D]
    w_gate: torch.Tensor  # [d_inner, D]
    conv1d: torch.Tensor  # [conv_ch, conv_k]
    a: torch.Tensor       # [Hv]
    alpha: torch.Tensor   # [Hv, D]
    beta: torch.Tensor    # [Hv, D]
    dt_bias: torch.Tensor  # [Hv]
    ssm_norm: torch.Tensor  # [Sv]
    w_out: torch.Tensor   # [D, d_inner]


def attn_forward(x: torch.Tensor, L: AttnW, cfg: CoreCfg, cos: torch.Tensor, sin: torch.Tensor,
                 kv_cache, start_pos: int):
    """x [B, T, D] -> (out [B, T, D], (k, v) cache [B, T_total, Hq, Dh]) (qwen/forward.py:133-239)."""
    B, T, D = x.shape
    Hq, Hkv, Dh, rd = cfg.n_head, cfg.n_head_kv, cfg.head_dim, cfg.rope_dim
    h = rms_norm(x, L.attn_norm, cfg.rms_eps)
    qf = F.linear(h, L.wq).view(B, T, Hq, 2, Dh)
    q, gate = qf[..., 0, :], qf[..., 1, :]
    k = F.linear(h, L.wk).view(B, T, Hkv, Dh)
    v = F.linear(h, L.wv).view(B, T, Hkv, Dh)
    q = rms_norm(q, L.q_norm, cfg.rms_eps)
    k = rms_norm(k, L.k_norm, cfg.rms_eps)
    c, s = cos[start_pos:start_pos + T], sin[start_pos:start_pos + T]
    q = apply_partial_rope(q, c, s, rd)
    k = apply_partial_rope(k, c, s, rd)
    k = k.repeat_interleave(Hq // Hkv, dim=2)
    v = v.repeat_interleave(Hq // Hkv, dim=2)
    if kv_cache is not None:
        k = torch.cat([kv_cache[0], k], dim=1)
        v = torch.cat([kv_cache[1], v], dim=1)
    qt, kt, vt = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    scores = torch.matmul(qt, kt.transpose(-2, -1)) / (Dh ** 0.5)
    Tk = kt.shape[-2]
    if T > 1:
        mask = torch.arange(Tk)[None, :] > (torch.arange(T) + start_pos)[:, None]
        scores = scores.masked_fill(mask, float("-inf"))
    p = F.softmax(scores.float(), dim=-1).to(q.dtype)
    o = torch.matmul(p, vt).transpose(1, 2).contiguous()
    o = (o * torch.sigmoid(gate)).view(B, T, Hq * Dh)
    return F.linear(o, L.wo), (k, v)


def l2_norm(x: torch.Tensor, eps: float) -> torch.Tensor:
    """x / sqrt(max(sum x^2, eps)) over the last axis (qwen/forward.py:287-291)."""
    return x / x.pow(2).sum(-1, keepdim=True).clamp_min(eps).sqrt()


def ssm_forward(x: torch.Tensor, L: SSMW, cfg: CoreCfg, state):
    """x [B, T, D] -> (out [B, T, D], (conv_state [B, C, k-1], S [B, Hv, Sk, Sv]))
    (qwen/forward.py:292-431)."""
    B, T, D = x.shape
    Hv, Hk, Sk = cfg.ssm_n_v_heads, cfg.ssm_n_k_heads, cfg.ssm_d_state
    Sv, Ck, di, ck = Sk, Hk * Sk, cfg.ssm_d_inner, cfg.ssm_d_conv
    C = 2 * Ck + di
    h = rms_norm(x, L.attn_norm, cfg.rms_eps)
    mixed = F.linear(h, L.w_in)
    z = F.linear(h, L.w_gate)
    g = F.softplus(F.linear(h, L.alpha) + L.dt_bias) * L.a
    beta = torch.sigmoid(F.linear(h, L.beta))
    if state is None:
        conv_state = torch.zeros(B, C, ck - 1)
        S = torch.zeros(B, Hv, Sk, Sv)
    else:
        conv_state, S = state
    cin = torch.cat([conv_state, mixed.transpose(1, 2)], dim=-1)          # [B, C, T + k - 1]
    conv = F.silu(F.conv1d(cin, L.conv1d.unsqueeze(1), groups=C)).transpose(1, 2)
    new_conv = cin[..., -(ck - 1):].contiguous()
    q = l2_norm(conv[..., :Ck].reshape(B, T, Hk, Sk), cfg.rms_eps).repeat(1, 1, Hv // Hk, 1)
    k = l2_norm(conv[..., Ck:2 * Ck].reshape(B, T, Hk, Sk), cfg.rms_eps).repeat(1, 1, Hv // Hk, 1)
    v = conv[..., 2 * Ck:].reshape(B, T, Hv, Sv)
    q = q * (1.0 / Sk ** 0.5)
    outs = []
    for t in range(T):
        S = S * torch.exp(g[:, t])[..., None, None]
        sk = torch.einsum("bhkv,bhk->bhv", S, k[:, t])
        d = (v[:, t] - sk) * beta[:, t][..., None]
        S = S + torch.einsum("bhk,bhv->bhkv", k[:, t], d)
        outs.append(torch.einsum("bhkv,bhk->bhv", S, q[:, t]))
    o = torch.stack(outs, dim=1)
    o = rms_norm(o, L.ssm_norm, cfg.rms_eps).reshape(B, T, Hv * Sv) * F.silu(z)
    return F.linear(o, L.w_out), (new_conv, S)


def decoder_forward(tokens, emb: torch.Tensor, layers, output_norm: torch.Tensor, lm_head: torch.Tensor,
                    cfg: CoreCfg, cos: torch.Tensor, sin: torch.Tensor, caches=None, start_pos: int = 0):
    """tokens -> (logits [T, vocab], caches) (qwen/forward.py:834-893).  ``layers``: per
    layer ``(core, moe)`` with core an ``AttnW`` or ``SSMW`` and moe an
    ``oracle.moe.OracleLayer`` (no RMSNorm of its own); ``caches`` per layer: the
    attention (k, v) tuple or the SSM (conv_state, S) tuple, or None."""
    from oracle.moe import moe_forward
    caches = list(caches) if caches is not None else [None] * len(layers)
    x = emb[torch.as_tensor(list(tokens), dtype=torch.long)].unsqueeze(0)
    for i, (core, moe) in enumerate(layers):
        if isinstance(core, AttnW):
            y, caches[i] = attn_forward(x, core, cfg, cos, sin, caches[i], start_pos)
        else:
            y, caches[i] = ssm_forward(x, core, cfg, caches[i])
        x = x + y
        x = x + moe_forward(rms_norm(x, core.post_norm, cfg.rms_eps), moe)
    x = rms_norm(x, output_norm, cfg.rms_eps)
    return F.linear(x, lm_head).squeeze(0), caches
