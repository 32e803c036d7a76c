"""Drop-in for the rest of the reference's decoder: gated attention, Gated DeltaNet and
the decoder loop of ``qwen/forward.py``, on the GPU.

Same names and call signatures as the reference:

* ``AttnLayer`` (:100-130) and ``SSMLayer`` (:242-284) with ``.load(ts, i)``;
* ``attn_forward(x, layer, cfg, cos, sin, kv_cache, start_pos)`` (:133-239) and
  ``ssm_forward(x, layer, cfg, ssm_state)`` (:292-431), each returning ``(out, state)``;
* ``build_partial_rope_cache`` (:64-78);
* ``Model`` (:672-709) and ``forward(model, tokens, *, start_pos, kv_caches,
  ssm_states, n_layer, skip_moe)`` (:834-893), returning ``(logits [T, vocab],
  kv_caches, ssm_states)``.

Each core layer runs as one C-ABI call per token (``gm_attn_decode`` /
``gm_ssm_decode``): its large projections are bf16 weights resident in HBM (as the
reference's NPU operators stage them, :813-831), its small ones and all state fp32.
The KV cache is preallocated as ``[max_pos][n_head_kv][head_dim]`` per layer (the
reference concatenates a ``[B, T, n_head, head_dim]`` cache per step, repeating each kv
head over its q heads); the Gated DeltaNet state is ``(conv_state [1, C, k - 1],
S [1, Hv, Sk, Sv])``, the reference's tuple, as device tensors updated in place.
Several tokens (prefill) run the core layers one token at a time, which is the
causal attention of the reference's masked prefill and the token loop of its
recurrence; the MoE block then takes the layer's T tokens at once.  There is no CPU
path: without the built library every call raises.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np
import torch

from npu_amd import _lib as L
from npu_amd._dropin import device
from npu_amd.profiler import profile
from npu_amd.qwen_moe import MoELayer, rms_norm


# ------------------------------------------------------------------ config
@dataclass
class Config:
    """The ``qwen/model.py:Config`` fields the decoder reads (defaults: Qwen3.6-35B-A3B)."""

    d_model: int = 2048
    n_layer: int = 40
    n_head: int = 16
    n_head_kv: int = 2
    head_dim: int = 256
    rms_eps: float = 1e-6
    rope_theta: float = 10_000_000.0
    rope_dim: int = 64
    n_expert: int = 256
    n_expert_used: int = 8
    d_expert_ff: int = 512
    vocab_size: int = 248_320
    ssm_d_conv: int = 4
    ssm_d_inner: int = 4096
    ssm_d_state: int = 128
    ssm_n_k_heads: int = 16
    ssm_n_v_heads: int = 32
    is_attention: list[bool] = field(default_factory=list)


def build_partial_rope_cache(rope_dim: int, max_pos: int, theta: float, dtype=torch.float32, device="cpu"):
    """(cos, sin) [max_pos, rope_dim] (qwen/forward.py:64-78)."""
    inv = 1.0 / (theta ** (torch.arange(0, rope_dim, 2, dtype=torch.float32, device=device) / rope_dim))
    ang = torch.outer(torch.arange(max_pos, dtype=torch.float32, device=device), inv)
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos().to(dtype), ang.sin().to(dtype)


def _t(ts, name: str) -> torch.Tensor:
    return torch.from_numpy(np.array(ts.get(name, dtype="fp32", keep=False), copy=True)).float()


def _bf16_dev(w: torch.Tensor) -> torch.Tensor:
    """An fp32 weight as bf16 bits on the device (the staging of the reference's NpuMatVec)."""
    return w.to(device()).to(torch.bfloat16).contiguous().view(torch.int16)


def _f32_dev(t: torch.Tensor | None) -> torch.Tensor | None:
    return None if t is None else t.to(device(), torch.float32).contiguous()


# ------------------------------------------------------------- attention
@dataclass
class AttnLayer:
    """Same fields as the reference's ``AttnLayer`` (qwen/forward.py:100-130), fp32 host
    tensors; ``gpu`` holds the device copy once built."""

    i: int
    attn_norm: torch.Tensor
    post_norm: torch.Tensor
    wq: torch.Tensor
    wk: torch.Tensor
    wv: torch.Tensor
    wo: torch.Tensor
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    npu: dict | None = None
    gpu: "GpuAttn | None" = field(default=None, repr=False)

    @classmethod
    def load(cls, ts, i: int) -> "AttnLayer":
        p = f"blk.{i}."
        return cls(i=i, attn_norm=_t(ts, p + "attn_norm.weight"), post_norm=_t(ts, p + "post_attention_norm.weight"),
                   wq=_t(ts, p + "attn_q.weight"), wk=_t(ts, p + "attn_k.weight"), wv=_t(ts, p + "attn_v.weight"),
                   wo=_t(ts, p + "attn_output.weight"), q_norm=_t(ts, p + "attn_q_norm.weight"),
                   k_norm=_t(ts, p + "attn_k_norm.weight"))


class GpuAttn:
    """One attention layer resident on the GPU: [wq; wk; wv] and wo as bf16, norms fp32."""

    def __init__(self, layer: AttnLayer, cfg: Config):
        self.cfg = cfg
        self.wqkv = _bf16_dev(torch.cat([layer.wq, layer.wk, layer.wv], dim=0))
        self.wo = _bf16_dev(layer.wo)
        self.attn_norm, self.q_norm, self.k_norm = (_f32_dev(t) for t in (layer.attn_norm, layer.q_norm,
                                                                            layer.k_norm))
        s = L.GmAttnLayer()
        s.wqkv, s.wo = L.ptr(self.wqkv), L.ptr(self.wo)
        s.attn_norm, s.q_norm, s.k_norm = L.ptr(self.attn_norm), L.ptr(self.q_norm), L.ptr(self.k_norm)
        s.eps = float(cfg.rms_eps)
        s.D, s.n_head, s.n_head_kv = cfg.d_model, cfg.n_head, cfg.n_head_kv
        s.head_dim, s.rope_dim = cfg.head_dim, cfg.rope_dim
        if tuple(self.wqkv.shape) != ((2 * cfg.n_head + 2 * cfg.n_head_kv) * cfg.head_dim, cfg.d_model):
            raise ValueError(f"attention weights do not match the config: wqkv {tuple(self.wqkv.shape)}")
        self.struct = s
        self._ws: dict[int, torch.Tensor] = {}

    def workspace(self, max_pos: int) -> torch.Tensor:
        ws = self._ws.get(max_pos)
        if ws is None:
            n = L.lib().gm_attn_workspace_bytes(ctypes.byref(self.struct), max_pos)
            if n == 0:
                raise ValueError(f"gm_attn_workspace_bytes: {L.last_error()}")
            ws = self._ws[max_pos] = torch.empty(n, dtype=torch.uint8, device=self.wo.device)
        return ws

    def step(self, x: torch.Tensor, cache: "KVCache", pos: int, cos: torch.Tensor, sin: torch.Tensor,
             residual: bool, out: torch.Tensor, moe_link=None) -> None:
        """One token; with ``moe_link = (moe struct, moe workspace)`` the layer also forms
        the following MoE block's router inputs (gm_attn_decode_moe)."""
        ws = self.workspace(cache.max_pos)
        flags = L.GM_MOE_RESIDUAL if residual else 0
        if moe_link is None:
            rc = L.lib().gm_attn_decode(ctypes.byref(self.struct), L.ptr(x), L.ptr(out), L.ptr(cache.k),
                                        L.ptr(cache.v), pos, cache.max_pos, L.ptr(cos), L.ptr(sin), flags,
                                        L.ptr(ws), ws.numel(), L.stream_ptr())
            L.check(rc, "gm_attn_decode")
            return
        st, mws = moe_link
        rc = L.lib().gm_attn_decode_moe(ctypes.byref(self.struct), L.ptr(x), L.ptr(out), L.ptr(cache.k),
                                        L.ptr(cache.v), pos, cache.max_pos, L.ptr(cos), L.ptr(sin), flags,
                                        L.ptr(ws), ws.numel(), ctypes.byref(st), L.ptr(mws), mws.numel(),
                                        L.stream_ptr())
        L.check(rc, "gm_attn_decode_moe")


class KVCache:
    """One attention layer's cache, ``[max_pos][n_head_kv][head_dim]`` fp32 for k and v,
    and the number of positions filled."""

    def __init__(self, cfg: Config, max_pos: int, dev=None):
        dev = dev or device()
        self.max_pos = int(max_pos)
        self.k = torch.zeros(self.max_pos, cfg.n_head_kv, cfg.head_dim, device=dev)
        self.v = torch.zeros_like(self.k)
        self.length = 0

    def expanded(self, n_head: int):
        """The reference's cache tuple ([1, length, n_head, head_dim] each, kv heads repeated)."""
        rep = n_head // self.k.shape[1]
        k, v = self.k[:self.length], self.v[:self.length]
        return (k.repeat_interleave(rep, dim=1).unsqueeze(0), v.repeat_interleave(rep, dim=1).unsqueeze(0))


def _rope_on_device(cos: torch.Tensor, sin: torch.Tensor):
    return cos.to(device(), torch.float32).contiguous(), sin.to(device(), torch.float32).contiguous()


def attn_forward(x: torch.Tensor, layer: AttnLayer, cfg: Config, cos: torch.Tensor, sin: torch.Tensor,
                 kv_cache: KVCache | None, start_pos: int, *, residual: bool = False, moe_link=None):
    """x [1, T, D] -> (out [1, T, D], kv_cache) (reference :133-239).  ``residual`` returns
    x + out (the decoder's ``x = x + y``) in the same pass; ``moe_link`` (T = 1) also forms
    the following MoE block's router inputs (see ``forward``)."""
    B, T, D = x.shape
    if B != 1:
        raise ValueError("attn_forward: batch 1 (the reference's decoder runs one sequence)")
    if moe_link is not None and T != 1:
        raise ValueError("attn_forward: a MoE link is for one token")
    if layer.gpu is None:
        layer.gpu = GpuAttn(layer, cfg)
    if kv_cache is None:
        kv_cache = KVCache(cfg, cos.shape[0])
    if start_pos != kv_cache.length:
        raise ValueError(f"start_pos {start_pos} != cached length {kv_cache.length}")
    if start_pos + T > kv_cache.max_pos:
        raise ValueError(f"positions up to {start_pos + T} exceed max_pos {kv_cache.max_pos}")
    on_host = not x.is_cuda
    xd = x.reshape(T, D).to(device(), torch.float32).contiguous()
    cd, sd = _rope_on_device(cos, sin)
    y = torch.empty_like(xd)
    with profile("attn.decode"):
        for t in range(T):
            layer.gpu.step(xd[t], kv_cache, start_pos + t, cd, sd, residual, y[t], moe_link)
            kv_cache.length += 1
    y = y.view(1, T, D)
    return (y.cpu() if on_host else y), kv_cache


# ---------------------------------------------------------------- SSM
@dataclass
class SSMLayer:
    """Same fields as the reference's ``SSMLayer`` (qwen/forward.py:242-284)."""

    i: int
    attn_norm: torch.Tensor
    post_norm: torch.Tensor
    w_in: torch.Tensor
    w_gate: torch.Tensor
    conv1d: torch.Tensor
    a: torch.Tensor
    alpha: torch.Tensor
    beta: torch.Tensor
    dt_bias: torch.Tensor
    ssm_norm: torch.Tensor
    w_out: torch.Tensor
    npu: dict | None = None
    gpu: "GpuSsm | None" = field(default=None, repr=False)

    @classmethod
    def load(cls, ts, i: int) -> "SSMLayer":
        p = f"blk.{i}."
        return cls(i=i, attn_norm=_t(ts, p + "attn_norm.weight"), post_norm=_t(ts, p + "post_attention_norm.weight"),
                   w_in=_t(ts, p + "attn_qkv.weight"), w_gate=_t(ts, p + "attn_gate.weight"),
                   conv1d=_t(ts, p + "ssm_conv1d.weight"), a=_t(ts, p + "ssm_a"), alpha=_t(ts, p + "ssm_alpha.weight"),
                   beta=_t(ts, p + "ssm_beta.weight"), dt_bias=_t(ts, p + "ssm_dt.bias"),
                   ssm_norm=_t(ts, p + "ssm_norm.weight"), w_out=_t(ts, p + "ssm_out.weight"))


class GpuSsm:
    """One Gated DeltaNet layer resident on the GPU: w_in / w_gate / w_out bf16, the rest fp32."""

    def __init__(self, layer: SSMLayer, cfg: Config):
        self.cfg = cfg
        self.w_in, self.w_gate, self.w_out = (_bf16_dev(w) for w in (layer.w_in, layer.w_gate, layer.w_out))
        (self.alpha, self.beta, self.conv1d, self.a, self.dt_bias, self.ssm_norm,
         self.attn_norm) = (_f32_dev(t) for t in (layer.alpha, layer.beta, layer.conv1d, layer.a, layer.dt_bias,
                                                   layer.ssm_norm, layer.attn_norm))
        s = L.GmSsmLayer()
        s.w_in, s.w_gate, s.w_out = L.ptr(self.w_in), L.ptr(self.w_gate), L.ptr(self.w_out)
        s.alpha, s.beta, s.conv1d = L.ptr(self.alpha), L.ptr(self.beta), L.ptr(self.conv1d)
        s.a, s.dt_bias, s.ssm_norm, s.attn_norm = L.ptr(self.a), L.ptr(self.dt_bias), L.ptr(self.ssm_norm), \
            L.ptr(self.attn_norm)
        s.eps = float(cfg.rms_eps)
        s.D, s.n_k_heads, s.n_v_heads = cfg.d_model, cfg.ssm_n_k_heads, cfg.ssm_n_v_heads
        s.d_state, s.conv_k = cfg.ssm_d_state, cfg.ssm_d_conv
        self.C = 2 * cfg.ssm_n_k_heads * cfg.ssm_d_state + cfg.ssm_n_v_heads * cfg.ssm_d_state
        if tuple(self.conv1d.shape) != (self.C, cfg.ssm_d_conv) or tuple(self.w_in.shape) != (self.C, cfg.d_model):
            raise ValueError("SSM weights do not match the config")
        self.struct = s
        n = L.lib().gm_ssm_workspace_bytes(ctypes.byref(s))
        if n == 0:
            raise ValueError(f"gm_ssm_workspace_bytes: {L.last_error()}")
        self.ws = torch.empty(n, dtype=torch.uint8, device=self.w_out.device)

    def new_state(self):
        c = self.cfg
        conv = torch.zeros(1, self.C, c.ssm_d_conv - 1, device=self.w_out.device)
        S = torch.zeros(1, c.ssm_n_v_heads, c.ssm_d_state, c.ssm_d_state, device=self.w_out.device)
        return conv, S

    def step(self, x: torch.Tensor, state, residual: bool, out: torch.Tensor, moe_link=None) -> None:
        """One token; with ``moe_link = (moe struct, moe workspace)`` the layer also forms
        the following MoE block's router inputs (gm_ssm_decode_moe)."""
        conv, S = state
        flags = L.GM_MOE_RESIDUAL if residual else 0
        if moe_link is None:
            rc = L.lib().gm_ssm_decode(ctypes.byref(self.struct), L.ptr(x), L.ptr(out), L.ptr(conv), L.ptr(S),
                                       flags, L.ptr(self.ws), self.ws.numel(), L.stream_ptr())
            L.check(rc, "gm_ssm_decode")
            return
        st, mws = moe_link
        rc = L.lib().gm_ssm_decode_moe(ctypes.byref(self.struct), L.ptr(x), L.ptr(out), L.ptr(conv), L.ptr(S),
                                       flags, L.ptr(self.ws), self.ws.numel(), ctypes.byref(st), L.ptr(mws),
                                       mws.numel(), L.stream_ptr())
        L.check(rc, "gm_ssm_decode_moe")


def ssm_forward(x: torch.Tensor, layer: SSMLayer, cfg: Config, ssm_state, *, residual: bool = False,
                moe_link=None):
    """x [1, T, D] -> (out [1, T, D], (conv_state [1, C, k-1], S [1, Hv, Sk, Sv])) (reference
    :292-431).  A state given as the reference's tuple of (possibly host) tensors is
    copied to the device once; the returned tuple is device tensors, updated in place by
    later calls.  ``moe_link`` (T = 1) also forms the following MoE block's router inputs."""
    B, T, D = x.shape
    if B != 1:
        raise ValueError("ssm_forward: batch 1 (the reference's decoder runs one sequence)")
    if moe_link is not None and T != 1:
        raise ValueError("ssm_forward: a MoE link is for one token")
    if layer.gpu is None:
        layer.gpu = GpuSsm(layer, cfg)
    if ssm_state is None:
        state = layer.gpu.new_state()
    else:
        state = tuple(t.to(device(), torch.float32).contiguous() for t in ssm_state)
    on_host = not x.is_cuda
    xd = x.reshape(T, D).to(device(), torch.float32).contiguous()
    y = torch.empty_like(xd)
    with profile("ssm.decode"):
        for t in range(T):
            layer.gpu.step(xd[t], state, residual, y[t], moe_link)
    y = y.view(1, T, D)
    return (y.cpu() if on_host else y), state


# -------------------------------------------------------------- decoder
@dataclass
class Model:
    """The reference's ``Model`` (qwen/forward.py:672-709): embedding, output norm, lm_head,
    ``(core, moe)`` layer pairs and the RoPE tables; lm_head staged as bf16 on first use."""

    cfg: Config
    token_embd: torch.Tensor
    output_norm: torch.Tensor
    lm_head: torch.Tensor
    layers: list
    rope_cos: torch.Tensor
    rope_sin: torch.Tensor
    gpu: dict = field(default_factory=dict, repr=False)

    @classmethod
    def load(cls, ts, *, max_pos: int = 4096) -> "Model":
        cfg = ts.cfg
        cos, sin = build_partial_rope_cache(cfg.rope_dim, max_pos, cfg.rope_theta)
        layers = []
        for i in range(cfg.n_layer):
            core = AttnLayer.load(ts, i) if cfg.is_attention[i] else SSMLayer.load(ts, i)
            layers.append((core, MoELayer.load(ts, i)))
        return cls(cfg=cfg, token_embd=_t(ts, "token_embd.weight"), output_norm=_t(ts, "output_norm.weight"),
                   lm_head=_t(ts, "output.weight"), layers=layers, rope_cos=cos, rope_sin=sin)


def forward(model: Model, tokens, *, start_pos: int = 0, kv_caches=None, ssm_states=None,
            n_layer: int | None = None, skip_moe: bool = False, link_moe: bool = True):
    """tokens -> (logits [T, vocab], kv_caches, ssm_states) for one sequence (reference
    :834-893): embedding, per layer ``x = x + core(x)`` then
    ``x = x + moe_forward(rms_norm(x, post_norm))``, the output norm and lm_head, all on
    the GPU (logits stay there).  At T = 1 (``link_moe``) each core layer whose MoE block
    fits the T = 1 accumulator kernels also forms that block's router inputs
    (gm_attn_decode_moe / gm_ssm_decode_moe), and the block runs without its router launch
    (gm_moe_forward_acc); the logits equal the unlinked ones to fp32 rounding."""
    cfg = model.cfg
    n = n_layer if n_layer is not None else cfg.n_layer
    kv_caches = list(kv_caches) if kv_caches is not None else [None] * cfg.n_layer
    ssm_states = list(ssm_states) if ssm_states is not None else [None] * cfg.n_layer
    g = model.gpu
    if "embd" not in g:
        g["embd"] = model.token_embd.to(device(), torch.float32).contiguous()
        g["onorm"] = _f32_dev(model.output_norm)
        g["lm_head"] = _bf16_dev(model.lm_head)
        g["rope"] = _rope_on_device(model.rope_cos, model.rope_sin)
    if isinstance(tokens, torch.Tensor):                 # already on the device: nothing to copy (capturable)
        tok = tokens.to(device(), torch.long).reshape(-1)
    else:
        tok = torch.as_tensor(list(tokens), dtype=torch.long, device=device())
    T = tok.numel()
    x = g["embd"][tok].view(1, T, cfg.d_model).contiguous()
    cos, sin = g["rope"]
    for i in range(n):
        core, moe = model.layers[i]
        link = _moe_link(g, i, core, moe, cfg) if (link_moe and not skip_moe and T == 1) else None
        if cfg.is_attention[i]:
            with profile("forward.attn"):
                x, kv_caches[i] = attn_forward(x, core, cfg, cos, sin, kv_caches[i], start_pos, residual=True,
                                               moe_link=link)
        else:
            with profile("forward.ssm"):
                x, ssm_states[i] = ssm_forward(x, core, cfg, ssm_states[i], residual=True, moe_link=link)
        if not skip_moe:
            with profile("forward.moe"):
                x = _moe_residual(g, i, x, core, moe, cfg, linked=link is not None)
    with profile("forward.out_norm"):
        xn = _rms_norm_dev(x, model.output_norm, cfg.rms_eps, w_dev=g["onorm"])
    with profile("forward.lm_head"):
        logits = torch.empty(T, g["lm_head"].shape[0], device=device())
        rc = L.lib().gm_matvec(L.GM_QTYPE_BF16, L.ptr(g["lm_head"]), logits.shape[1], cfg.d_model,
                               L.ptr(xn.view(T, -1)), T, L.ptr(logits), L.stream_ptr())
        L.check(rc, "gm_matvec")
    return logits, kv_caches, ssm_states


def _moe_struct(g: dict, i: int, core, moe, cfg: Config):
    """(struct, block) of layer i's MoE step: a copy of the block's struct carrying
    post_norm as its RMSNorm weight (the block's own struct, which the drop-in moe_forward
    uses, is left as it is).  ``moe`` is a ``MoELayer`` or an already resident
    ``GpuMoeBlock``."""
    from npu_amd.moe import GpuMoeBlock
    from npu_amd.qwen_moe import _build_block
    if isinstance(moe, GpuMoeBlock):
        blk = moe
    else:
        if moe.npu is None:
            moe.npu = {}
        blk = moe.npu.get("moe_block")
        if blk is None:
            blk = moe.npu["moe_block"] = _build_block(moe)
    key = ("moe", i)
    if key not in g:
        nw = _f32_dev(core.post_norm)
        st = L.GmMoeLayer.from_buffer_copy(blk.struct)
        st.norm_w, st.norm_eps = L.ptr(nw), float(cfg.rms_eps)
        g[key] = (st, nw, L.lib().gm_moe_chain_fused(ctypes.byref(st), 1, 1) == 1 and bool(st.router_t))
    return g[key][0], blk


def _moe_link(g: dict, i: int, core, moe, cfg: Config):
    """(struct, workspace) for a core layer to form layer i's MoE router inputs, or None
    when the block does not fit the T = 1 accumulator kernels."""
    st, blk = _moe_struct(g, i, core, moe, cfg)
    return (st, blk.workspace(1)) if g[("moe", i)][2] else None


def _moe_residual(g: dict, i: int, x: torch.Tensor, core, moe, cfg: Config, linked: bool = False) -> torch.Tensor:
    """x + moe_forward(rms_norm(x, core.post_norm)) in one gm_moe_forward call (with the
    residual flag), or, ``linked``, one gm_moe_forward_acc call on the router inputs the
    core layer formed."""
    from npu_amd import ops
    st, blk = _moe_struct(g, i, core, moe, cfg)
    T, D = x.shape[1], x.shape[2]
    xf = x.reshape(T, D).contiguous()
    y = torch.empty_like(xf)
    if linked:
        ws = blk.workspace(1)
        rc = L.lib().gm_moe_forward_acc(ctypes.byref(st), L.ptr(xf), L.ptr(y), L.GM_MOE_RESIDUAL, L.ptr(ws),
                                        ws.numel(), L.stream_ptr())
        L.check(rc, "gm_moe_forward_acc")
    else:
        ops.moe_forward_raw(st, xf, y, blk.workspace(T), residual=True)
    return y.view(1, T, D)


def _rms_norm_dev(x: torch.Tensor, w: torch.Tensor, eps: float, w_dev: torch.Tensor | None = None) -> torch.Tensor:
    """rms_norm (reference :58-61) over the last axis, on the GPU (gm_rms_norm)."""
    D = x.shape[-1]
    xf = x.reshape(-1, D).contiguous()
    wd = w_dev if w_dev is not None else _f32_dev(w)
    y = torch.empty_like(xf)
    L.check(L.lib().gm_rms_norm(L.ptr(xf), L.ptr(wd), D, xf.shape[0], float(eps), L.ptr(y), L.stream_ptr()),
            "gm_rms_norm")
    return y.view(x.shape)


__all__ = ["Config", "AttnLayer", "SSMLayer", "KVCache", "Model", "attn_forward", "ssm_forward", "forward",
           "build_partial_rope_cache", "rms_norm"]
