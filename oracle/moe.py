"""CPU restatement of the reference MoE block -- test infrastructure (oracle).

Follows BojanFaletic/NPU ``qwen/forward.py:563-665`` (``moe_forward``, CPU
branch 652-663) step by step in torch fp32:

1. shared expert: three fp32 ``F.linear`` on dequantised shared weights,
   ``silu(gate) * up`` then down (:592-598), scaled by the scalar gate
   ``sigmoid(x . w_gate_inp_sh)`` (:599-600);
2. router: ``F.linear(x, w_router)`` (:608), softmax over all experts in fp32
   (:609), ``topk`` (:610), renormalise with ``clamp_min(1e-20)`` (:611);
3. ``torch.unique`` of the picked ids (:612) and, per picked expert in
   ascending id order, ``nonzero`` gather (:623-629), per-call dequant of that
   expert (``MoELayer.dequant_one`` -> ``TensorStore.get_expert``, :480-491,
   qwen/model.py:230-277), gate/up/SwiGLU/down ``F.linear`` (:656-659) and a
   weighted ``index_add_`` (:663);
4. ``out_routed + shared_out`` (:665).

``rms_norm`` follows :58-61.  The router logit bias is a synthetic skew used
only by the prefill config (the reference model has none); it is added to the
logits before the softmax.

Pinning: the router/softmax/top-k/index_add stages are torch library routines;
the composed block is cross-checked against an fp64 dense restatement
(``moe_forward_dense64``: every expert's full product, weighted by a dense
routing matrix) and against the committed small fixture
``tests/golden/moe_small.npz``.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from oracle.quants import dequant_matrix


def from_bf16(b: np.ndarray) -> np.ndarray:
    """bf16 bits (uint16) -> fp32 (qwen/model.py:292-295)."""
    return (np.ascontiguousarray(b).view(np.uint16).astype(np.uint32) << 16).view(np.float32)


def _f32(a: np.ndarray) -> np.ndarray:
    """Router / shared-gate weights as fp32: fp32 arrays as they are, bf16 bits widened
    (the reference reads both tensors in fp32, qwen/forward.py:41-47)."""
    return np.ascontiguousarray(a, dtype=np.float32) if np.asarray(a).dtype == np.float32 else from_bf16(a)


def rms_norm(x: torch.Tensor, w: torch.Tensor | None, eps: float) -> torch.Tensor:
    """qwen/forward.py:58-61 (w=None means weight 1)."""
    x_f = x.float()
    rms = x_f.pow(2).mean(-1, keepdim=True).add(eps).rsqrt()
    y = x_f * rms
    if w is not None:
        y = y * w.float()
    return y.to(x.dtype)


class OracleLayer:
    """Host view of one block with per-call dequant, mirroring MoELayer."""

    def __init__(self, h):
        self.h = h
        self.w_router = torch.from_numpy(_f32(h.router).reshape(h.E, h.D).copy())
        self.w_gate_inp_sh = (torch.from_numpy(_f32(h.sh_gate_inp).copy())
                              if h.sh_gate_inp is not None else None)
        self.has_shared = h.gate_sh is not None
        self.bias = torch.from_numpy(h.router_bias.copy()) if h.router_bias is not None else None
        self.norm_w = torch.from_numpy(h.norm_w.copy()) if h.norm_w is not None else None

    def dequant_one(self, e: int):
        """(gate[FF,D], up[FF,D], down[D,FF]) fp32, dequantised on every call."""
        h = self.h
        g = dequant_matrix(h.gate[e], h.q_gate, h.FF, h.D)
        u = dequant_matrix(h.up[e], h.q_gate, h.FF, h.D)
        d = dequant_matrix(h.down[e], h.q_down, h.D, h.FF)
        return torch.from_numpy(g), torch.from_numpy(u), torch.from_numpy(d)

    def shared_weights(self):
        h = self.h
        g = dequant_matrix(h.gate_sh, h.q_gate, h.FF, h.D)
        u = dequant_matrix(h.up_sh, h.q_gate, h.FF, h.D)
        d = dequant_matrix(h.down_sh, h.q_down, h.D, h.FF)
        return torch.from_numpy(g), torch.from_numpy(u), torch.from_numpy(d)


def moe_forward(x: torch.Tensor, layer: OracleLayer, *, stages: dict | None = None,
                pre_dequant: dict | None = None) -> torch.Tensor:
    """x [B, T, D] (already normalised, as at qwen/forward.py:881-883) -> [B, T, D]."""
    B, T, D = x.shape
    h = layer.h
    E, K = h.E, h.k
    x_flat = x.reshape(B * T, D)

    if layer.has_shared:
        wg, wu, wd = layer.shared_weights() if pre_dequant is None else pre_dequant["shared"]
        sh_gate = F.linear(x_flat, wg)
        sh_up = F.linear(x_flat, wu)
        sh = F.silu(sh_gate) * sh_up
        shared_out = F.linear(sh, wd)
        if layer.w_gate_inp_sh is not None:
            shared_scalar_gate = torch.sigmoid(x_flat @ layer.w_gate_inp_sh)
            shared_out = shared_out * shared_scalar_gate.unsqueeze(-1)
            if stages is not None:
                stages["shared_expert_gate_sigmoid"] = shared_scalar_gate
    else:
        shared_out = torch.zeros_like(x_flat)

    router_logits = F.linear(x_flat, layer.w_router)
    if layer.bias is not None:
        router_logits = router_logits + layer.bias
    probs = F.softmax(router_logits.float(), dim=-1).to(x.dtype)
    topk_vals, topk_ids = probs.topk(K, dim=-1)
    topk_w = topk_vals / topk_vals.sum(-1, keepdim=True).clamp_min(1e-20)
    picked = torch.unique(topk_ids)
    if stages is not None:
        stages["ffn_moe_logits"] = router_logits
        stages["ffn_moe_probs"] = probs
        stages["topk_ids"] = topk_ids
        stages["ffn_moe_weights_norm"] = topk_w

    out_routed = torch.zeros_like(x_flat)
    for e in picked.tolist():
        mask = topk_ids == e
        idx = mask.nonzero(as_tuple=False)
        tok_idx = idx[:, 0]
        slot_idx = idx[:, 1]
        xe = x_flat[tok_idx]
        we = topk_w[tok_idx, slot_idx]
        if pre_dequant is None:
            wg, wu, wd = layer.dequant_one(int(e))
        else:
            wg, wu, wd = pre_dequant[int(e)]
        g = F.linear(xe, wg)
        u = F.linear(xe, wu)
        y = F.silu(g) * u
        y = F.linear(y, wd)
        out_routed.index_add_(0, tok_idx, y * we.unsqueeze(-1))
    return (out_routed + shared_out).view(B, T, D)


def block_forward(x: torch.Tensor, layer: OracleLayer, eps: float = 1e-6, residual: bool = False,
                  stages: dict | None = None, pre_dequant: dict | None = None) -> torch.Tensor:
    """x [T, D]: y = moe(rmsnorm(x)) (+ x), the glue of qwen/forward.py:880-884."""
    xn = rms_norm(x, layer.norm_w, eps) if layer.norm_w is not None else x
    y = moe_forward(xn.unsqueeze(0), layer, stages=stages, pre_dequant=pre_dequant).squeeze(0)
    return x + y if residual else y


def chain_forward(x: torch.Tensor, layers: list[OracleLayer], eps: float = 1e-6) -> torch.Tensor:
    """Config 5: x_{l+1} = x_l + moe_l(rmsnorm(x_l))."""
    for L in layers:
        x = block_forward(x, L, eps=eps, residual=True)
    return x


def router_logits64(x: torch.Tensor, layer: OracleLayer, eps: float = 1e-6) -> torch.Tensor:
    """fp64 router logits (for near-tie classification of top-k comparisons)."""
    xn = rms_norm(x, layer.norm_w, eps) if layer.norm_w is not None else x
    lg = xn.double() @ layer.w_router.double().T
    if layer.bias is not None:
        lg = lg + layer.bias.double()
    return lg


def topk_margin(logits64: torch.Tensor, k: int) -> torch.Tensor:
    """Gap between the k-th and (k+1)-th largest logit per row (fp64)."""
    s = torch.sort(logits64, dim=-1, descending=True).values
    return s[:, k - 1] - s[:, k]


def moe_forward_dense64(x: torch.Tensor, layer: OracleLayer, eps: float = 1e-6) -> torch.Tensor:
    """Independent fp64 restatement: dense routing matrix times every expert's output.

    Used to cross-check ``moe_forward`` on small blocks (it evaluates all E
    experts, so it is only practical for small E)."""
    h = layer.h
    xn = rms_norm(x, layer.norm_w, eps) if layer.norm_w is not None else x
    xd = xn.double()
    lg = xd @ layer.w_router.double().T
    if layer.bias is not None:
        lg = lg + layer.bias.double()
    p = torch.softmax(lg, dim=-1)
    order = torch.argsort(-p, dim=-1, stable=True)[:, :h.k]
    R = torch.zeros_like(p)
    sel = torch.gather(p, 1, order)
    R.scatter_(1, order, sel / sel.sum(-1, keepdim=True))
    out = torch.zeros_like(xd)
    for e in range(h.E):
        if not bool((R[:, e] != 0).any()):
            continue
        wg, wu, wd = (w.double() for w in layer.dequant_one(e))
        y = (F.silu(xd @ wg.T) * (xd @ wu.T)) @ wd.T
        out += R[:, e:e + 1] * y
    if layer.has_shared:
        wg, wu, wd = (w.double() for w in layer.shared_weights())
        s = (F.silu(xd @ wg.T) * (xd @ wu.T)) @ wd.T
        if layer.w_gate_inp_sh is not None:
            s = s * torch.sigmoid(xd @ layer.w_gate_inp_sh.double()).unsqueeze(-1)
        out += s
    return out


def rel_err(y: torch.Tensor, ref: torch.Tensor) -> float:
    """max|y - ref| / max|ref| (qwen/test_npu_experts.py:91-93)."""
    y = y.double()
    ref = ref.double()
    return float((y - ref).abs().max() / ref.abs().max().clamp_min(1e-300))


def cos(a: torch.Tensor, b: torch.Tensor) -> float:
    af, bf = a.flatten().double(), b.flatten().double()
    return float((af @ bf) / (af.norm() * bf.norm()).clamp_min(1e-300))
