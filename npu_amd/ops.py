"""Functional torch wrappers over the C ABI (device tensors in, device tensors out).

Every function enqueues on torch's current stream and returns without
synchronising.  Weight tensors are raw GGUF bytes (``torch.uint8``) or bf16
bits (``torch.uint16``/``torch.bfloat16``/``torch.int16``) already on the GPU.
"""
from __future__ import annotations

import ctypes

import torch

from npu_amd import _lib as L
from npu_amd.gguf_types import QK, GGMLQuantizationType, block_bytes, block_weights


def _as_bf16_bits(w: torch.Tensor) -> torch.Tensor:
    if w.dtype == torch.bfloat16:
        return w.view(torch.int16)
    if w.dtype in (torch.int16, torch.uint16):
        return w
    raise TypeError(f"bf16 weights must be bfloat16/uint16/int16, got {w.dtype}")


def dequant(qtype: int, raw: torch.Tensor, n_superblocks: int | None = None) -> torch.Tensor:
    """Raw blocks (uint8, on GPU) -> fp32 [n_blocks * block weights] (256, or 32 for Q8_0)."""
    bb = block_bytes(qtype)
    if raw.dtype != torch.uint8:
        raise TypeError(f"raw must be uint8, got {raw.dtype}")
    if n_superblocks is None:
        if raw.numel() % bb:
            raise ValueError(f"{raw.numel()} bytes is not a whole number of {bb}-byte superblocks")
        n_superblocks = raw.numel() // bb
    out = torch.empty(n_superblocks * block_weights(qtype), dtype=torch.float32, device=raw.device)
    L.check(L.lib().gm_dequant_f32(int(qtype), L.ptr(raw), n_superblocks, L.ptr(out), L.stream_ptr()),
            "gm_dequant_f32")
    return out


def transcode_i8(qtype: int, raw: torch.Tensor) -> torch.Tensor:
    """Raw Q8_0 / Q4_K / Q5_K / Q6_K blocks (uint8, on GPU) -> I8 sub-blocks (uint8, 48 bytes
    per 32 weights, in weight order; ``gm_transcode_i8``)."""
    bb, bw = block_bytes(qtype), block_weights(qtype)
    if raw.dtype != torch.uint8:
        raise TypeError(f"raw must be uint8, got {raw.dtype}")
    if raw.numel() % bb:
        raise ValueError(f"{raw.numel()} bytes is not a whole number of {bb}-byte blocks")
    n = raw.numel() // bb
    out = torch.empty(n * bw // 32 * 48, dtype=torch.uint8, device=raw.device)
    L.check(L.lib().gm_transcode_i8(int(qtype), L.ptr(raw.contiguous()), n, L.ptr(out), L.stream_ptr()),
            "gm_transcode_i8")
    return out


def matvec(qtype: int, w: torch.Tensor, M: int, K: int, x: torch.Tensor) -> torch.Tensor:
    """y[..., M] = W[M, K] @ x[..., K] with W raw (IQ4_XS/IQ3_XXS) or bf16."""
    if qtype == GGMLQuantizationType.BF16:
        w = _as_bf16_bits(w)
    elif w.dtype != torch.uint8:
        raise TypeError(f"quantized weights must be uint8, got {w.dtype}")
    if x.shape[-1] != K:
        raise ValueError(f"x last dim {x.shape[-1]} != K={K}")
    xf = x.reshape(-1, K).to(torch.float32).contiguous()
    n_tok = xf.shape[0]
    y = torch.empty((n_tok, M), dtype=torch.float32, device=xf.device)
    L.check(L.lib().gm_matvec(int(qtype), L.ptr(w), M, K, L.ptr(xf), n_tok, L.ptr(y), L.stream_ptr()),
            "gm_matvec")
    return y.reshape(*x.shape[:-1], M)


def swiglu_mlp(q_gu: int, w_gate: torch.Tensor, w_up: torch.Tensor, q_down: int, w_down: torch.Tensor,
               D: int, FF: int, x: torch.Tensor) -> torch.Tensor:
    """down(silu(gate x) * up x) for x[..., D]."""
    if q_gu == GGMLQuantizationType.BF16:
        w_gate, w_up = _as_bf16_bits(w_gate), _as_bf16_bits(w_up)
    if q_down == GGMLQuantizationType.BF16:
        w_down = _as_bf16_bits(w_down)
    xf = x.reshape(-1, D).to(torch.float32).contiguous()
    n_tok = xf.shape[0]
    h = torch.empty((n_tok, FF), dtype=torch.float32, device=xf.device)
    y = torch.empty((n_tok, D), dtype=torch.float32, device=xf.device)
    L.check(L.lib().gm_swiglu_mlp(int(q_gu), L.ptr(w_gate), L.ptr(w_up), int(q_down), L.ptr(w_down), D, FF,
                                  L.ptr(xf), n_tok, L.ptr(h), L.ptr(y), L.stream_ptr()), "gm_swiglu_mlp")
    return y.reshape(*x.shape[:-1], D)


def router_topk(w_router: torch.Tensor, x: torch.Tensor, k: int, *, bias: torch.Tensor | None = None,
                w_sh_gate: torch.Tensor | None = None, norm_w: torch.Tensor | None = None,
                eps: float = 1e-6):
    """Router logits, top-k ids (int32), renormalised weights and sigmoid shared gate.

    Returns ``(ids [T,k], weights [T,k], logits [T,E], sh_gate [T] or None)``.
    """
    w = _as_bf16_bits(w_router)
    E, D = w.shape
    xf = x.reshape(-1, D).to(torch.float32).contiguous()
    T = xf.shape[0]
    dev = xf.device
    ids = torch.empty((T, k), dtype=torch.int32, device=dev)
    wts = torch.empty((T, k), dtype=torch.float32, device=dev)
    logits = torch.empty((T, E), dtype=torch.float32, device=dev)
    shg = torch.empty((T,), dtype=torch.float32, device=dev) if w_sh_gate is not None else None
    wsh = _as_bf16_bits(w_sh_gate).contiguous() if w_sh_gate is not None else None
    b = bias.to(torch.float32).contiguous() if bias is not None else None
    nw = norm_w.to(torch.float32).contiguous() if norm_w is not None else None
    L.check(L.lib().gm_router_topk(L.ptr(w.contiguous()), L.ptr(b), L.ptr(xf), T, D, E, k, L.ptr(wsh), L.ptr(nw),
                                   float(eps), L.ptr(ids), L.ptr(wts), L.ptr(logits), L.ptr(shg), L.stream_ptr()),
            "gm_router_topk")
    return ids, wts, logits, shg


def moe_dispatch(ids: torch.Tensor, E: int):
    """Expert-sorted dispatch of top-k ids [T, k]: (counts[E], offsets[E+1], sorted_pairs[T*k])."""
    ids32 = ids.to(torch.int32).contiguous()
    T, k = ids32.shape
    dev = ids32.device
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    pairs = torch.empty(T * k, dtype=torch.int32, device=dev)
    L.check(L.lib().gm_moe_dispatch(L.ptr(ids32), T, k, E, L.ptr(counts), L.ptr(offsets), L.ptr(pairs),
                                    L.stream_ptr()), "gm_moe_dispatch")
    return counts, offsets, pairs


def moe_workspace_bytes(layer: L.GmMoeLayer, T: int) -> int:
    n = L.lib().gm_moe_workspace_bytes(ctypes.byref(layer), T)
    if n == 0:
        raise ValueError(f"gm_moe_workspace_bytes: {L.last_error()}")
    return int(n)


def moe_workspace_offsets(layer: L.GmMoeLayer, T: int) -> dict[str, int]:
    o = [ctypes.c_size_t() for _ in range(4)]
    L.check(L.lib().gm_moe_workspace_offsets(ctypes.byref(layer), T, *[ctypes.byref(v) for v in o]),
            "gm_moe_workspace_offsets")
    return dict(zip(("logits", "ids", "weights", "sh_gate"), (v.value for v in o)))


def moe_forward_raw(layer: L.GmMoeLayer, x: torch.Tensor, y: torch.Tensor, ws: torch.Tensor,
                    residual: bool = False, stage: int = 0, path: str = "auto") -> None:
    """Enqueue the fused MoE block (stage 0) or one of its stages 1..3: y = moe(rmsnorm(x)) (+ x).

    path: "auto" (decode kernels for T <= 8, prefill GEMMs above), "decode" or "prefill"."""
    T = x.shape[0]
    flags = L.GM_MOE_RESIDUAL if residual else 0
    if stage == 0:
        fn = {"auto": "gm_moe_forward", "decode": "gm_moe_decode", "prefill": "gm_moe_prefill"}[path]
        rc = getattr(L.lib(), fn)(ctypes.byref(layer), L.ptr(x), L.ptr(y), T, flags, L.ptr(ws), ws.numel(),
                                  L.stream_ptr())
    else:
        rc = L.lib().gm_moe_forward_stage(ctypes.byref(layer), L.ptr(x), L.ptr(y), T, flags, L.ptr(ws),
                                          ws.numel(), stage, L.stream_ptr())
    L.check(rc, "gm_moe_forward")


def moe_chain_raw(layers, x: torch.Tensor, y: torch.Tensor, buf: torch.Tensor | None, workspaces,
                  residual: bool = False) -> None:
    """Enqueue gm_moe_chain over ``layers`` (GmMoeLayer structs) with one workspace per layer:
    x_{l+1} = moe_l(rmsnorm_l(x_l)) (+ x_l); the last layer writes y, the others alternate
    between y and buf."""
    n = len(layers)
    if n < 1 or len(workspaces) != n:
        raise ValueError("moe_chain_raw: one workspace per layer")
    arr = (L.GmMoeLayer * n)(*layers)
    wsp = (ctypes.c_void_p * n)(*[L.ptr(w) for w in workspaces])
    wsb = (ctypes.c_size_t * n)(*[w.numel() for w in workspaces])
    flags = L.GM_MOE_RESIDUAL if residual else 0
    rc = L.lib().gm_moe_chain(arr, n, L.ptr(x), L.ptr(y), L.ptr(buf) if buf is not None else None, x.shape[0],
                              flags, wsp, wsb, L.stream_ptr())
    L.check(rc, "gm_moe_chain")



def moe_chain_mode(layers, T: int) -> int:
    """gm_moe_chain's path for ``layers`` at ``T`` tokens: 1 = the accumulator-linked T = 1
    kernels (one router launch, then two launches per layer), 2 = the combine-linked T > 1
    kernels (one router launch, then four launches per layer; needs distinct workspaces per
    layer), 0 = one gm_moe_forward per layer."""
    n = len(layers)
    arr = (L.GmMoeLayer * n)(*layers)
    rc = L.lib().gm_moe_chain_fused(arr, n, T)
    if rc < 0:
        L.check(rc, "gm_moe_chain_fused")
    return int(rc)


def moe_chain_fused(layers, T: int) -> bool:
    """Whether gm_moe_chain links consecutive layers at ``T`` tokens (mode 1 or 2 above)
    rather than running one gm_moe_forward per layer."""
    return moe_chain_mode(layers, T) > 0
