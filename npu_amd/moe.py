"""Device-resident MoE block: raw GGUF expert stacks in HBM + the fused forward.

``GpuMoeBlock`` owns one block's weights on the GPU in the layout GGUF stores
them (experts outermost, rows of raw superblocks), fills the C struct
``gm_moe_layer`` and runs ``gm_moe_forward``: router -> top-k -> expert
grouping -> gate/up SwiGLU -> down -> weighted combine + shared expert, all on
the device from device-resident ids.  Reference semantics:
``qwen/forward.py:563-665`` (moe_forward).
"""
from __future__ import annotations

import numpy as np
import torch

from npu_amd import _lib as L
from npu_amd import ops
from npu_amd.gguf_types import GGMLQuantizationType as QT, row_bytes


def _dev(a, dtype=None, device="cuda") -> torch.Tensor | None:
    if a is None:
        return None
    if isinstance(a, torch.Tensor):
        t = a.to(device)
    else:
        arr = np.ascontiguousarray(a)
        if not arr.flags.writeable:           # e.g. a read-only memory map of a GGUF file
            arr = arr.copy()
        if arr.dtype == np.uint16:
            arr = arr.view(np.int16)
        t = torch.from_numpy(arr).to(device)
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    return t.contiguous()


# Expert tensors in these types (the Q5_K / Q6_K outliers of the reference model,
# qwen/forward.py:495-498, Q8_0 / Q6_K shared experts, and Q4_K) are transcoded on
# the device once, at load, into I8 rows (int8 quants, fp32 scales per 16 weights,
# an fp32 offset per 32; exact): the decode kernels multiply them on v_dot4 like the
# IQ formats.
_KQUANTS = (QT.Q8_0, QT.Q4_K, QT.Q5_K, QT.Q6_K)
I8 = L.GM_QTYPE_I8


def _row_bytes(q: int, K: int) -> int:
    return K // 32 * 48 if q == I8 else row_bytes(q, K)


def _kquant_to_i8(raw: torch.Tensor, q: int, M: int, K: int) -> torch.Tensor:
    """uint8 [n?, M, row_bytes] K-quant rows on the GPU -> I8 rows uint8 [n?, M, K / 32 * 48]."""
    out = ops.transcode_i8(q, raw.contiguous().reshape(-1))
    return out.view(*raw.shape[:-2], M, K // 32 * 48)


def _router_fmt(t: torch.Tensor | None, f32: bool) -> torch.Tensor | None:
    """bf16 bits (int16) or fp32 on the device; bf16 input widened exactly when f32."""
    if t is None:
        return None
    if t.dtype in (torch.int16, torch.uint16):
        t = t.view(torch.bfloat16) if t.dtype == torch.int16 else t.view(torch.int16).view(torch.bfloat16)
    if f32:
        return t.to(torch.float32).contiguous()
    if t.dtype != torch.bfloat16:
        raise ValueError(f"router / sh_gate_inp: expected bf16 or fp32, got {t.dtype}")
    return t.contiguous().view(torch.int16)


class GpuMoeBlock:
    """One MoE block resident on the GPU."""

    def __init__(self, *, gate, up, down, router, q_gate: int, q_down: int, D: int, FF: int, E: int, k: int,
                 gate_sh=None, up_sh=None, down_sh=None, q_gate_sh: int | None = None,
                 q_down_sh: int | None = None, sh_gate_inp=None, router_bias=None, norm_w=None,
                 norm_eps: float = 1e-6, device="cuda"):
        L.require_gpu()
        self.D, self.FF, self.E, self.k = int(D), int(FF), int(E), int(k)
        self.q_gate, self.q_down = int(q_gate), int(q_down)
        self.q_gate_sh = int(q_gate_sh if q_gate_sh is not None else q_gate)
        self.q_down_sh = int(q_down_sh if q_down_sh is not None else q_down)
        self.gate = _dev(gate, device=device)
        self.up = _dev(up, device=device)
        self.down = _dev(down, device=device)
        # Router and shared scalar gate: bf16 (bits as int16 / uint16, or torch.bfloat16) or
        # fp32, as the file holds them (the reference reads both in fp32,
        # qwen/forward.py:41-47).  Both go to the device in one format: fp32 when
        # either is fp32 (widening bf16 is exact).
        self.router = _dev(router, device=device)
        self.sh_gate_inp = _dev(sh_gate_inp, device=device)
        f32 = self.router.dtype == torch.float32 or (self.sh_gate_inp is not None
                                                      and self.sh_gate_inp.dtype == torch.float32)
        self.q_router = QT.F32 if f32 else QT.BF16
        self.router = _router_fmt(self.router, f32)
        self.sh_gate_inp = _router_fmt(self.sh_gate_inp, f32)
        self.gate_sh = _dev(gate_sh, device=device)
        self.up_sh = _dev(up_sh, device=device)
        self.down_sh = _dev(down_sh, device=device)
        if self.q_gate_sh == QT.BF16 and self.gate_sh is not None and self.gate_sh.dtype == torch.bfloat16:
            self.gate_sh, self.up_sh = self.gate_sh.view(torch.int16), self.up_sh.view(torch.int16)
        if self.q_down_sh == QT.BF16 and self.down_sh is not None and self.down_sh.dtype == torch.bfloat16:
            self.down_sh = self.down_sh.view(torch.int16)
        # K-quant experts (routed and shared) -> I8 rows on the device
        if self.q_gate in _KQUANTS:
            self.gate = _kquant_to_i8(self.gate, self.q_gate, self.FF, self.D)
            self.up = _kquant_to_i8(self.up, self.q_gate, self.FF, self.D)
            self.q_gate = I8
        if self.q_down in _KQUANTS:
            self.down = _kquant_to_i8(self.down, self.q_down, self.D, self.FF)
            self.q_down = I8
        if self.gate_sh is not None and self.q_gate_sh in _KQUANTS:
            self.gate_sh = _kquant_to_i8(self.gate_sh, self.q_gate_sh, self.FF, self.D)
            self.up_sh = _kquant_to_i8(self.up_sh, self.q_gate_sh, self.FF, self.D)
            self.q_gate_sh = I8
        if self.down_sh is not None and self.q_down_sh in _KQUANTS:
            self.down_sh = _kquant_to_i8(self.down_sh, self.q_down_sh, self.D, self.FF)
            self.q_down_sh = I8
        if self.q_gate == QT.BF16 and self.gate.dtype == torch.bfloat16:
            self.gate, self.up = self.gate.view(torch.int16), self.up.view(torch.int16)
        if self.q_down == QT.BF16 and self.down.dtype == torch.bfloat16:
            self.down = self.down.view(torch.int16)
        self.router_bias = _dev(router_bias, torch.float32, device)
        self.norm_w = _dev(norm_w, torch.float32, device)
        self.norm_eps = float(norm_eps)
        self._check_shapes()
        s = L.GmMoeLayer()
        s.gate_exps, s.up_exps, s.down_exps = L.ptr(self.gate), L.ptr(self.up), L.ptr(self.down)
        s.gate_sh, s.up_sh, s.down_sh = L.ptr(self.gate_sh), L.ptr(self.up_sh), L.ptr(self.down_sh)
        s.router, s.sh_gate_inp = L.ptr(self.router), L.ptr(self.sh_gate_inp)
        s.router_bias, s.norm_w = L.ptr(self.router_bias), L.ptr(self.norm_w)
        s.norm_eps = self.norm_eps
        s.q_gate = s.q_up = self.q_gate
        s.q_down = self.q_down
        s.q_gate_sh = s.q_up_sh = self.q_gate_sh
        s.q_down_sh = self.q_down_sh
        s.D, s.FF, s.FF_sh, s.E, s.k = self.D, self.FF, self.FF if self.gate_sh is not None else 0, self.E, self.k
        s.q_router = int(self.q_router)
        # [D/8][E+1][8]: router and shared gate columns in groups of 8 (gm_moe_chain's
        # down kernels read the next layer's router 8 columns at a time)
        rt = torch.zeros(self.E + 1, self.D, dtype=self.router.dtype, device=self.router.device)
        rt[:self.E] = self.router
        if self.sh_gate_inp is not None:
            rt[self.E] = self.sh_gate_inp
        self.router_t = rt.view(self.E + 1, self.D // 8, 8).permute(1, 0, 2).contiguous()
        s.router_t = L.ptr(self.router_t)
        self.struct = s
        self._ws: torch.Tensor | None = None
        self._retired: list[torch.Tensor] = []

    def _check_shapes(self) -> None:
        D, FF, E = self.D, self.FF, self.E

        def want(q, M, K):                     # raw or I8 rows, or bf16 bits [.., M, K]
            return ((E, M, K), torch.int16) if q == QT.BF16 else ((E, M, _row_bytes(q, K)), torch.uint8)
        for name, (shp, dt) in {"gate": want(self.q_gate, FF, D), "up": want(self.q_gate, FF, D),
                                "down": want(self.q_down, D, FF)}.items():
            t = getattr(self, name)
            if tuple(t.shape) != shp or t.dtype != dt:
                raise ValueError(f"{name}: expected {dt} {shp}, got {t.dtype} {tuple(t.shape)}")
        if tuple(self.router.shape) != (E, D):
            raise ValueError(f"router: expected ({E}, {D}), got {tuple(self.router.shape)}")
        if self.gate_sh is not None:
            rb = (lambda q, K: _row_bytes(q, K) if q != QT.BF16 else 2 * K)
            g_elt = 1 if self.gate_sh.dtype == torch.uint8 else 2
            if self.gate_sh.numel() * g_elt != FF * rb(self.q_gate_sh, D):
                raise ValueError("gate_sh size does not match FF x D")
            d_elt = 1 if self.down_sh.dtype == torch.uint8 else 2
            if self.down_sh.numel() * d_elt != D * rb(self.q_down_sh, FF):
                raise ValueError("down_sh size does not match D x FF")

    @classmethod
    def from_host(cls, h, device="cuda") -> "GpuMoeBlock":
        """Upload a ``synth.HostMoeLayer`` (or anything with the same fields)."""
        return cls(gate=h.gate, up=h.up, down=h.down, router=h.router, q_gate=h.q_gate, q_down=h.q_down,
                   D=h.D, FF=h.FF, E=h.E, k=h.k, gate_sh=h.gate_sh, up_sh=h.up_sh, down_sh=h.down_sh,
                   sh_gate_inp=h.sh_gate_inp, router_bias=h.router_bias, norm_w=h.norm_w, device=device)

    # ------------------------------------------------------------------
    def workspace(self, T: int) -> torch.Tensor:
        """The block's one workspace, grown (never shrunk) to the largest T seen.  Offsets
        inside it are recomputed from T on every call, so every smaller T reuses it.  A
        call with a larger T installs a larger buffer; the smaller ones stay referenced
        (``_retired``) for the block's lifetime, so a graph captured before the growth
        still replays into memory that nothing else has been handed (growth happens at
        most a few times: each step at least doubles the size)."""
        n = ops.moe_workspace_bytes(self.struct, T)
        if self._ws is None or self._ws.numel() < n:
            if self._ws is not None:
                self._retired.append(self._ws)
                n = max(n, 2 * self._ws.numel())
            self._ws = torch.zeros(n, dtype=torch.uint8, device=self.gate.device)
        return self._ws

    def forward(self, x: torch.Tensor, *, residual: bool = False, out: torch.Tensor | None = None,
                stage: int = 0, path: str = "auto") -> torch.Tensor:
        """x fp32 [T, D] on the GPU -> y [T, D] = moe(rmsnorm(x)) (+ x).

        ``stage`` 1..3 runs one decode stage only (router, gate/up, down);
        ``path`` forces the decode kernels or the prefill GEMMs ("auto" picks by T)."""
        if x.dim() != 2 or x.shape[1] != self.D:
            raise ValueError(f"x must be [T, {self.D}], got {tuple(x.shape)}")
        x = x.to(torch.float32).contiguous()
        T = x.shape[0]
        y = out if out is not None else torch.empty_like(x)
        ops.moe_forward_raw(self.struct, x, y, self.workspace(T), residual=residual, stage=stage, path=path)
        return y

    __call__ = forward

    def stages(self, T: int) -> dict[str, torch.Tensor]:
        """Views of the last call's intermediates (router logits, ids, weights, shared gate)."""
        ws = self.workspace(T)
        off = ops.moe_workspace_offsets(self.struct, T)
        E, k = self.E, self.k

        def view(o, n, dt):
            return ws[o:o + n * 4].view(dt)

        return {
            "ffn_moe_logits": view(off["logits"], T * E, torch.float32).view(T, E),
            "topk_ids": view(off["ids"], T * k, torch.int32).view(T, k),
            "ffn_moe_weights_norm": view(off["weights"], T * k, torch.float32).view(T, k),
            "shared_expert_gate_sigmoid": view(off["sh_gate"], T, torch.float32),
        }

    def weight_bytes_per_token(self) -> int:
        per_exp = (self.gate[0].numel() + self.up[0].numel() + self.down[0].numel())
        sh = 0
        if self.gate_sh is not None:
            sh = sum(t.numel() * t.element_size() for t in (self.gate_sh, self.up_sh, self.down_sh))
        g = 0 if self.sh_gate_inp is None else self.sh_gate_inp.numel() * self.sh_gate_inp.element_size()
        return self.k * per_exp + sh + self.router.numel() * self.router.element_size() + g


class GpuMoeChain:
    """Consecutive ``GpuMoeBlock`` layers run by one ``gm_moe_chain`` call: x_{l+1} =
    x_l + moe_l(rmsnorm_l(x_l)) (the MoE step of the decoder loop,
    qwen/forward.py:880-884).  At T = 1 the library links the layers through router
    accumulators (each layer's down kernel computes the next layer's router dot
    products), so the chain costs one router launch plus two launches per layer.  Each
    layer keeps its own workspace, so ``blocks[l].stages(T)`` shows layer l's ids and
    weights after a call."""

    def __init__(self, blocks: list[GpuMoeBlock]):
        if not blocks:
            raise ValueError("GpuMoeChain needs at least one block")
        if len({b.D for b in blocks}) != 1:
            raise ValueError("every block of a chain must have the same D")
        self.blocks = list(blocks)
        self.D = blocks[0].D
        self._buf: torch.Tensor | None = None

    def fused(self, T: int) -> bool:
        """True when a T-token call links consecutive layers: at T = 1 the accumulator-linked
        kernels, at 2 <= T <= 8 each layer's combine kernel forming the next layer's router
        inputs (the blocks' workspaces are distinct); False when it runs one gm_moe_forward
        per layer."""
        return ops.moe_chain_fused([b.struct for b in self.blocks], T)

    def mode(self, T: int) -> int:
        """gm_moe_chain_fused's answer: 1 (T = 1 linked), 2 (T > 1 linked) or 0."""
        return ops.moe_chain_mode([b.struct for b in self.blocks], T)

    def __call__(self, x: torch.Tensor, *, residual: bool = True, out: torch.Tensor | None = None) -> torch.Tensor:
        if x.dim() != 2 or x.shape[1] != self.D:
            raise ValueError(f"x must be [T, {self.D}], got {tuple(x.shape)}")
        x = x.to(torch.float32).contiguous()
        T = x.shape[0]
        y = out if out is not None else torch.empty_like(x)
        if self._buf is None or self._buf.shape != x.shape or self._buf.device != x.device:
            self._buf = torch.empty_like(x)
        ops.moe_chain_raw([b.struct for b in self.blocks], x, y, self._buf,
                          [b.workspace(T) for b in self.blocks], residual=residual)
        return y
