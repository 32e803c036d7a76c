"""Drop-in for the MoE half of the reference's ``qwen/forward.py``.

Same names and call signatures as the reference: ``MoELayer`` (438-491),
``moe_forward(x, layer, cfg)`` (563-665), ``enable_npu(model, ops, *,
expert_cache_limit)`` (723-831) with the same op names and ``layer.npu`` keys,
and ``rms_norm`` (58-61).  The difference is where the block runs: the whole
MoE block (router, top-k, dispatch, expert products, shared expert, combine)
executes on the GPU from raw GGUF expert bytes resident in HBM, with routing
kept on the device (no ``picked.tolist()`` host loop).  There is no CPU path:
``moe_forward`` builds the device block on first use if ``enable_npu`` was not
called.  Prefill (T > 8 tokens) uses the grouped MFMA kernels.

``SyntheticTensorStore`` provides the ``TensorStore`` surface (``get``,
``raw``, ``get_expert``, ``cfg``) over seeded synthetic layers, since the
reference's 16 GB GGUF is not available.
"""
from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass, field
from typing import Sequence

import numpy as np
import torch

from npu_amd import _lib as L
from npu_amd import ops
from npu_amd._dropin import device
from npu_amd.gguf_types import GGMLQuantizationType as QT, QuantTensor, row_bytes
from npu_amd.moe import GpuMoeBlock
from npu_amd.profiler import profile

VALID_OPS = {"router", "shexp", "shexp_split", "attn_o", "attn_qkv", "ssm",
             "experts", "experts_split", "experts_dense", "experts_packed_down"}


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    x_f = x.float()
    rms = x_f.pow(2).mean(-1, keepdim=True).add(eps).rsqrt()
    return ((x_f * rms) * w.float()).to(x.dtype)


@dataclass
class Config:
    """The ``qwen/model.py:Config`` fields the MoE block reads."""

    d_model: int = 2048
    n_expert: int = 256
    n_expert_used: int = 8
    d_expert_ff: int = 512
    rms_eps: float = 1e-6
    n_layer: int = 1


# ------------------------------------------------------------- tensor store
class SyntheticTensorStore:
    """GGUF-TensorStore stand-in over ``synth.HostMoeLayer`` blocks.

    Names follow the GGUF file (``blk.{i}.ffn_gate_exps.weight`` ...); quantised
    tensors come back from ``raw`` as ``QuantTensor`` records with ggml-order
    shapes, dense ones from ``get`` as fp32 numpy arrays in (out, in) order.
    """

    def __init__(self, layers, cfg: Config | None = None):
        self.layers = list(layers)
        h = self.layers[0]
        self.cfg = cfg or Config(d_model=h.D, n_expert=h.E, n_expert_used=h.k, d_expert_ff=h.FF,
                                 n_layer=len(self.layers))
        self._raw: dict[str, QuantTensor] = {}
        self._dense: dict[str, np.ndarray] = {}
        for i, L in enumerate(self.layers):
            p = f"blk.{i}."
            self._raw[p + "ffn_gate_exps.weight"] = QuantTensor(p + "ffn_gate_exps.weight", L.q_gate, (L.D, L.FF, L.E), L.gate)
            self._raw[p + "ffn_up_exps.weight"] = QuantTensor(p + "ffn_up_exps.weight", L.q_gate, (L.D, L.FF, L.E), L.up)
            self._raw[p + "ffn_down_exps.weight"] = QuantTensor(p + "ffn_down_exps.weight", L.q_down, (L.FF, L.D, L.E), L.down)
            if L.gate_sh is not None:
                self._raw[p + "ffn_gate_shexp.weight"] = QuantTensor(p + "ffn_gate_shexp.weight", L.q_gate, (L.D, L.FF), L.gate_sh)
                self._raw[p + "ffn_up_shexp.weight"] = QuantTensor(p + "ffn_up_shexp.weight", L.q_gate, (L.D, L.FF), L.up_sh)
                self._raw[p + "ffn_down_shexp.weight"] = QuantTensor(p + "ffn_down_shexp.weight", L.q_down, (L.FF, L.D), L.down_sh)
            from npu_amd.synth import as_f32
            self._dense[p + "ffn_gate_inp.weight"] = as_f32(L.router).reshape(L.E, L.D)
            if L.sh_gate_inp is not None:
                self._dense[p + "ffn_gate_inp_shexp.weight"] = as_f32(L.sh_gate_inp)
            if L.norm_w is not None:
                self._dense[p + "post_attention_norm.weight"] = L.norm_w
            if L.router_bias is not None:
                self._dense[p + "ffn_gate_inp.bias"] = L.router_bias

    def names(self) -> list[str]:
        return list(self._raw) + list(self._dense)

    def has(self, name: str) -> bool:
        return name in self._raw or name in self._dense

    def raw(self, name: str):
        t = self._raw.get(name)
        if t is None:
            raise KeyError(name)
        return t

    def get(self, name: str, dtype: str = "fp32", keep: bool = True) -> np.ndarray:
        if name in self._dense:
            return self._dense[name]
        t = self.raw(name)
        full = ops.dequant(t.tensor_type, torch.from_numpy(np.ascontiguousarray(t.data).reshape(-1)).to(device()))
        return full.cpu().numpy().reshape(tuple(reversed(t.shape)))

    def get_expert(self, name: str, expert_idx: int, dtype: str = "fp32") -> np.ndarray:
        t = self.raw(name)
        if len(t.shape) != 3:
            raise ValueError(f"{name} is not a stacked expert tensor (got shape {list(t.shape)})")
        if not 0 <= expert_idx < t.shape[2]:
            raise IndexError(expert_idx)
        chunk = np.ascontiguousarray(t.data[expert_idx]).reshape(-1)
        full = ops.dequant(t.tensor_type, torch.from_numpy(chunk).to(device()))
        return full.cpu().numpy().reshape(t.shape[1], t.shape[0])


# ------------------------------------------------------------------ layer
def _w(ts, name: str, dtype=torch.float32) -> torch.Tensor | None:
    if not ts.has(name):
        return None
    return torch.from_numpy(np.array(ts.get(name, dtype="fp32", keep=False), copy=True)).to(dtype)


@dataclass
class MoELayer:
    """Same fields as the reference's ``MoELayer``; ``npu`` holds the device block."""

    i: int
    ts: object = field(repr=False)
    dtype: torch.dtype = torch.float32
    w_router: torch.Tensor | None = None          # [n_expert, D]
    w_gate_sh: torch.Tensor | None = None          # [ff_sh, D] (dense models) or None
    w_up_sh: torch.Tensor | None = None
    w_down_sh: torch.Tensor | None = None          # [D, ff_sh]
    w_gate_inp_sh: torch.Tensor | None = None      # [D]
    npu: dict | None = None

    @classmethod
    def load(cls, ts, i: int, dtype=torch.float32) -> "MoELayer":
        p = f"blk.{i}."

        def dense_or_none(name):
            if not ts.has(name):
                return None
            try:
                raw = ts.raw(name)
            except KeyError:
                raw = None
            if raw is not None and int(raw.tensor_type) in (QT.IQ4_XS, QT.IQ3_XXS):
                return None          # quantised shared expert stays raw (see enable_npu)
            return _w(ts, name, dtype)

        return cls(i=i, ts=ts, dtype=dtype,
                   w_router=_w(ts, p + "ffn_gate_inp.weight", dtype),
                   w_gate_sh=dense_or_none(p + "ffn_gate_shexp.weight"),
                   w_up_sh=dense_or_none(p + "ffn_up_shexp.weight"),
                   w_down_sh=dense_or_none(p + "ffn_down_shexp.weight"),
                   w_gate_inp_sh=_w(ts, p + "ffn_gate_inp_shexp.weight", dtype))

    def dequant_one(self, expert_idx: int):
        """(gate[ff,D], up[ff,D], down[D,ff]) of one expert, dequantised on the GPU."""
        p = f"blk.{self.i}."
        out = []
        for n in ("ffn_gate_exps.weight", "ffn_up_exps.weight", "ffn_down_exps.weight"):
            out.append(torch.from_numpy(self.ts.get_expert(p + n, expert_idx).copy()).to(self.dtype))
        return tuple(out)


_IQ = (int(QT.IQ4_XS), int(QT.IQ3_XXS))
_KQ = (int(QT.Q8_0), int(QT.Q4_K), int(QT.Q5_K), int(QT.Q6_K))


def _shared_raw(ts, names, D: int, FF: int) -> dict | None:
    """The shared expert from the file's raw bytes when its formats run natively: gate and
    up both IQ4_XS / IQ3_XXS of one type (kept raw), or both K-quants (each transcoded to
    I8 rows, so Q6_K gate with Q8_0 up works); down IQ (raw) or a K-quant (I8).  None
    when the tensors are absent or in other types (then the dense fp32 copy is used)."""
    if not all(ts.has(n) for n in names):
        return None
    gs, us, ds = (ts.raw(n) for n in names)
    tg, tu, td = int(gs.tensor_type), int(us.tensor_type), int(ds.tensor_type)

    def dev(t):
        a = np.ascontiguousarray(t.data).reshape(-1)
        return torch.from_numpy(a if a.flags.writeable else a.copy()).to(device())

    def i8(t, q, M, K):
        return ops.transcode_i8(q, dev(t)).view(M, K // 32 * 48)

    if tg == tu and tg in _IQ:
        out = dict(gate_sh=gs.data, up_sh=us.data, q_gate_sh=tg)
    elif tg in _KQ and tu in _KQ:
        out = dict(gate_sh=i8(gs, tg, FF, D), up_sh=i8(us, tu, FF, D), q_gate_sh=L.GM_QTYPE_I8)
    else:
        return None
    if td in _IQ:
        out.update(down_sh=ds.data, q_down_sh=td)
    elif td in _KQ:
        out.update(down_sh=i8(ds, td, D, FF), q_down_sh=L.GM_QTYPE_I8)
    else:
        return None
    return out


def _exact_bf16_or_f32(w: torch.Tensor) -> torch.Tensor:
    """fp32 weights as bf16 when every value is a bf16 value (half the bytes, same
    numbers), else unchanged fp32."""
    w = torch.as_tensor(w).float().contiguous()
    b = w.to(torch.bfloat16)
    return b if torch.equal(b.float(), w) else w


def _build_block(layer: MoELayer) -> GpuMoeBlock:
    ts = layer.ts
    p = f"blk.{layer.i}."
    g, u, d = (ts.raw(p + n) for n in ("ffn_gate_exps.weight", "ffn_up_exps.weight", "ffn_down_exps.weight"))
    if int(g.tensor_type) != int(u.tensor_type):
        raise NotImplementedError("gate and up experts must share a quant type")
    D, FF, E = int(g.shape[0]), int(g.shape[1]), int(g.shape[2])
    cfg = getattr(ts, "cfg", None)
    k = int(getattr(cfg, "n_expert_used", 8))
    # The router and the shared gate keep the fp32 values the reference computes with
    # (qwen/forward.py:41-47, 599, 608); they are stored as bf16 only when that is exact.
    router = _exact_bf16_or_f32(layer.w_router)
    kw = {}
    sh_names = tuple(p + n for n in ("ffn_gate_shexp.weight", "ffn_up_shexp.weight", "ffn_down_shexp.weight"))
    sh_raw = _shared_raw(ts, sh_names, D, FF)
    if sh_raw is not None:                       # the file's shared expert bytes: IQ kept raw, K-quants as I8
        kw.update(sh_raw)
    elif layer.w_gate_sh is not None:            # a dense shared expert without raw bytes: bf16
        kw.update(gate_sh=layer.w_gate_sh.to(torch.bfloat16), up_sh=layer.w_up_sh.to(torch.bfloat16),
                  down_sh=layer.w_down_sh.to(torch.bfloat16), q_gate_sh=QT.BF16, q_down_sh=QT.BF16)
    sh_inp = None
    if layer.w_gate_inp_sh is not None:
        sh_inp = _exact_bf16_or_f32(layer.w_gate_inp_sh)
    bias = torch.from_numpy(ts.get(p + "ffn_gate_inp.bias")) if ts.has(p + "ffn_gate_inp.bias") else None
    return GpuMoeBlock(gate=g.data, up=u.data, down=d.data, router=router, q_gate=int(g.tensor_type),
                       q_down=int(d.tensor_type), D=D, FF=FF, E=E, k=k, sh_gate_inp=sh_inp, router_bias=bias,
                       device=device(), **kw)


def _expert_cache_limit_from_env(default: int) -> int | None:
    import os
    raw = os.environ.get("QWEN_NPU_EXPERT_CACHE_LIMIT")
    if raw is None or raw == "":
        return default
    val = raw.strip().lower()
    if val in {"none", "unlimited", "inf", "-1"}:
        return None
    limit = int(val)
    return None if limit < 0 else limit


def _is_attn(core) -> bool:
    """An attention core (the reference's ``AttnLayer``, qwen/forward.py:100-130): wq/wk/wv/wo."""
    return core is not None and all(hasattr(core, n) for n in ("wq", "wk", "wv", "wo"))


def _is_ssm(core) -> bool:
    """A Gated DeltaNet core (the reference's ``SSMLayer``, :245-285): w_in/w_gate/w_out."""
    return core is not None and all(hasattr(core, n) for n in ("w_in", "w_gate", "w_out"))


def _pairs(model):
    """(core, moe) per layer: ``model.layers`` holds the pairs (reference :775); a plain
    sequence of MoE layers has no cores."""
    if hasattr(model, "layers"):
        for item in model.layers:
            if isinstance(item, tuple):
                yield item
            else:
                yield None, item
    else:
        for moe in model:
            yield None, moe


def enable_npu(model, ops: Sequence[str] = ("router",), *, expert_cache_limit: int | None = None) -> None:
    """Attach device operators to every layer of ``model`` (reference :723-831, same op names
    and ``npu`` keys).

    For each ``(core, moe)`` pair of ``model.layers``: every expert-family op makes the MoE
    layer run through the fused device block; ``router`` / ``shexp`` / ``shexp_split``
    additionally expose the stand-alone operators under the reference's ``layer.npu`` keys.
    The expert cache limit is kept for compatibility: all experts are resident in HBM, so
    nothing is evicted.  On the cores: ``attn_o`` puts ``NpuMatVec(core.wo)`` under
    ``core.npu["wo"]``, ``attn_qkv`` ``NpuConcatMatVec((wq, wk, wv))`` under ``"wqkv"``
    (attention cores), and ``ssm`` ``NpuMatVec`` of ``w_in`` / ``w_gate`` / ``w_out`` under
    the same names (Gated DeltaNet cores), as :813-831 do.
    """
    from npu_amd.mlp import NpuFusedMLP
    from npu_amd.mv import NpuConcatMatVec, NpuMatVec

    unknown = set(ops) - VALID_OPS
    if unknown:
        raise ValueError(f"unknown NPU ops: {sorted(unknown)} (valid: {sorted(VALID_OPS)})")
    for core, moe in _pairs(model):
        if moe.npu is None:
            moe.npu = {}
        if "router" in ops:
            moe.npu["router"] = NpuMatVec(moe.w_router)
        if "shexp" in ops and moe.w_gate_sh is not None:
            moe.npu["sh_mlp"] = NpuFusedMLP(moe.w_gate_sh, moe.w_down_sh, w_up=moe.w_up_sh)
        if "shexp_split" in ops and moe.w_gate_sh is not None:
            moe.npu["sh_gate"] = NpuMatVec(moe.w_gate_sh)
            moe.npu["sh_up"] = NpuMatVec(moe.w_up_sh)
            moe.npu["sh_down"] = NpuMatVec(moe.w_down_sh)
        if {"experts", "experts_split", "experts_dense", "experts_packed_down"} & set(ops):
            p = f"blk.{moe.i}."
            moe.npu["expert_tensors"] = tuple(moe.ts.raw(p + n) for n in (
                "ffn_gate_exps.weight", "ffn_up_exps.weight", "ffn_down_exps.weight"))
            moe.npu["expert_cache"] = OrderedDict()
            moe.npu["expert_dense"] = "experts_dense" in ops
            moe.npu["expert_fused"] = "experts" in ops
            moe.npu["expert_packed_down"] = "experts_packed_down" in ops
            moe.npu["expert_cache_limit"] = (_expert_cache_limit_from_env(8) if expert_cache_limit is None
                                             else (None if expert_cache_limit < 0 else expert_cache_limit))
        moe.npu["moe_block"] = _build_block(moe)
        if "attn_o" in ops and _is_attn(core):
            if core.npu is None:
                core.npu = {}
            core.npu["wo"] = NpuMatVec(core.wo)
        if "attn_qkv" in ops and _is_attn(core):
            if core.npu is None:
                core.npu = {}
            core.npu["wqkv"] = NpuConcatMatVec((core.wq, core.wk, core.wv), profile_prefix="attn_qkv_mv")
        if "ssm" in ops and _is_ssm(core):
            if core.npu is None:
                core.npu = {}
            core.npu["w_in"] = NpuMatVec(core.w_in)
            core.npu["w_gate"] = NpuMatVec(core.w_gate)
            core.npu["w_out"] = NpuMatVec(core.w_out)


def moe_forward(x: torch.Tensor, layer: MoELayer, cfg) -> torch.Tensor:
    """x [B, T, D] -> [B, T, D]: the whole MoE block on the GPU (reference :563-665)."""
    B, T, D = x.shape
    if layer.npu is None:
        layer.npu = {}
    blk = layer.npu.get("moe_block")
    if blk is None:
        blk = layer.npu["moe_block"] = _build_block(layer)
    on_host = not x.is_cuda
    with profile("moe.block"):
        xf = x.reshape(B * T, D).to(device() if on_host else x.device, torch.float32).contiguous()
        y = blk(xf)
    if on_host:
        y = y.cpu()
    return y.to(x.dtype).view(B, T, D)
