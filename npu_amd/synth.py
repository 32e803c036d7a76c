"""Seeded synthetic inputs with the distributions BASELINE.json's configs state.

* IQ4_XS superblock (136 B): fp16 d = |N(0,1)| * 2e-3, then uniform random
  scales_h (u16), scales_l (4 x u8) and qs (128 x u8).
* IQ3_XXS superblock (98 B): fp16 d = |N(0,1)| * 2e-3, then 64 uniform qs bytes
  and 8 uniform u32 sign/scale words (four 7-bit ksigns indices + a 4-bit
  scale each, uniform == a uniform u32).
* Router: bf16(N(0, 0.02)) [E, D]; shared-expert scalar gate bf16(N(0, 0.02)) [D].
* Activations: fp32 N(0, 1), RMSNorm'd (eps 1e-6, weight 1) where the config says so.
* Prefill skew: per-expert router-logit bias ~ N(0, 1).

Two generators produce these: ``host_*`` (numpy PCG64, used by the tests and
small configs, bytes reproducible anywhere) and ``device_*`` (torch's seeded
GPU generator, for the ~16 GB 40-layer decode config where host generation
would take minutes).  Both follow the same distributions; their bytes differ.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from npu_amd.gguf_types import QK, GGMLQuantizationType as QT, block_bytes, row_bytes

D_SCALE = 2e-3
ROUTER_STD = 0.02


def to_bf16(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits (uint16), round to nearest even (as qwen/model.py:280-289).
    A NaN stays a NaN (its top mantissa bit is set, as torch's bf16 cast does); the
    rounding add alone would carry a NaN with a small payload into +-inf."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def from_bf16(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def as_f32(a: np.ndarray) -> np.ndarray:
    """A router / shared-gate array held as bf16 bits (uint16) or fp32, as fp32."""
    return np.ascontiguousarray(a) if np.asarray(a).dtype == np.float32 else from_bf16(a)


def _gen(seed: int, *stream: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(np.random.SeedSequence([int(seed), *map(int, stream)])))


# ------------------------------------------------------------------ host
def host_superblocks(g: np.random.Generator, qtype: int, n_sb: int) -> np.ndarray:
    """uint8 [n_sb, block_bytes] raw superblocks."""
    bb = block_bytes(qtype)
    if qtype not in (QT.IQ4_XS, QT.IQ3_XXS):
        raise ValueError(f"not a superblock format: {qtype}")
    out = np.empty((n_sb, bb), dtype=np.uint8)
    d = (np.abs(g.standard_normal(n_sb)) * D_SCALE).astype(np.float16)
    out[:, 0:2] = d.view(np.uint8).reshape(n_sb, 2)
    out[:, 2:] = g.integers(0, 256, size=(n_sb, bb - 2), dtype=np.uint8)
    return out


# Byte offsets of the fp16 scale fields of the K-quant blocks (d, and dmin where
# the format has one), and each block's (weights, bytes).
_KQ_FIELDS = {QT.Q8_0: (0,), QT.Q4_K: (0, 2), QT.Q5_K: (0, 2), QT.Q6_K: (208,)}
_KQ_BLOCK = {QT.Q8_0: (32, 34), QT.Q4_K: (256, 144), QT.Q5_K: (256, 176), QT.Q6_K: (256, 210)}


def host_kquant_blocks(g: np.random.Generator, qtype: int, n_blocks: int) -> np.ndarray:
    """uint8 [n_blocks, bytes] of a K-quant type: uniform random quants / scales, fp16 d
    (and dmin) = |N(0,1)| * 2e-3 (the IQ superblocks' distribution of d)."""
    nb = _KQ_BLOCK[int(qtype)][1]
    out = g.integers(0, 256, size=(n_blocks, nb), dtype=np.uint8)
    for off in _KQ_FIELDS[int(qtype)]:
        v = (np.abs(g.standard_normal(n_blocks)) * D_SCALE).astype(np.float16)
        out[:, off:off + 2] = v.view(np.uint8).reshape(n_blocks, 2)
    return out


def host_quant_matrix(g: np.random.Generator, qtype: int, M: int, K: int, n_expert: int | None = None) -> np.ndarray:
    """Raw weight bytes [n_expert?, M, row_bytes] for an [M x K] matrix (per expert)."""
    E = 1 if n_expert is None else n_expert
    if int(qtype) in _KQ_BLOCK:
        w = _KQ_BLOCK[int(qtype)][0]
        sb = host_kquant_blocks(g, qtype, E * M * (K // w))
        shape = (M, row_bytes(qtype, K)) if n_expert is None else (E, M, row_bytes(qtype, K))
        return sb.reshape(shape)
    sb = host_superblocks(g, qtype, E * M * (K // QK))
    shape = (M, row_bytes(qtype, K)) if n_expert is None else (E, M, row_bytes(qtype, K))
    return sb.reshape(shape)


def host_bf16_normal(g: np.random.Generator, shape, std: float) -> np.ndarray:
    return to_bf16((g.standard_normal(shape) * std).astype(np.float32))


def rms_norm_np(x: np.ndarray, eps: float = 1e-6, w: np.ndarray | None = None) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    rms = (1.0 / np.sqrt((x.astype(np.float32) ** 2).mean(-1, keepdims=True) + np.float32(eps))).astype(np.float32)
    y = (x * rms).astype(np.float32)
    return y if w is None else (y * w).astype(np.float32)


def host_input(seed: int, T: int, D: int, rmsnorm: bool = True) -> np.ndarray:
    x = _gen(seed, 99).standard_normal((T, D)).astype(np.float32)
    return rms_norm_np(x) if rmsnorm else x


@dataclass
class HostMoeLayer:
    """One MoE block's weights as raw host arrays (GGUF layout)."""

    D: int
    FF: int
    E: int
    k: int
    q_gate: int
    q_down: int
    gate: np.ndarray          # uint8 [E, FF, row_bytes(q_gate, D)]
    up: np.ndarray            # uint8 [E, FF, row_bytes(q_gate, D)]
    down: np.ndarray          # uint8 [E, D, row_bytes(q_down, FF)]
    router: np.ndarray        # [E, D] bf16 bits (uint16) or float32
    gate_sh: np.ndarray | None = None   # uint8 [FF, row_bytes(q_gate, D)]
    up_sh: np.ndarray | None = None
    down_sh: np.ndarray | None = None   # uint8 [D, row_bytes(q_down, FF)]
    sh_gate_inp: np.ndarray | None = None  # [D] bf16 bits (uint16) or float32
    router_bias: np.ndarray | None = None  # float32 [E]
    norm_w: np.ndarray | None = None       # float32 [D]
    meta: dict = field(default_factory=dict)

    @property
    def q_up(self) -> int:
        return self.q_gate

    def weight_bytes_per_token(self) -> int:
        """Raw bytes one T=1 decode reads: k experts + shared + router + shared gate."""
        per_exp = self.gate[0].nbytes + self.up[0].nbytes + self.down[0].nbytes
        sh = 0 if self.gate_sh is None else self.gate_sh.nbytes + self.up_sh.nbytes + self.down_sh.nbytes
        g = 0 if self.sh_gate_inp is None else self.sh_gate_inp.nbytes
        return self.k * per_exp + sh + self.router.nbytes + g


def host_moe_layer(seed: int, *, D: int = 2048, FF: int = 512, E: int = 256, k: int = 8,
                   q_gate: int = QT.IQ4_XS, q_down: int = QT.IQ3_XXS, shared: bool = True,
                   bias: bool = False, norm: bool = False, router_f32: bool = False) -> HostMoeLayer:
    """Config-3/4 style MoE block (defaults: BASELINE's IQ4_XS gate/up, IQ3_XXS down, bf16
    router and shared gate).  ``router_f32``: router and shared gate N(0, 0.02) in fp32, as
    a GGUF file's F32 ``ffn_gate_inp`` holds them (values that bf16 cannot represent)."""
    def small(gen, shape):
        if router_f32:
            return (gen.standard_normal(shape) * ROUTER_STD).astype(np.float32)
        return host_bf16_normal(gen, shape, ROUTER_STD)
    L = HostMoeLayer(
        D=D, FF=FF, E=E, k=k, q_gate=int(q_gate), q_down=int(q_down),
        gate=host_quant_matrix(_gen(seed, 1), q_gate, FF, D, E),
        up=host_quant_matrix(_gen(seed, 2), q_gate, FF, D, E),
        down=host_quant_matrix(_gen(seed, 3), q_down, D, FF, E),
        router=small(_gen(seed, 4), (E, D)),
    )
    if shared:
        L.gate_sh = host_quant_matrix(_gen(seed, 5), q_gate, FF, D)
        L.up_sh = host_quant_matrix(_gen(seed, 6), q_gate, FF, D)
        L.down_sh = host_quant_matrix(_gen(seed, 7), q_down, D, FF)
        L.sh_gate_inp = small(_gen(seed, 8), (D,))
    if bias:
        L.router_bias = _gen(seed, 9).standard_normal(E).astype(np.float32)
    if norm:
        L.norm_w = (1.0 + 0.1 * _gen(seed, 10).standard_normal(D)).astype(np.float32)
    return L


# ---------------------------------------------------------------- device
def _dev_superblocks(gen: torch.Generator, qtype: int, n_sb: int, device) -> torch.Tensor:
    bb = block_bytes(qtype)
    out = torch.randint(0, 256, (n_sb, bb), dtype=torch.uint8, device=device, generator=gen)
    d = (torch.randn(n_sb, device=device, generator=gen).abs() * D_SCALE).to(torch.float16)
    out[:, 0:2] = d.view(torch.uint8).reshape(n_sb, 2)
    return out


def device_quant_matrix(gen: torch.Generator, qtype: int, M: int, K: int, n_expert: int | None = None,
                        device="cuda") -> torch.Tensor:
    E = 1 if n_expert is None else n_expert
    sb = _dev_superblocks(gen, qtype, E * M * (K // QK), device)
    shape = (M, row_bytes(qtype, K)) if n_expert is None else (E, M, row_bytes(qtype, K))
    return sb.reshape(shape)


def device_bf16_normal(gen: torch.Generator, shape, std: float, device="cuda") -> torch.Tensor:
    return (torch.randn(shape, device=device, generator=gen) * std).to(torch.bfloat16)


CONFIG5 = dict(D=2048, FF=512, E=256, k=8)


def device_config5_layers(n_layers: int, device, seed: int):
    """``n_layers`` BASELINE config-5 blocks generated on the device: IQ4_XS gate/up and
    IQ3_XXS down experts (E=256, D=2048, FF=512), a shared expert in the same formats,
    bf16 router and shared gate N(0, 0.02), RMSNorm weight 1, eps 1e-6."""
    from npu_amd.moe import GpuMoeBlock
    D, FF, E, k = CONFIG5["D"], CONFIG5["FF"], CONFIG5["E"], CONFIG5["k"]
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    layers = []
    for _ in range(n_layers):
        gate = device_quant_matrix(gen, QT.IQ4_XS, FF, D, E, device)
        up = device_quant_matrix(gen, QT.IQ4_XS, FF, D, E, device)
        down = device_quant_matrix(gen, QT.IQ3_XXS, D, FF, E, device)
        router = device_bf16_normal(gen, (E, D), ROUTER_STD, device)
        gate_sh = device_quant_matrix(gen, QT.IQ4_XS, FF, D, None, device)
        up_sh = device_quant_matrix(gen, QT.IQ4_XS, FF, D, None, device)
        down_sh = device_quant_matrix(gen, QT.IQ3_XXS, D, FF, None, device)
        sh_inp = device_bf16_normal(gen, (D,), ROUTER_STD, device)
        norm_w = torch.ones(D, dtype=torch.float32, device=device)
        layers.append(GpuMoeBlock(gate=gate, up=up, down=down, router=router, q_gate=QT.IQ4_XS,
                                  q_down=QT.IQ3_XXS, D=D, FF=FF, E=E, k=k, gate_sh=gate_sh, up_sh=up_sh,
                                  down_sh=down_sh, sh_gate_inp=sh_inp, norm_w=norm_w, norm_eps=1e-6,
                                  device=device))
    return layers


class _DeviceStack:
    """Expert e of a device-resident [E, M, row_bytes] stack, copied to the host on access."""

    def __init__(self, t: torch.Tensor):
        self.t = t

    def __getitem__(self, e: int) -> np.ndarray:
        return self.t[e].cpu().numpy()


def host_view(blk) -> HostMoeLayer:
    """A ``HostMoeLayer`` over a ``GpuMoeBlock``'s weights that copies only what is read: the
    router, shared expert and norm weight up front, one expert's rows on each ``gate[e]`` /
    ``up[e]`` / ``down[e]`` (a 40-layer config-5 chain is 15.6 GB; a routed token reads 8
    experts per layer).  IQ4_XS / IQ3_XXS routed and shared formats only."""
    def host(t):
        return None if t is None else t.cpu().numpy()

    def small(t):
        if t is None:
            return None
        a = t.cpu()
        return a.numpy() if a.dtype == torch.float32 else a.view(torch.int16).numpy().view(np.uint16)

    for q in (blk.q_gate, blk.q_down, blk.q_gate_sh, blk.q_down_sh):
        if q not in (QT.IQ4_XS, QT.IQ3_XXS):
            raise ValueError("host_view serves IQ4_XS / IQ3_XXS blocks")
    return HostMoeLayer(D=blk.D, FF=blk.FF, E=blk.E, k=blk.k, q_gate=blk.q_gate, q_down=blk.q_down,
                        gate=_DeviceStack(blk.gate), up=_DeviceStack(blk.up), down=_DeviceStack(blk.down),
                        router=small(blk.router), gate_sh=host(blk.gate_sh), up_sh=host(blk.up_sh),
                        down_sh=host(blk.down_sh), sh_gate_inp=small(blk.sh_gate_inp),
                        router_bias=host(blk.router_bias), norm_w=host(blk.norm_w))


# ------------------------------------------------------------------ files
def write_gguf_model(path, layers, *, arch: str = "qwen3next", rms_eps: float = 1e-6) -> None:
    """A GGUF file holding the MoE tensors of `layers` (``HostMoeLayer``) under the model's
    tensor names (``blk.{i}.ffn_gate_exps.weight`` ...) and the metadata ``build_config``
    reads: raw expert / shared-expert superblocks, the router and shared gate as F32 (the
    bf16 values widened), the norm weight and router bias as F32."""
    from npu_amd.gguf_file import write_gguf
    h = layers[0]
    kv = {"general.architecture": arch, f"{arch}.block_count": len(layers), f"{arch}.embedding_length": h.D,
          f"{arch}.expert_count": h.E, f"{arch}.expert_used_count": h.k,
          f"{arch}.expert_feed_forward_length": h.FF, f"{arch}.attention.layer_norm_rms_epsilon": rms_eps}
    tensors = []
    for i, L in enumerate(layers):
        p = f"blk.{i}."
        tensors += [(p + "ffn_gate_exps.weight", L.q_gate, (L.D, L.FF, L.E), L.gate),
                    (p + "ffn_up_exps.weight", L.q_gate, (L.D, L.FF, L.E), L.up),
                    (p + "ffn_down_exps.weight", L.q_down, (L.FF, L.D, L.E), L.down),
                    (p + "ffn_gate_inp.weight", int(QT.F32), (L.D, L.E), as_f32(L.router).reshape(L.E, L.D))]
        if L.gate_sh is not None:
            tensors += [(p + "ffn_gate_shexp.weight", L.q_gate, (L.D, L.FF), L.gate_sh),
                        (p + "ffn_up_shexp.weight", L.q_gate, (L.D, L.FF), L.up_sh),
                        (p + "ffn_down_shexp.weight", L.q_down, (L.FF, L.D), L.down_sh),
                        (p + "ffn_gate_inp_shexp.weight", int(QT.F32), (L.D,), as_f32(L.sh_gate_inp))]
        if L.router_bias is not None:
            tensors.append((p + "ffn_gate_inp.bias", int(QT.F32), (L.E,), L.router_bias))
        if L.norm_w is not None:
            tensors.append((p + "post_attention_norm.weight", int(QT.F32), (L.D,), L.norm_w))
    write_gguf(path, kv, [(n, int(t), d, a) for n, t, d, a in tensors])
