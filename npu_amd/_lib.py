"""ctypes binding of ``libnpu_amd.so`` (the C ABI declared in ``include/npu_amd.h``).

Tensors handed to these wrappers must already live on the GPU; the wrappers
pass raw device pointers and torch's current HIP stream, and never
synchronise.  There is no CPU fallback: if the library is missing or no GPU is
present the calls raise.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

# NPU_AMD_LIB=timeline selects the timestamped profiling build (libnpu_amd_tl.so),
# NPU_AMD_LIB=asan the host-only AddressSanitizer build (libnpu_amd_asan.so; CPU tests).
LIB_PATH = Path(__file__).resolve().with_name(
    {"timeline": "libnpu_amd_tl.so", "asan": "libnpu_amd_asan.so"}.get(os.environ.get("NPU_AMD_LIB", ""),
                                                                      "libnpu_amd.so"))

GM_QTYPE_F32 = 0
GM_QTYPE_F16 = 1
GM_QTYPE_IQ3_XXS = 18
GM_QTYPE_IQ4_XS = 23
GM_QTYPE_BF16 = 30
GM_QTYPE_I8 = 100        # transcoded K-quant rows (gm_transcode_i8)

GM_OK = 0
GM_EINVAL = -1
GM_EUNSUPPORTED = -2
GM_EWORKSPACE = -3

GM_MOE_RESIDUAL = 1
GM_NOALLOC_SCRATCH_BYTES = 16 << 20   # gm_moe_forward_noalloc's static scratch per GPU

_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t
_f32 = ctypes.c_float


class GmMoeLayer(ctypes.Structure):
    """Mirror of ``gm_moe_layer`` (include/npu_amd.h)."""

    _fields_ = [
        ("gate_exps", _vp), ("up_exps", _vp), ("down_exps", _vp),
        ("gate_sh", _vp), ("up_sh", _vp), ("down_sh", _vp),
        ("router", _vp), ("sh_gate_inp", _vp), ("router_bias", _vp), ("norm_w", _vp),
        ("norm_eps", _f32),
        ("q_gate", _i32), ("q_up", _i32), ("q_down", _i32),
        ("q_gate_sh", _i32), ("q_up_sh", _i32), ("q_down_sh", _i32),
        ("D", _i32), ("FF", _i32), ("FF_sh", _i32), ("E", _i32), ("k", _i32),
        ("q_router", _i32),
        ("router_t", _vp),
    ]


class GmAttnLayer(ctypes.Structure):
    """Mirror of ``gm_attn_layer`` (include/npu_amd.h)."""

    _fields_ = [
        ("wqkv", _vp), ("wo", _vp), ("attn_norm", _vp), ("q_norm", _vp), ("k_norm", _vp),
        ("eps", _f32),
        ("D", _i32), ("n_head", _i32), ("n_head_kv", _i32), ("head_dim", _i32), ("rope_dim", _i32),
    ]


class GmSsmLayer(ctypes.Structure):
    """Mirror of ``gm_ssm_layer`` (include/npu_amd.h)."""

    _fields_ = [
        ("w_in", _vp), ("w_gate", _vp), ("w_out", _vp), ("alpha", _vp), ("beta", _vp), ("conv1d", _vp),
        ("a", _vp), ("dt_bias", _vp), ("ssm_norm", _vp), ("attn_norm", _vp),
        ("eps", _f32),
        ("D", _i32), ("n_k_heads", _i32), ("n_v_heads", _i32), ("d_state", _i32), ("conv_k", _i32),
    ]


# name -> (restype, argtypes); every symbol include/npu_amd.h declares.
SIGNATURES = {
    "gm_last_error": (ctypes.c_char_p, []),
    "gm_abi_version": (_i32, []),
    "gm_dequant_f32": (_i32, [_i32, _vp, _i64, _vp, _vp]),
    "gm_transcode_i8": (_i32, [_i32, _vp, _i64, _vp, _vp]),
    "gm_matvec": (_i32, [_i32, _vp, _i32, _i32, _vp, _i32, _vp, _vp]),
    "gm_swiglu_mlp": (_i32, [_i32, _vp, _vp, _i32, _vp, _i32, _i32, _vp, _i32, _vp, _vp, _vp]),
    "gm_router_topk": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _f32, _vp, _vp, _vp, _vp, _vp]),
    "gm_moe_dispatch": (_i32, [_vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp]),
    "gm_moe_workspace_bytes": (_sz, [ctypes.POINTER(GmMoeLayer), _i32]),
    "gm_moe_workspace_offsets": (_i32, [ctypes.POINTER(GmMoeLayer), _i32, ctypes.POINTER(_sz),
                                        ctypes.POINTER(_sz), ctypes.POINTER(_sz), ctypes.POINTER(_sz)]),
    "gm_moe_forward": (_i32, [ctypes.POINTER(GmMoeLayer), _vp, _vp, _i32, _i32, _vp, _sz, _vp]),
    "gm_moe_forward_stage": (_i32, [ctypes.POINTER(GmMoeLayer), _vp, _vp, _i32, _i32, _vp, _sz, _i32, _vp]),
    "gm_moe_forward_noalloc": (_i32, [ctypes.POINTER(GmMoeLayer), _vp, _vp, _i32, _i32, _vp]),
    "gm_moe_decode": (_i32, [ctypes.POINTER(GmMoeLayer), _vp, _vp, _i32, _i32, _vp, _sz, _vp]),
    "gm_moe_prefill": (_i32, [ctypes.POINTER(GmMoeLayer), _vp, _vp, _i32, _i32, _vp, _sz, _vp]),
    "gm_moe_chain": (_i32, [ctypes.POINTER(GmMoeLayer), _i32, _vp, _vp, _vp, _i32, _i32,
                            ctypes.POINTER(_vp), ctypes.POINTER(_sz), _vp]),
    "gm_moe_chain_fused": (_i32, [ctypes.POINTER(GmMoeLayer), _i32, _i32]),
    "gm_attn_workspace_bytes": (_sz, [ctypes.POINTER(GmAttnLayer), _i32]),
    "gm_attn_decode": (_i32, [ctypes.POINTER(GmAttnLayer), _vp, _vp, _vp, _vp, _i32, _i32, _vp, _vp, _i32, _vp,
                              _sz, _vp]),
    "gm_attn_decode_moe": (_i32, [ctypes.POINTER(GmAttnLayer), _vp, _vp, _vp, _vp, _i32, _i32, _vp, _vp, _i32,
                                  _vp, _sz, ctypes.POINTER(GmMoeLayer), _vp, _sz, _vp]),
    "gm_ssm_workspace_bytes": (_sz, [ctypes.POINTER(GmSsmLayer)]),
    "gm_ssm_decode": (_i32, [ctypes.POINTER(GmSsmLayer), _vp, _vp, _vp, _vp, _i32, _vp, _sz, _vp]),
    "gm_ssm_decode_moe": (_i32, [ctypes.POINTER(GmSsmLayer), _vp, _vp, _vp, _vp, _i32, _vp, _sz,
                                 ctypes.POINTER(GmMoeLayer), _vp, _sz, _vp]),
    "gm_moe_forward_acc": (_i32, [ctypes.POINTER(GmMoeLayer), _vp, _vp, _i32, _vp, _sz, _vp]),
    "gm_rms_norm": (_i32, [_vp, _vp, _i32, _i32, _f32, _vp, _vp]),
}

_LIB: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """Load the library once; raise if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m npu_amd.build`")
        h = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        if h.gm_abi_version() != 6:
            raise RuntimeError("libnpu_amd.so ABI version mismatch; rebuild it")
        _LIB = h
    return _LIB


def last_error() -> str:
    return (lib().gm_last_error() or b"").decode(errors="replace")


def check(rc: int, fn: str) -> None:
    if rc == GM_OK:
        return
    msg = f"{fn}: {last_error()} (status {rc})"
    if rc in (GM_EINVAL, GM_EWORKSPACE):
        raise ValueError(msg)
    if rc == GM_EUNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


def stream_ptr() -> int:
    return torch.cuda.current_stream().cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("tensor must be on the GPU")
    if not t.is_contiguous():
        raise ValueError("tensor must be contiguous")
    return t.data_ptr()


def require_gpu() -> None:
    if not torch.cuda.is_available():
        raise RuntimeError("npu_amd needs a HIP GPU (gfx950); none is available")
    lib()
