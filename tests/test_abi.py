"""The C-ABI library loads and exports every entry point include/npu_amd.h declares.

Runs without a GPU: only host-side paths (argument validation, workspace
sizing) are exercised, never a kernel launch.
"""
import ctypes
import re
from pathlib import Path

import pytest

from npu_amd import _lib as L

ROOT = Path(__file__).resolve().parents[1]
HEADER = (ROOT / "include" / "npu_amd.h").read_text()


def declared_functions():
    body = re.sub(r"/\*.*?\*/", "", HEADER, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w]+\*?\s+\*?(gm_\w+)\s*\(", body, flags=re.M)))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    assert {"gm_dequant_f32", "gm_matvec", "gm_moe_forward", "gm_router_topk", "gm_moe_dispatch"} <= set(names)


def test_library_exports_every_declared_symbol():
    lib = L.lib()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in include/npu_amd.h but not exported"
        assert name in L.SIGNATURES, f"{name} has no ctypes signature in npu_amd._lib"


@pytest.mark.parametrize("cname,mirror", [("gm_moe_layer", "GmMoeLayer"), ("gm_attn_layer", "GmAttnLayer"),
                                          ("gm_ssm_layer", "GmSsmLayer")])
def test_struct_layout_matches_header(cname, mirror):
    fields = re.search(r"typedef struct %s \{(.*?)\} %s;" % (cname, cname), HEADER, re.S).group(1)
    fields = re.sub(r"/\*.*?\*/", "", fields, flags=re.S)
    names =re.findall(r"(\w+)(?:\s*,\s*(\w+))?(?:\s*,\s*(\w+))?(?:\s*,\s*(\w+))?(?:\s*,\s*(\w+))?;", fields)
    flat = [n for grp in names for n in grp if n]
    assert flat == [f for f, _ in getattr(L, mirror)._fields_]


def test_argument_errors_without_gpu():
    lib = L.lib()
    rc = lib.gm_matvec(L.GM_QTYPE_IQ4_XS, None, 512, 500, None, 1, None, None)
    assert rc == L.GM_EINVAL and "multiple of 256" in L.last_error()
    rc = lib.gm_dequant_f32(7, None, 1, None, None)
    assert rc == L.GM_EINVAL and "qtype" in L.last_error()
    assert lib.gm_dequant_f32(L.GM_QTYPE_IQ3_XXS, None, 0, None, None) == L.GM_OK
    with pytest.raises(ValueError):
        L.check(L.GM_EINVAL, "x")


def _layer(**kw):
    s = L.GmMoeLayer()
    s.gate_exps = s.up_exps = s.down_exps = s.router = 256
    s.q_gate = s.q_up = L.GM_QTYPE_IQ4_XS
    s.q_down = L.GM_QTYPE_IQ3_XXS
    s.D, s.FF, s.FF_sh, s.E, s.k = 2048, 512, 0, 256, 8
    for k, v in kw.items():
        setattr(s, k, v)
    return s


def test_workspace_sizing_and_layer_validation():
    lib = L.lib()
    s = _layer()
    n1 = lib.gm_moe_workspace_bytes(ctypes.byref(s), 1)
    n8 = lib.gm_moe_workspace_bytes(ctypes.byref(s), 8)
    assert 0 < n1 < n8
    assert n1 % 256 == 0
    bad = _layer(k=9)
    assert lib.gm_moe_workspace_bytes(ctypes.byref(bad), 1) == 0
    bad = _layer(q_up=L.GM_QTYPE_IQ3_XXS)
    assert lib.gm_moe_workspace_bytes(ctypes.byref(bad), 1) == 0
    rc = lib.gm_moe_forward(ctypes.byref(s), 1024, 1024, 1, 0, 4096, 16, None)
    assert rc == L.GM_EINVAL and "alias" in L.last_error()
    rc = lib.gm_moe_forward(ctypes.byref(s), 1024, 2048, 1, 0, 4096, 16, None)
    assert rc == L.GM_EWORKSPACE and "workspace" in L.last_error()
    # the kernels read x, norm_w and the weights with 16-byte loads
    rc = lib.gm_moe_forward(ctypes.byref(s), 1028, 2048, 1, 0, 4096, 1 << 30, None)
    assert rc == L.GM_EINVAL and "x and y must be 16-byte aligned" in L.last_error()
    rc = lib.gm_swiglu_mlp(L.GM_QTYPE_IQ4_XS, 256, 256, L.GM_QTYPE_BF16, 264, 2048, 512, 1024, 1, 2048, 4096, None)
    assert rc == L.GM_EINVAL and "aligned" in L.last_error()
    # the prefill router keeps at most 16 K-range partials: D = 4352 would need 17
    wide = _layer(D=4352)
    need = lib.gm_moe_workspace_bytes(ctypes.byref(wide), 16)
    rc = lib.gm_moe_prefill(ctypes.byref(wide), 1024, 1 << 20, 16, 0, 1 << 24, need, None)
    assert rc == L.GM_EINVAL and "prefill supports D <= 8192" in L.last_error()
    # the no-allocation variant rejects a T whose workspace exceeds its static scratch
    assert lib.gm_moe_workspace_bytes(ctypes.byref(s), 200) > L.GM_NOALLOC_SCRATCH_BYTES
    rc = lib.gm_moe_forward_noalloc(ctypes.byref(s), 1024, 1 << 24, 200, 0, None)
    assert rc == L.GM_EWORKSPACE and "static scratch" in L.last_error()
    m = re.search(r"#define GM_NOALLOC_SCRATCH_BYTES \(\(size_t\)(\d+) << (\d+)\)", HEADER)
    assert int(m.group(1)) << int(m.group(2)) == L.GM_NOALLOC_SCRATCH_BYTES
    bad = _layer(norm_w=4100)
    rc = lib.gm_moe_forward(ctypes.byref(bad), 1024, 2048, 1, 0, 4096, 1 << 30, None)
    assert rc == L.GM_EINVAL and "16-byte aligned" in L.last_error()


def test_chain_path_query_without_gpu():
    """gm_moe_chain_fused reports the accumulator-linked path (1) only at T = 1 and the
    combine-linked path (2) only at 2 <= T <= 8, decode shapes with D a multiple of 256 up to
    4096, both with every layer after the first carrying router_t; a rejected layer gives
    its GM_E* code."""
    lib = L.lib()
    a, b = _layer(router_t=512), _layer(router_t=512)
    arr = (L.GmMoeLayer * 2)(a, b)
    assert lib.gm_moe_chain_fused(arr, 2, 1) == 1
    assert lib.gm_moe_chain_fused(arr, 2, 2) == 2
    assert lib.gm_moe_chain_fused(arr, 2, 8) == 2
    assert lib.gm_moe_chain_fused(arr, 2, 9) == 0          # past the decode path
    assert lib.gm_moe_chain_fused((L.GmMoeLayer * 1)(a), 1, 8) == 0
    arr = (L.GmMoeLayer * 2)(_layer(router_t=512, D=4096), _layer(router_t=512, D=4096))
    assert lib.gm_moe_chain_fused(arr, 2, 8) == 2          # 16 slices of 256 columns
    arr = (L.GmMoeLayer * 2)(_layer(router_t=512, D=2048), _layer(router_t=512, D=4096))
    assert lib.gm_moe_chain_fused(arr, 2, 8) == 0          # layers must share D
    arr = (L.GmMoeLayer * 2)(a, _layer())          # layer 1 without router_t: per-layer path
    assert lib.gm_moe_chain_fused(arr, 2, 1) == 0
    assert lib.gm_moe_chain_fused(arr, 2, 8) == 0
    arr = (L.GmMoeLayer * 2)(a, _layer(router_t=512, E=128))   # layers must share E
    assert lib.gm_moe_chain_fused(arr, 2, 1) == 0
    arr = (L.GmMoeLayer * 2)(a, _layer(k=9))
    assert lib.gm_moe_chain_fused(arr, 2, 1) == L.GM_EINVAL
    assert lib.gm_moe_chain_fused(None, 2, 1) == L.GM_EINVAL


def test_core_layer_argument_errors_without_gpu():
    """gm_attn_decode / gm_ssm_decode reject bad shapes, positions and workspaces before
    any launch."""
    lib = L.lib()
    a = L.GmAttnLayer(wqkv=256, wo=256, attn_norm=256, q_norm=256, k_norm=256, eps=1e-6, D=2048, n_head=16,
                      n_head_kv=2, head_dim=256, rope_dim=64)
    n = lib.gm_attn_workspace_bytes(ctypes.byref(a), 4096)
    assert n > 0 and n % 256 == 0
    assert lib.gm_attn_workspace_bytes(ctypes.byref(a), 8192) > n
    bad = L.GmAttnLayer.from_buffer_copy(a)
    bad.head_dim = 96
    assert lib.gm_attn_workspace_bytes(ctypes.byref(bad), 4096) == 0 and "head_dim" in L.last_error()
    rc = lib.gm_attn_decode(ctypes.byref(a), 1024, 2048, 4096, 4096, 4096, 4096, 256, 256, 0, 1 << 20, n, None)
    assert rc == L.GM_EINVAL and "pos" in L.last_error()
    rc = lib.gm_attn_decode(ctypes.byref(a), 1024, 2048, 4096, 4096, 3, 4096, 256, 256, 0, 1 << 20, n - 1, None)
    assert rc == L.GM_EWORKSPACE
    s = L.GmSsmLayer(w_in=256, w_gate=256, w_out=256, alpha=256, beta=256, conv1d=256, a=256, dt_bias=256,
                     ssm_norm=256, attn_norm=256, eps=1e-6, D=2048, n_k_heads=16, n_v_heads=32, d_state=128,
                     conv_k=4)
    m = lib.gm_ssm_workspace_bytes(ctypes.byref(s))
    assert m > 0 and m % 256 == 0
    bad = L.GmSsmLayer.from_buffer_copy(s)
    bad.n_v_heads = 24
    assert lib.gm_ssm_workspace_bytes(ctypes.byref(bad), ) == 0 and "multiple" in L.last_error()
    rc = lib.gm_ssm_decode(ctypes.byref(s), 1024, 1024, 4096, 4096, 0, 1 << 20, m, None)
    assert rc == L.GM_EINVAL and "alias" in L.last_error()
    # the input projections form the RMSNorm from attn_norm with 16-byte loads
    bad = L.GmAttnLayer.from_buffer_copy(a)
    bad.attn_norm = 260
    assert lib.gm_attn_workspace_bytes(ctypes.byref(bad), 4096) == 0 and "attn_norm" in L.last_error()
    bad = L.GmSsmLayer.from_buffer_copy(s)
    bad.attn_norm = 260
    assert lib.gm_ssm_workspace_bytes(ctypes.byref(bad)) == 0 and "attn_norm" in L.last_error()


def test_linked_core_moe_argument_errors_without_gpu():
    """gm_attn_decode_moe / gm_ssm_decode_moe / gm_moe_forward_acc reject a MoE block that
    does not fit the T = 1 accumulator kernels, lacks router_t, has another D, or comes
    with a short workspace, before any launch."""
    lib = L.lib()
    s = L.GmSsmLayer(w_in=256, w_gate=256, w_out=256, alpha=256, beta=256, conv1d=256, a=256, dt_bias=256,
                     ssm_norm=256, attn_norm=256, eps=1e-6, D=2048, n_k_heads=16, n_v_heads=32, d_state=128,
                     conv_k=4)
    m = lib.gm_ssm_workspace_bytes(ctypes.byref(s))
    good = _layer(router_t=512)
    n1 = lib.gm_moe_workspace_bytes(ctypes.byref(good), 1)
    assert n1 > 0

    def ssm(moe, ws_bytes=n1, moe_ws=1 << 22):
        return lib.gm_ssm_decode_moe(ctypes.byref(s), 1024, 1 << 20, 4096, 1 << 21, 0, 1 << 23, m,
                                     ctypes.byref(moe), moe_ws, ws_bytes, None)
    assert ssm(_layer()) == L.GM_EINVAL and "router_t" in L.last_error()
    assert ssm(_layer(router_t=512, D=1024)) == L.GM_EINVAL and "D=2048" in L.last_error()
    assert ssm(_layer(router_t=512, k=4, FF=256)) == L.GM_EINVAL and "accumulator" in L.last_error()
    assert ssm(good, ws_bytes=n1 - 256) == L.GM_EWORKSPACE
    assert ssm(good, moe_ws=1024 + 16) == L.GM_EINVAL and "256-byte" in L.last_error()
    a = L.GmAttnLayer(wqkv=256, wo=256, attn_norm=256, q_norm=256, k_norm=256, eps=1e-6, D=2048, n_head=16,
                      n_head_kv=2, head_dim=256, rope_dim=64)
    na = lib.gm_attn_workspace_bytes(ctypes.byref(a), 64)
    rc = lib.gm_attn_decode_moe(ctypes.byref(a), 1024, 1 << 20, 4096, 4096, 0, 64, 256, 256, 0, 1 << 23, na,
                                ctypes.byref(_layer()), 1 << 22, n1, None)
    assert rc == L.GM_EINVAL and "router_t" in L.last_error()
    rc = lib.gm_moe_forward_acc(ctypes.byref(_layer(router_t=512, k=4, FF=256)), 1024, 1 << 20, 0, 1 << 22, n1, None)
    assert rc == L.GM_EINVAL and "accumulator" in L.last_error()
    rc = lib.gm_moe_forward_acc(ctypes.byref(good), 1024, 1 << 20, 0, 1 << 22, n1 - 256, None)
    assert rc == L.GM_EWORKSPACE
