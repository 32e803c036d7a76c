"""The C-ABI host layer under AddressSanitizer (CPU only).

``python -m npu_amd.build --asan`` builds ``libnpu_amd_asan.so``: the host code of
the library (argument checks, workspace layout, the no-allocation entry point's size
check, error reporting) instrumented with ASan and without device code.  A child
Python process preloads the clang ASan runtime, loads that library
(``NPU_AMD_LIB=asan``) and drives every entry point's host-side paths that return
before any kernel launch: invalid arguments, workspace sizing for many shapes,
alignment and size rejections, and long error messages through ``gm_last_error``.
Any ASan report ends the child with a non-zero status.
"""
import os
import subprocess
import sys
from pathlib import Path

import pytest

from npu_amd import build as B

ROOT = Path(__file__).resolve().parents[1]

CHILD = r'''
import ctypes
from npu_amd import _lib as L
lib = L.lib()
assert "asan" in str(L.LIB_PATH)

def layer(**kw):
    s = L.GmMoeLayer()
    s.gate_exps = s.up_exps = s.down_exps = s.router = 256
    s.q_gate = s.q_up = L.GM_QTYPE_IQ4_XS
    s.q_down = L.GM_QTYPE_IQ3_XXS
    s.q_router = L.GM_QTYPE_BF16
    s.D, s.FF, s.FF_sh, s.E, s.k = 2048, 512, 0, 256, 8
    for k, v in kw.items():
        setattr(s, k, v)
    return s

n = 0
for D in (256, 768, 2048, 4096, 8192):
    for FF in (256, 512, 1024):
        for E in (8, 64, 256, 512):
            for k in (1, 4, 8):
                for T in (0, 1, 3, 8, 9, 64, 512, 2000):
                    s = layer(D=D, FF=FF, E=E, k=min(k, E))
                    w = lib.gm_moe_workspace_bytes(ctypes.byref(s), T)
                    assert w % 256 == 0
                    offs = [ctypes.c_size_t() for _ in range(4)]
                    assert lib.gm_moe_workspace_offsets(ctypes.byref(s), T, *[ctypes.byref(o) for o in offs]) == 0
                    assert all(o.value < max(w, 1) for o in offs)
                    n += 1
for bad in (dict(k=9), dict(k=0), dict(E=600), dict(D=100), dict(q_up=L.GM_QTYPE_IQ3_XXS), dict(q_router=7),
            dict(norm_w=4100), dict(router=0)):
    s = layer(**bad)
    assert lib.gm_moe_workspace_bytes(ctypes.byref(s), 1) == 0
    assert lib.gm_moe_forward(ctypes.byref(s), 1024, 2048, 1, 0, 4096, 1 << 30, None) != 0
    assert len(L.last_error()) > 0
s = layer()
assert lib.gm_moe_forward(ctypes.byref(s), 1024, 1024, 1, 0, 4096, 16, None) == L.GM_EINVAL
assert lib.gm_moe_forward(ctypes.byref(s), 1024, 2048, 1, 0, 4096, 16, None) == L.GM_EWORKSPACE
assert lib.gm_moe_forward(ctypes.byref(s), 1028, 2048, 1, 0, 4096, 1 << 30, None) == L.GM_EINVAL
assert lib.gm_moe_forward(ctypes.byref(s), 1024, 2048, -1, 0, 4096, 1 << 30, None) == L.GM_EINVAL
assert lib.gm_moe_forward_noalloc(ctypes.byref(s), 1024, 1 << 24, 200, 0, None) == L.GM_EWORKSPACE
assert lib.gm_moe_forward_stage(ctypes.byref(s), 1024, 2048, 1, 0, 4096, 1 << 30, 9, None) == L.GM_EINVAL
wide = layer(D=4352)
need = lib.gm_moe_workspace_bytes(ctypes.byref(wide), 16)
assert lib.gm_moe_prefill(ctypes.byref(wide), 1024, 1 << 20, 16, 0, 1 << 24, need, None) == L.GM_EINVAL
assert lib.gm_matvec(L.GM_QTYPE_IQ4_XS, None, 512, 500, None, 1, None, None) == L.GM_EINVAL
assert lib.gm_dequant_f32(7, None, 1, None, None) == L.GM_EINVAL
assert lib.gm_dequant_f32(L.GM_QTYPE_IQ3_XXS, None, 0, None, None) == L.GM_OK
assert lib.gm_moe_dispatch(None, -1, 8, 256, None, None, None, None) == L.GM_EINVAL
assert lib.gm_swiglu_mlp(L.GM_QTYPE_IQ4_XS, 256, 256, L.GM_QTYPE_BF16, 264, 2048, 512, 1024, 1, 2048, 4096,
                         None) == L.GM_EINVAL
# gm_moe_chain argument errors (host checks before any GPU call)
arr = (L.GmMoeLayer * 2)(layer(), layer())
wsp = (ctypes.c_void_p * 2)(1 << 24, 1 << 24)
big = (ctypes.c_size_t * 2)(1 << 30, 1 << 30)
small = (ctypes.c_size_t * 2)(16, 16)
assert lib.gm_moe_chain(arr, 0, 1024, 2048, 4096, 1, 1, wsp, big, None) == L.GM_EINVAL
assert lib.gm_moe_chain(None, 2, 1024, 2048, 4096, 1, 1, wsp, big, None) == L.GM_EINVAL
assert lib.gm_moe_chain(arr, 2, 1024, 1024, 4096, 1, 1, wsp, big, None) == L.GM_EINVAL        # x aliases y
assert lib.gm_moe_chain(arr, 2, 1024, 2048, None, 1, 1, wsp, big, None) == L.GM_EINVAL        # no buf
assert lib.gm_moe_chain(arr, 2, 1024, 2048, 4104, 1, 1, wsp, big, None) == L.GM_EINVAL        # buf alignment
assert lib.gm_moe_chain(arr, 2, 1024, 2048, 4096, 1, 1, wsp, small, None) == L.GM_EWORKSPACE
assert lib.gm_moe_chain(arr, 2, 1024, 2048, 4096, 0, 1, wsp, big, None) == L.GM_OK             # T = 0
mixed = (L.GmMoeLayer * 2)(layer(), layer(D=1024))
assert lib.gm_moe_chain(mixed, 2, 1024, 2048, 4096, 1, 1, wsp, big, None) == L.GM_EINVAL
assert "same" in L.last_error() or "D=" in L.last_error()
print("asan child ok", n)
'''


def test_host_abi_under_asan():
    rt = B.asan_runtime()
    if rt is None:
        pytest.skip("no clang ASan runtime in this ROCm install")
    if B.is_stale(B.LIB_ASAN):
        B.build(asan=True)
    env = dict(os.environ, NPU_AMD_LIB="asan", LD_PRELOAD=rt, HIP_VISIBLE_DEVICES="",
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0:exitcode=86")
    r = subprocess.run([sys.executable, "-c", CHILD], cwd=ROOT, env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "asan child ok" in r.stdout, (r.returncode, r.stdout[-2000:], r.stderr[-4000:])
