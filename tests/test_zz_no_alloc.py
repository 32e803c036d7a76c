"""gm_moe_forward_noalloc (static device scratch, no allocation) against gm_moe_forward.

Both run the same kernels, so the bar is bit-identical outputs.  Each case makes two
calls in a row through the C ABI, the second with fewer tokens and on a second layer,
so the static scratch still holds the larger first call's intermediates when the
second one runs; the calls go on a non-default stream.  Cases: the decode path
(T = 8 then 3), the prefill path (T = 100 then 24) and a layer with K-quant experts
held as bf16 (decode chunks, T = 12 then 5).
"""
import ctypes

import pytest
import torch

from npu_amd import _lib as L
from npu_amd import synth
from npu_amd.gguf_types import GGMLQuantizationType as QT
from npu_amd.moe import GpuMoeBlock

pytestmark = pytest.mark.gpu


def _noalloc(blk, x, residual, stream):
    y = torch.empty_like(x)
    flags = L.GM_MOE_RESIDUAL if residual else 0
    rc = L.lib().gm_moe_forward_noalloc(ctypes.byref(blk.struct), L.ptr(x), L.ptr(y), x.shape[0], flags,
                                        stream.cuda_stream)
    L.check(rc, "gm_moe_forward_noalloc")
    return y


@pytest.mark.parametrize("name,T1,T2,kw", [
    ("decode", 8, 3, dict()),
    ("prefill", 100, 24, dict()),
    ("kquant-bf16", 12, 5, dict(D=512, FF=256, E=64, q_gate=QT.Q4_K, q_down=QT.Q6_K)),
])
def test_noalloc_matches_forward(gpu, name, T1, T2, kw):
    print(f"noalloc case {name} T1={T1} T2={T2}", flush=True)
    blocks = [GpuMoeBlock.from_host(synth.host_moe_layer(400 + i, norm=True, **kw), device=gpu) for i in range(2)]
    assert L.lib().gm_moe_workspace_bytes(ctypes.byref(blocks[0].struct), T1) <= L.GM_NOALLOC_SCRATCH_BYTES
    s = torch.cuda.Stream()
    for blk, T, residual in ((blocks[0], T1, True), (blocks[1], T2, False)):
        x = torch.from_numpy(synth.host_input(500 + T, T, blk.D, rmsnorm=False)).to(gpu)
        want = blk(x, residual=residual)                        # gm_moe_forward, caller's workspace
        torch.cuda.synchronize()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            got = _noalloc(blk, x, residual, s)
        s.synchronize()
        assert torch.isfinite(got).all()
        assert torch.equal(got, want), f"{name} T={T}: max diff {float((got - want).abs().max()):.3e}"


def test_noalloc_rejects_oversize(gpu):
    blk = GpuMoeBlock.from_host(synth.host_moe_layer(410), device=gpu)
    T = 200
    assert L.lib().gm_moe_workspace_bytes(ctypes.byref(blk.struct), T) > L.GM_NOALLOC_SCRATCH_BYTES
    x = torch.zeros(T, blk.D, device=gpu)
    y = torch.full_like(x, 7.0)
    rc = L.lib().gm_moe_forward_noalloc(ctypes.byref(blk.struct), L.ptr(x), L.ptr(y), T, 0,
                                        torch.cuda.current_stream().cuda_stream)
    assert rc == L.GM_EWORKSPACE and "static scratch" in L.last_error()
    torch.cuda.synchronize()
    assert bool((y == 7.0).all()), "nothing may run on a rejected call"


def test_noalloc_under_graph_capture(gpu):
    """After a first eager call on the device (which resolves the static scratch's address,
    and so must happen outside capture), gm_moe_forward_noalloc is captured in a hipGraph and
    replayed three times with other work between the replays: every replay bit-identical to
    gm_moe_forward, and neither torch's allocator nor the device's free memory moves across
    the eager calls and replays that follow the capture."""
    print("noalloc capture case T=1 and T=8", flush=True)
    blk = GpuMoeBlock.from_host(synth.host_moe_layer(420, norm=True), device=gpu)
    s = torch.cuda.Stream()
    for T in (1, 8):
        x = torch.from_numpy(synth.host_input(520 + T, T, blk.D, rmsnorm=False)).to(gpu)
        want = blk(x, residual=True)
        torch.cuda.synchronize()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            y = torch.empty_like(x)
            L.check(L.lib().gm_moe_forward_noalloc(ctypes.byref(blk.struct), L.ptr(x), L.ptr(y), T,
                                                   L.GM_MOE_RESIDUAL, s.cuda_stream), "gm_moe_forward_noalloc")
        s.synchronize()
        assert torch.equal(y, want)
        y.zero_()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            L.check(L.lib().gm_moe_forward_noalloc(ctypes.byref(blk.struct), L.ptr(x), L.ptr(y), T,
                                                   L.GM_MOE_RESIDUAL, s.cuda_stream), "gm_moe_forward_noalloc")
        with torch.cuda.stream(s):
            z = torch.empty_like(x)                 # the eager calls' output, allocated before measuring
        torch.cuda.synchronize()
        alloc0, free0 = torch.cuda.memory_allocated(), torch.cuda.mem_get_info()[0]
        for rep in range(3):
            y.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, want), f"T={T} replay {rep} differs from gm_moe_forward"
            with torch.cuda.stream(s):              # eager no-alloc work on the same scratch in between
                L.check(L.lib().gm_moe_forward_noalloc(ctypes.byref(blk.struct), L.ptr(want), L.ptr(z), T, 0,
                                                       s.cuda_stream), "gm_moe_forward_noalloc")
            s.synchronize()
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated() == alloc0
        assert torch.cuda.mem_get_info()[0] == free0, "device free memory changed across no-alloc calls"
