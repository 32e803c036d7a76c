"""GPU parity: dequant, matvec, SwiGLU MLP, router top-k and dispatch vs the CPU oracle.

Tolerances: dequant is float-equal (exact products); fp32-accumulate
products use rel = max|y - ref| / max|ref| <= 1e-3 (
qwen/test_npu_experts.py:93 defines rel); top-k ids must be identical except
for tokens whose fp64 8th/9th logit gap is below 1e-5 (reported as ambiguous,
the near-tie rule of qwen/test_npu_generate5.py:107-124).
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from npu_amd import _lib as L
from npu_amd import ops, synth
from npu_amd.gguf_types import GGMLQuantizationType as QT
from oracle import moe as OM
from oracle import quants as Q

pytestmark = pytest.mark.gpu
KAT = np.load(__import__("pathlib").Path(__file__).resolve().parent / "golden" / "iq_kat.npz")
REL_TOL = 1e-3


def _g(seed):
    return np.random.Generator(np.random.PCG64(seed))


@pytest.mark.parametrize("qtype", [QT.IQ4_XS, QT.IQ3_XXS])
def test_dequant_kat_exact(gpu, qtype):
    blocks = KAT["iq4_blocks" if qtype == QT.IQ4_XS else "iq3_blocks"]
    want = KAT["iq4_expected" if qtype == QT.IQ4_XS else "iq3_expected"].reshape(-1)
    got = ops.dequant(qtype, torch.from_numpy(blocks.copy()).to(gpu)).cpu().numpy()
    assert np.array_equal(got, want)


@pytest.mark.parametrize("qtype", [QT.IQ4_XS, QT.IQ3_XXS])
def test_dequant_random_exact(gpu, qtype):
    blocks = synth.host_superblocks(_g(11), qtype, 4096)
    got = ops.dequant(qtype, torch.from_numpy(blocks).to(gpu)).cpu().numpy()
    want = Q.dequant(blocks, qtype)
    assert np.array_equal(got, want)


def _ref_matvec(w_raw, qtype, M, K, x):
    W = torch.from_numpy(Q.dequant_matrix(w_raw, qtype, M, K))
    return F.linear(x, W), (x.double() @ W.double().T)


@pytest.mark.parametrize("qtype,M,K", [
    (QT.IQ4_XS, 512, 2048),    # config 1
    (QT.IQ3_XXS, 2048, 512),   # config 2
    (QT.IQ3_XXS, 512, 2048),   # config 2, transposed shape
    (QT.IQ4_XS, 2048, 512),    # model's down shape
    (QT.IQ4_XS, 40, 256),
    (QT.IQ3_XXS, 33, 4096),
    (QT.IQ4_XS, 70, 1024),     # one-token kernel: every lanes-per-row / sub-blocks-per-lane branch
    (QT.IQ3_XXS, 9, 8192),
    (QT.IQ4_XS, 3, 12288),     # one token past the one-token kernel's K limit
    (QT.IQ3_XXS, 21, 1536),    # one-token kernel: lanes 48..63 of each row past the last sub-block
    (QT.IQ4_XS, 50, 3072),     # one-token kernel: second sub-block per lane live on half the lanes
    (QT.IQ4_XS, 26, 768),      # 32 lanes per row, 8 of them past the last sub-block
])
@pytest.mark.parametrize("n_tok", [1, 3, 8, 13])
def test_matvec(gpu, qtype, M, K, n_tok):
    w = synth.host_quant_matrix(_g(M * 7 + K), qtype, M, K)
    x = torch.from_numpy(_g(5).standard_normal((n_tok, K)).astype(np.float32))
    y = ops.matvec(qtype, torch.from_numpy(w).to(gpu), M, K, x.to(gpu)).cpu()
    ref32, ref64 = _ref_matvec(w, qtype, M, K, x)
    assert y.shape == (n_tok, M)
    assert OM.rel_err(y, ref32) <= REL_TOL
    assert OM.rel_err(y, ref64) <= 1e-5
    # per-token relative error: a row or token mix-up moves one entry, not the max
    assert float(((y.double() - ref64).abs() / ref64.abs().amax(dim=1, keepdim=True)).max()) <= 1e-5


# Tall one-token matvecs (a batched launch over many matrices stacked by rows, as
# bench.py's configs 1-2 legs run them): the kernel then gives each wave 2, 4 or 8 row
# groups with all their sub-blocks in flight.  Against float64 on the exact device
# dequant, and row slices recomputed as separate short calls (1 row group per wave)
# must be bit-identical: each row's sum is formed in the same order either way.
@pytest.mark.parametrize("qtype,M,K", [
    (QT.IQ4_XS, 32768 + 37, 2048),     # 8 row groups per wave, ragged last block
    (QT.IQ3_XXS, 131072 + 6, 512),     # 16 lanes per row, 8 row groups
    (QT.IQ3_XXS, 16384 + 1, 2048),     # 4 row groups
    (QT.IQ4_XS, 8192 + 3, 8192),       # 4 sub-blocks per lane, 2 row groups
    (QT.IQ4_XS, 8192, 4096),           # 2 sub-blocks per lane, 2 row groups
])
def test_matvec_tall(gpu, qtype, M, K):
    gen = torch.Generator(device=gpu)
    gen.manual_seed(M + K)
    W = synth.device_quant_matrix(gen, qtype, M, K, None, gpu)
    x = torch.randn(K, generator=gen, device=gpu)
    y = ops.matvec(qtype, W, M, K, x.view(1, K)).view(M)
    Wd = ops.dequant(qtype, W.reshape(-1)).view(M, K).double()
    ref = Wd @ x.double()
    assert OM.rel_err(y, ref) <= 1e-5
    assert float(((y.double() - ref).abs() / ref.abs().max()).max()) <= 1e-5
    for r0, n in ((0, 512), (M - 300, 300), (M // 2 + 5, 96)):
        ys = ops.matvec(qtype, W[r0:r0 + n].clone(), n, K, x.view(1, K)).view(n)   # clone: 16-byte aligned
        assert torch.equal(ys, y[r0:r0 + n]), f"rows {r0}..{r0 + n} differ from the tall call"


# The projection shapes of qwen/test_npu_ssm.py and test_npu_attn_o.py (8192 x 2048,
# 4096 x 2048, 2048 x 4096), plus ragged M, K tails inside a 512-wide slot, and K
# large enough for two passes over the row.
@pytest.mark.parametrize("M,K", [(8192, 2048), (4096, 2048), (2048, 4096), (33, 256), (100, 768),
                                 (17, 12288), (5, 16384), (256, 2048), (576, 576), (40, 800), (9000, 96)])
@pytest.mark.parametrize("n_tok", [1, 2, 3, 8, 13, 17])
def test_matvec_bf16(gpu, M, K, n_tok):
    W = synth.host_bf16_normal(_g(M + K), (M, K), 0.02)
    x = torch.from_numpy(_g(2).standard_normal((n_tok, K)).astype(np.float32))
    y = ops.matvec(QT.BF16, torch.from_numpy(W.view(np.int16)).to(gpu), M, K, x.to(gpu)).cpu()
    ref = x.double() @ torch.from_numpy(synth.from_bf16(W)).double().T
    assert y.shape == (n_tok, M)
    assert OM.rel_err(y, ref) <= 1e-5
    # per-token relative error: a row or token mix-up moves one entry, not the max
    assert float(((y.double() - ref).abs() / ref.abs().amax(dim=1, keepdim=True)).max()) <= 1e-5


@pytest.mark.parametrize("q_gu,q_d", [(QT.IQ4_XS, QT.IQ3_XXS), (QT.IQ3_XXS, QT.IQ4_XS)])
@pytest.mark.parametrize("n_tok", [1, 5])
def test_swiglu_mlp(gpu, q_gu, q_d, n_tok):
    D, FF = 2048, 512
    wg = synth.host_quant_matrix(_g(21), q_gu, FF, D)
    wu = synth.host_quant_matrix(_g(22), q_gu, FF, D)
    wd = synth.host_quant_matrix(_g(23), q_d, D, FF)
    x = torch.from_numpy(synth.host_input(3, n_tok, D))
    dev = [torch.from_numpy(a).to(gpu) for a in (wg, wu, wd)]
    y = ops.swiglu_mlp(q_gu, dev[0], dev[1], q_d, dev[2], D, FF, x.to(gpu)).cpu()
    G = torch.from_numpy(Q.dequant_matrix(wg, q_gu, FF, D))
    U = torch.from_numpy(Q.dequant_matrix(wu, q_gu, FF, D))
    Dn = torch.from_numpy(Q.dequant_matrix(wd, q_d, D, FF))
    ref = F.linear(F.silu(F.linear(x, G)) * F.linear(x, U), Dn)
    assert OM.rel_err(y, ref) <= REL_TOL


@pytest.mark.parametrize("T,E,k,bias", [(1, 256, 8, False), (8, 256, 8, False), (64, 256, 8, True),
                                        (5, 16, 4, False), (3, 512, 8, True)])
def test_router_topk(gpu, T, E, k, bias):
    D = 2048
    h = synth.host_moe_layer(31 + E, D=D, FF=256, E=E, k=k, shared=True, bias=bias, norm=True)
    ol = OM.OracleLayer(h)
    x = torch.from_numpy(synth.host_input(4, T, D, rmsnorm=False))
    dev = lambda a: torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to(gpu)
    ids, wts, logits, shg = ops.router_topk(dev(h.router), x.to(gpu), k,
                                            bias=dev(h.router_bias) if bias else None,
                                            w_sh_gate=dev(h.sh_gate_inp), norm_w=dev(h.norm_w), eps=1e-6)
    st = {}
    xn = OM.rms_norm(x, ol.norm_w, 1e-6)
    OM.moe_forward(xn.unsqueeze(0), ol, stages=st)
    margin = OM.topk_margin(OM.router_logits64(x, ol), k)
    assert bool((margin > 1e-5).all()), "near-tie token: choose another seed"
    assert torch.equal(ids.cpu().long(), st["topk_ids"])
    assert torch.allclose(logits.cpu(), st["ffn_moe_logits"], rtol=0, atol=2e-5)
    assert torch.allclose(wts.cpu(), st["ffn_moe_weights_norm"], rtol=1e-5, atol=1e-6)
    assert torch.allclose(shg.cpu(), st["shared_expert_gate_sigmoid"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("T,D", [(1, 16384), (3, 8192), (8, 4864), (9, 5120)])
def test_router_topk_wide_d(gpu, T, D):
    """gm_router_topk at its advertised width limits: one token at D = 16384 (x staged in
    64 KiB + 64 B of LDS), eight tokens at D = 4864 (8 staged rows in 152 KiB, near the
    160 KiB limit), and T > 1 beyond that (one launch per token)."""
    h = synth.host_moe_layer(50 + T, D=D, FF=256, E=64, k=4, shared=True, norm=True)
    ol = OM.OracleLayer(h)
    x = torch.from_numpy(synth.host_input(6 + T, T, D, rmsnorm=False))
    dev = lambda a: torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to(gpu)
    ids, wts, logits, shg = ops.router_topk(dev(h.router), x.to(gpu), 4, w_sh_gate=dev(h.sh_gate_inp),
                                            norm_w=dev(h.norm_w), eps=1e-6)
    st = {}
    OM.moe_forward(OM.rms_norm(x, ol.norm_w, 1e-6).unsqueeze(0), ol, stages=st)
    assert bool((OM.topk_margin(OM.router_logits64(x, ol), 4) > 1e-5).all())
    assert torch.equal(ids.cpu().long(), st["topk_ids"])
    assert torch.allclose(logits.cpu(), st["ffn_moe_logits"], rtol=0, atol=5e-5)
    assert torch.allclose(shg.cpu(), st["shared_expert_gate_sigmoid"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("T,k,E", [(512, 8, 256), (1, 8, 256), (37, 4, 16), (2000, 8, 512)])
def test_dispatch_stable_sort(gpu, T, k, E):
    g = _g(T + E)
    ids = np.stack([g.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    counts, offsets, pairs = ops.moe_dispatch(torch.from_numpy(ids).to(gpu), E)
    counts, offsets, pairs = counts.cpu().numpy(), offsets.cpu().numpy(), pairs.cpu().numpy()
    flat = ids.reshape(-1)
    assert np.array_equal(counts, np.bincount(flat, minlength=E))
    assert np.array_equal(offsets, np.concatenate([[0], np.cumsum(counts)]))
    assert np.array_equal(pairs, np.argsort(flat, kind="stable"))


def _kquant_blocks(rng, qtype, n):
    """Random blocks of a K-quant / Q8_0 type with finite fp16 d (and dmin)."""
    from oracle import kquants as KQ
    w, nb = KQ.BLOCK[qtype]
    b = rng.integers(0, 256, (n, nb), dtype=np.uint8)
    d = (rng.standard_normal(n) * 1e-2).astype(np.float16).view(np.uint8).reshape(n, 2)
    if qtype == KQ.Q6_K:
        b[:, 208:210] = d
    else:
        b[:, 0:2] = d
        if qtype != KQ.Q8_0:
            b[:, 2:4] = (np.abs(rng.standard_normal(n)) * 1e-2).astype(np.float16).view(np.uint8).reshape(n, 2)
    return b


@pytest.mark.parametrize("qtype", [QT.Q8_0, QT.Q4_K, QT.Q5_K, QT.Q6_K])
def test_transcode_i8_exact(gpu, qtype):
    """gm_transcode_i8: every I8 sub-block's s q + off (fp32, one rounding at most) equals
    the oracle's dequant bit for bit; the padding is zero."""
    from oracle import kquants as KQ
    rng = np.random.default_rng(int(qtype) + 40)
    for n in (1, 9, 300):
        b = _kquant_blocks(rng, int(qtype), n)
        out = ops.transcode_i8(int(qtype), torch.from_numpy(b.reshape(-1)).to(gpu)).cpu().numpy().reshape(-1, 48)
        q = out[:, :32].view(np.int8).astype(np.float32)
        s = out[:, 32:48].view(np.float32)
        w = np.where(np.arange(32)[None, :] < 16, s[:, 0:1], s[:, 1:2]) * q + s[:, 2:3]
        assert np.array_equal(w.reshape(-1), KQ.dequant(b, int(qtype)))
        assert np.all(out[:, 44:48] == 0)


@pytest.mark.parametrize("qtype", [QT.Q8_0, QT.Q4_K, QT.Q5_K, QT.Q6_K])
def test_dequant_kquants_exact(gpu, qtype):
    """Device dequant of the loader-path types equals the oracle restatement (float equality)."""
    from oracle import kquants as KQ
    rng = np.random.default_rng(int(qtype))
    for n in (1, 7, 300):
        b = _kquant_blocks(rng, int(qtype), n)
        got = ops.dequant(int(qtype), torch.from_numpy(b.reshape(-1)).to(gpu)).cpu().numpy()
        assert np.array_equal(got, KQ.dequant(b, int(qtype)))


@pytest.mark.parametrize("T", [1, 12])
def test_tensor_store_kquant_shared_expert(gpu, tmp_path, T):
    """A layer whose shared expert is Q6_K / Q8_0 in the file (as in the real model): the
    drop-in transcodes the file's bytes to I8 rows (Q6_K gate beside Q8_0 up) and runs
    them beside the IQ routed experts, also for T > 8 (the routed experts on the prefill
    GEMMs, the shared expert as an fp32 pass of its own).  Bar: 1e-3 (decode), 1e-2
    (prefill)."""
    from npu_amd import gguf_file, qwen_moe
    from oracle import kquants as KQ
    rng = np.random.default_rng(7)
    D, FF, E = 256, 256, 8
    h = synth.host_moe_layer(70, D=D, FF=FF, E=E, k=2, shared=False)
    gate_sh = _kquant_blocks(rng, KQ.Q6_K, FF * D // 256).reshape(FF, -1)
    up_sh = _kquant_blocks(rng, KQ.Q8_0, FF * D // 32).reshape(FF, -1)
    down_sh = _kquant_blocks(rng, KQ.Q6_K, D * FF // 256).reshape(D, -1)
    path = tmp_path / "k.gguf"
    synth.write_gguf_model(path, [h])
    r = gguf_file.GGUFReader(path)
    kv = {k: f.contents() for k, f in r.fields.items()}
    tensors = [(t.name, int(t.tensor_type), t.shape, np.array(t.data)) for t in r.tensors]
    tensors += [("blk.0.ffn_gate_shexp.weight", int(QT.Q6_K), (D, FF), gate_sh),
                ("blk.0.ffn_up_shexp.weight", int(QT.Q8_0), (D, FF), up_sh),
                ("blk.0.ffn_down_shexp.weight", int(QT.Q6_K), (FF, D), down_sh),
                ("blk.0.ffn_gate_inp_shexp.weight", int(QT.F32), (D,), np.full(D, 0.01, np.float32))]
    gguf_file.write_gguf(path, kv, tensors)
    ts = gguf_file.TensorStore(path)
    g = ts.get("blk.0.ffn_gate_shexp.weight")
    assert np.array_equal(g, KQ.dequant(gate_sh, KQ.Q6_K).reshape(FF, D))
    assert np.array_equal(ts.get("blk.0.ffn_up_shexp.weight"), KQ.dequant(up_sh, KQ.Q8_0).reshape(FF, D))
    layer = qwen_moe.MoELayer.load(ts, 0)
    assert layer.w_gate_sh is not None and layer.w_gate_sh.shape == (FF, D)
    x = torch.from_numpy(synth.host_input(3, T, D)).reshape(1, T, D)
    ol = OM.OracleLayer(h)
    assert bool((OM.topk_margin(OM.router_logits64(x.reshape(T, D), ol), h.k) > 1e-5).all())
    y = qwen_moe.moe_forward(x, layer, ts.cfg)
    # reference: routed part from the oracle, shared expert in fp64 from the dequantised weights
    routed = OM.moe_forward(x, ol).double()
    xs = x.reshape(T, D).double()
    gs, us, ds = (torch.from_numpy(KQ.dequant(a, t).reshape(shp)).double() for a, t, shp in
                  ((gate_sh, KQ.Q6_K, (FF, D)), (up_sh, KQ.Q8_0, (FF, D)), (down_sh, KQ.Q6_K, (D, FF))))
    hsh = F.silu(xs @ gs.T) * (xs @ us.T)
    sgate = torch.sigmoid(xs @ torch.full((D,), 0.01, dtype=torch.float64))
    ref = routed.reshape(T, D) + sgate[:, None] * (hsh @ ds.T)
    assert layer.npu["moe_block"].q_gate_sh == L.GM_QTYPE_I8
    assert OM.rel_err(y.reshape(T, D).double(), ref) <= (1e-3 if T <= 8 else 1e-2)
