"""The MoE-block oracle (restatement of qwen/forward.py:563-665) against an
independent fp64 formulation and against the committed small-block fixture.

``moe_forward_dense64`` shares no code path with ``moe_forward`` beyond the
dequantisation (pinned separately): it builds a dense [T, E] routing matrix
from an fp64 softmax, a stable argsort instead of topk, evaluates every
selected expert on every token and weights the outputs, then adds the gated
shared expert.  A dropped renormalisation, a softmax applied after top-k, a
missing shared gate, a wrong combine order or index would all break the
agreement.  The fixture pins the oracle's outputs on fixed seeds.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from npu_amd import synth
from npu_amd.gguf_types import GGMLQuantizationType as QT
from oracle import moe as OM

FIX = Path(__file__).parent / "golden" / "moe_small.npz"


@pytest.mark.parametrize("seed,bias,norm,shared,q_gate,q_down", [
    (1, False, False, True, QT.IQ4_XS, QT.IQ3_XXS),
    (2, True, False, True, QT.IQ3_XXS, QT.IQ4_XS),
    (3, False, True, False, QT.IQ4_XS, QT.IQ4_XS),
    (4, True, True, True, QT.IQ3_XXS, QT.IQ3_XXS),
])
@pytest.mark.parametrize("T", [1, 5])
def test_oracle_matches_dense_fp64(seed, bias, norm, shared, q_gate, q_down, T):
    h = synth.host_moe_layer(seed, D=256, FF=256, E=16, k=4, q_gate=q_gate, q_down=q_down, shared=shared,
                             bias=bias, norm=norm)
    ol = OM.OracleLayer(h)
    x = torch.from_numpy(synth.host_input(seed + 100, T, h.D, rmsnorm=not norm))
    margin = OM.topk_margin(OM.router_logits64(x, ol), h.k)
    assert bool((margin > 1e-5).all())
    y = OM.block_forward(x, ol)
    ref = OM.moe_forward_dense64(x, ol)
    assert OM.rel_err(y, ref) < 2e-6


def test_oracle_routing_stages_follow_definitions():
    """softmax over all E, top-k of the probabilities, renormalisation with clamp_min."""
    h = synth.host_moe_layer(7, D=256, FF=256, E=16, k=4, bias=True)
    ol = OM.OracleLayer(h)
    x = torch.from_numpy(synth.host_input(8, 6, h.D))
    st = {}
    OM.block_forward(x, ol, stages=st)
    p = torch.softmax(st["ffn_moe_logits"].double(), -1)
    order = torch.argsort(-p, dim=-1, stable=True)[:, :h.k]
    assert torch.equal(order, st["topk_ids"])
    sel = torch.gather(p, 1, order)
    assert torch.allclose(st["ffn_moe_weights_norm"].double(), sel / sel.sum(-1, keepdim=True), rtol=1e-6)
    assert torch.allclose(st["ffn_moe_weights_norm"].sum(-1), torch.ones(6), atol=1e-6)


def test_oracle_small_block_fixture():
    d = np.load(FIX)
    for case in range(int(d["n_cases"])):
        p = {k: int(d[f"c{case}_{k}"]) for k in ("seed", "T", "bias", "norm", "shared", "q_gate", "q_down")}
        h = synth.host_moe_layer(p["seed"], D=256, FF=256, E=16, k=4, q_gate=p["q_gate"], q_down=p["q_down"],
                                 shared=bool(p["shared"]), bias=bool(p["bias"]), norm=bool(p["norm"]))
        x = d[f"c{case}_x"]
        assert np.array_equal(x, synth.host_input(p["seed"] + 100, p["T"], 256, rmsnorm=not p["norm"]))
        st = {}
        y = OM.block_forward(torch.from_numpy(x), OM.OracleLayer(h), stages=st).numpy()
        np.testing.assert_allclose(y, d[f"c{case}_y64"], rtol=0, atol=2e-6 * np.abs(d[f"c{case}_y64"]).max())
        assert np.array_equal(st["topk_ids"].numpy(), d[f"c{case}_ids"])


def test_rms_norm_invariants():
    """oracle.moe.rms_norm (qwen/forward.py:58-61) against what the formula fixes, with no
    second copy of it: with weight 1 the output's mean square is 1 (to eps), so a sum in
    place of a mean or a missing square root fails; scaling x by c leaves the output
    unchanged (up to eps), so a missing normalisation fails; the weight multiplies element by
    element (a weight of 2 doubles exactly, a one-hot weight keeps one column), so a weight
    applied before the statistics or broadcast on the wrong axis fails; eps enters under the
    root (x = 0 gives 0, a constant row c gives c / sqrt(c^2 + eps) in closed form); the
    reduction runs over the last axis only."""
    g = torch.Generator().manual_seed(7)
    x = torch.randn(5, 2048, generator=g, dtype=torch.float32) * 3.0 + 0.5
    eps = 1e-6
    y = OM.rms_norm(x, None, eps)
    ms = y.double().pow(2).mean(-1)
    assert torch.allclose(ms, torch.ones_like(ms), rtol=0, atol=1e-5)
    for c in (1e-3, 7.0, 1e4):
        assert torch.allclose(OM.rms_norm(x * c, None, 0.0), OM.rms_norm(x, None, 0.0), rtol=1e-6, atol=1e-6)
    assert torch.equal(OM.rms_norm(x, torch.full((2048,), 2.0), eps), 2.0 * y)
    onehot = torch.zeros(2048)
    onehot[17] = 1.0
    z = OM.rms_norm(x, onehot, eps)
    assert torch.equal(z[:, 17], y[:, 17]) and int((z != 0).sum()) == 5
    assert torch.equal(OM.rms_norm(torch.zeros(3, 64), None, eps), torch.zeros(3, 64))
    for c in (0.25, 3.0, -5.0):
        row = torch.full((1, 256), c, dtype=torch.float32)
        want = c / np.sqrt(np.float64(c) ** 2 + 1e-2)
        assert abs(float(OM.rms_norm(row, None, 1e-2)[0, 0]) - want) < 1e-6 * abs(want)
    # last axis only: each row normalised by its own statistics
    rows = torch.stack([x[0], 100.0 * x[1]])
    assert torch.allclose(OM.rms_norm(rows, None, eps)[1], y[1], rtol=1e-5, atol=1e-6)
