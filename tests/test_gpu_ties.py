"""Exact ties, zero logits and infinite logits at the four top-k sites.

torch.topk's order on exact ties is not specified, so the reference
(qwen/forward.py:610) pins no rule; this build's (include/npu_amd.h): ties go to the
lower expert id, -0 equals +0, NaN and +inf rank above every number.  The router rows
here are c_e * v for one positive bf16 vector v and power-of-two (or zero) factors c_e,
and the inputs are positive, so every logit is exactly c_e times the same dot product
(scaling by a power of two is exact at every step, and each row is reduced in the same
order): rows with equal c_e give bit-equal logits, and the expected picks follow from
sorting (-c_e, e).  Sites: the T = 1 decode gate/up kernel (every block selects), the
T > 1 decode routing kernel, the prefill top-k kernel and gm_router_topk.  Tied picks
must also get bit-equal renormalised weights.
"""
import numpy as np
import pytest
import torch

from npu_amd import ops, synth
from npu_amd.moe import GpuMoeBlock

pytestmark = pytest.mark.gpu
E, K, D, FF = 256, 8, 512, 256
BF16_INF, BF16_NINF = 0x7F80, 0xFF80


def _expected(c):
    order = sorted(range(E), key=lambda e: (-c[e], e))
    return order[:K]


def _layer(c, inf_rows=(), ninf_rows=()):
    h = synth.host_moe_layer(77, D=D, FF=FF, E=E, k=K, shared=True)
    v = np.abs(np.random.default_rng(5).standard_normal(D)).astype(np.float32) * 0.05
    rows = c[:, None].astype(np.float32) * synth.from_bf16(synth.to_bf16(v))[None, :]
    h.router = synth.to_bf16(rows).reshape(E, D)          # power-of-two multiples of bf16 values: exact
    for e in inf_rows:
        h.router[e, :] = BF16_INF
    for e in ninf_rows:
        h.router[e, :] = BF16_NINF
    return h


def _sites(gpu, h):
    """ids [T, k] (int64, descending) and weights from every top-k site."""
    x = torch.from_numpy(np.abs(np.random.default_rng(9).standard_normal((12, D))).astype(np.float32) + 0.1)
    blk = GpuMoeBlock.from_host(h, device=gpu)
    out = {}
    for name, T in (("decode T=1", 1), ("decode T=5", 5), ("prefill T=12", 12)):
        blk(x[:T].to(gpu))
        st = blk.stages(T)
        out[name] = (st["topk_ids"].cpu().long(), st["ffn_moe_weights_norm"].cpu())
    router = torch.from_numpy(h.router.view(np.int16)).to(gpu)
    ids, wts, _, _ = ops.router_topk(router, x[:3].to(gpu), K)
    out["gm_router_topk"] = (ids.cpu().long(), wts.cpu())
    return out


def _check_ties(out, c, exp):
    want = torch.tensor(exp)
    for name, (ids, wts) in out.items():
        for t in range(ids.shape[0]):
            assert torch.equal(ids[t], want), f"{name} token {t}: {ids[t].tolist()} != {exp}"
            for a in range(K):
                for b in range(a + 1, K):
                    if c[exp[a]] == c[exp[b]]:
                        assert wts[t, a] == wts[t, b], f"{name}: tied picks {exp[a]}, {exp[b]} differ in weight"


def test_ties_at_the_kth_pick(gpu):
    """Five rows tie for the last three picks: the three lowest ids win."""
    c = np.full(E, -1.0)
    c[[10, 50, 200]] = 4.0
    c[[7, 90]] = 2.0
    c[[255, 3, 100, 31, 30]] = 1.0
    exp = _expected(c)
    assert exp == [10, 50, 200, 7, 90, 3, 30, 31]
    _check_ties(_sites(gpu, _layer(c)), c, exp)


# One row in each of the eight 8-lane groups of the selection's first pass
# (lane l holds ids l + 64 i, so id 8 g lies in group g).  The selection takes
# as candidates the rows at or above the smallest group maximum and sorts them
# in a network when there are at most 32; these cases put the ties there.
ANCHORS = [0, 8, 16, 24, 32, 40, 48, 56]


def test_ties_in_the_candidate_network(gpu):
    """18 candidates (the anchors at 0.5 set the threshold): five rows tie for the
    last three picks inside the 32-lane merge."""
    c = np.full(E, -1.0)
    c[[10, 50, 200]] = 4.0
    c[[7, 90]] = 2.0
    c[[255, 3, 100, 31, 30]] = 1.0
    c[ANCHORS] = 0.5
    exp = _expected(c)
    assert exp == [10, 50, 200, 7, 90, 3, 30, 31]
    _check_ties(_sites(gpu, _layer(c)), c, exp)


def test_ties_with_the_threshold_rows(gpu):
    """13 candidates (16-lane merge): the anchors tie with two more rows at the
    threshold value itself, and the five lowest ids of the ten fill the last picks."""
    c = np.full(E, -1.0)
    c[[10, 50]] = 4.0
    c[7] = 2.0
    c[[255, 100]] = 1.0
    c[ANCHORS] = 1.0
    exp = _expected(c)
    assert exp == [10, 50, 7, 0, 8, 16, 24, 32]
    _check_ties(_sites(gpu, _layer(c)), c, exp)


def test_eight_tied_candidates(gpu):
    """Exactly eight candidates, all tied (the 8-lane sort alone): picks in id order."""
    c = np.full(E, -1.0)
    c[ANCHORS] = 1.0
    exp = _expected(c)
    assert exp == ANCHORS
    _check_ties(_sites(gpu, _layer(c)), c, exp)


def test_zero_logits_at_the_boundary(gpu):
    """Six positive logits, four exact +0.0 logits from zero rows, the rest negative:
    the two lowest-id zero rows fill the last picks."""
    c = np.full(E, -1.0)
    c[[5, 60, 61, 120, 130, 250]] = 1.0
    c[[77, 40, 9, 8]] = 0.0
    exp = _expected(c)
    assert exp == [5, 60, 61, 120, 130, 250, 8, 9]
    _check_ties(_sites(gpu, _layer(c)), c, exp)


def test_infinite_logits(gpu):
    """Router rows of +inf give +inf logits, which rank first in id order; a -inf row
    gives -inf and is never picked (the fp32 sums of the decode kernels and
    gm_router_topk, as F.linear does).  The prefill router multiplies each row with
    three exact bf16 planes of the input, and a plane that is exactly 0 meets the
    infinite weight as inf * 0 = NaN: there every infinite row becomes NaN, so the
    -inf row ranks first too (a deviation confined to non-finite router weights).
    The weights are NaN (softmax of inf), as in torch."""
    c = np.full(E, -1.0)
    c[[11, 12, 13, 14, 15, 16]] = 2.0
    out = _sites(gpu, _layer(c, inf_rows=(21, 20), ninf_rows=(22,)))
    exp = [20, 21, 11, 12, 13, 14, 15, 16]
    exp_prefill = [20, 21, 22, 11, 12, 13, 14, 15]
    for name, (ids, _) in out.items():
        want = exp_prefill if name.startswith("prefill") else exp
        for t in range(ids.shape[0]):
            assert ids[t].tolist() == want, f"{name} token {t}: {ids[t].tolist()}"
