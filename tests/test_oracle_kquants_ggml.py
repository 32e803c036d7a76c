"""oracle.kquants against ggml's own scalar dequantizers, restated loop by loop.

The oracle decodes whole arrays with numpy, from a written layout description; its
other test (test_oracle_kquants.py) checks it against packers written from the same
description.  This test follows the structure of ggml's published reference loops
instead (ggml-quants.c ``dequantize_row_q8_0`` / ``q4_K`` / ``q5_K`` / ``q6_K``, the
functions gguf-py 0.18.0's ``gguf.quants.dequantize`` mirrors; gguf-py is not
vendored in the reference, which pins it at ``uv.lock:132-134``): one block at a time,
ggml's struct field order (``block_q8_0 {d; qs[32]}``, ``block_q4_K {d; dmin;
scales[12]; qs[128]}``, ``block_q5_K {d; dmin; scales[12]; qh[32]; qs[128]}``,
``block_q6_K {ql[128]; qh[64]; scales[16]; d}``) and its loop nesting (64-weight
steps with ``get_scale_min_k4`` for Q4_K / Q5_K, 128-weight halves with four
quarter-streams for Q6_K).  A misreading shared by the oracle and its packers (a
swapped nibble, a scale index off by one) fails here.  Blocks: random bytes with
finite fp16 d / dmin, and all-0x00 / all-0xff payloads.
"""
import numpy as np
import pytest

from oracle import kquants as KQ


def _h(b, o):
    return float(np.frombuffer(bytes(b[o:o + 2]), np.float16)[0])


def _get_scale_min_k4(j, q):
    if j < 4:
        return q[j] & 63, q[j + 4] & 63
    return (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4), (q[j + 4] >> 4) | ((q[j] >> 6) << 4)


def ggml_q8_0(b):
    d = np.float32(_h(b, 0))
    return [np.float32(int(np.int8(np.uint8(b[2 + j])))) * d for j in range(32)]


def ggml_q4_k(b, five=False):
    d, dmin = np.float32(_h(b, 0)), np.float32(_h(b, 2))
    scales = [int(v) for v in b[4:16]]
    qh = [int(v) for v in b[16:48]] if five else None
    q = [int(v) for v in (b[48:176] if five else b[16:144])]
    y, is_, qo, u1, u2 = [], 0, 0, 1, 2
    for _ in range(0, 256, 64):
        sc, m = _get_scale_min_k4(is_ + 0, scales)
        d1, m1 = d * np.float32(sc), dmin * np.float32(m)
        sc, m = _get_scale_min_k4(is_ + 1, scales)
        d2, m2 = d * np.float32(sc), dmin * np.float32(m)
        for l in range(32):
            v = (q[qo + l] & 0xF) + ((16 if qh[l] & u1 else 0) if five else 0)
            y.append(d1 * np.float32(v) - m1)
        for l in range(32):
            v = (q[qo + l] >> 4) + ((16 if qh[l] & u2 else 0) if five else 0)
            y.append(d2 * np.float32(v) - m2)
        qo += 32
        is_ += 2
        u1 <<= 2
        u2 <<= 2
    return y


def ggml_q6_k(b):
    ql = [int(v) for v in b[0:128]]
    qh = [int(v) for v in b[128:192]]
    sc = [int(np.int8(np.uint8(v))) for v in b[192:208]]
    d = np.float32(_h(b, 208))
    y = [None] * 256
    for half in range(2):
        lo, hi, so, yo = 64 * half, 32 * half, 8 * half, 128 * half
        for l in range(32):
            is_ = l // 16
            q1 = ((ql[lo + l] & 0xF) | (((qh[hi + l] >> 0) & 3) << 4)) - 32
            q2 = ((ql[lo + l + 32] & 0xF) | (((qh[hi + l] >> 2) & 3) << 4)) - 32
            q3 = ((ql[lo + l] >> 4) | (((qh[hi + l] >> 4) & 3) << 4)) - 32
            q4 = ((ql[lo + l + 32] >> 4) | (((qh[hi + l] >> 6) & 3) << 4)) - 32
            y[yo + l] = d * np.float32(sc[so + is_ + 0]) * np.float32(q1)
            y[yo + l + 32] = d * np.float32(sc[so + is_ + 2]) * np.float32(q2)
            y[yo + l + 64] = d * np.float32(sc[so + is_ + 4]) * np.float32(q3)
            y[yo + l + 96] = d * np.float32(sc[so + is_ + 6]) * np.float32(q4)
    return y


GGML = {KQ.Q8_0: ggml_q8_0, KQ.Q4_K: ggml_q4_k, KQ.Q5_K: lambda b: ggml_q4_k(b, five=True), KQ.Q6_K: ggml_q6_k}


def _blocks(rng, qtype, n):
    nb = KQ.BLOCK[qtype][1]
    b = rng.integers(0, 256, (n, nb), dtype=np.uint8)
    d_off = 208 if qtype == KQ.Q6_K else 0
    b[:, d_off:d_off + 2] = (rng.standard_normal(n) * 1e-2).astype(np.float16).view(np.uint8).reshape(n, 2)
    if qtype in (KQ.Q4_K, KQ.Q5_K):
        b[:, 2:4] = (np.abs(rng.standard_normal(n)) * 1e-2).astype(np.float16).view(np.uint8).reshape(n, 2)
    edge = b[:2].copy()
    for e, fill in zip(edge, (0x00, 0xFF)):          # all-zero / all-one payloads, d and dmin kept finite
        keep = e.copy()
        e[:] = fill
        for o in ((208,) if qtype == KQ.Q6_K else (0, 2) if qtype in (KQ.Q4_K, KQ.Q5_K) else (0,)):
            e[o:o + 2] = keep[o:o + 2]
    return np.concatenate([b, edge])


@pytest.mark.parametrize("qtype", [KQ.Q8_0, KQ.Q4_K, KQ.Q5_K, KQ.Q6_K])
def test_oracle_matches_ggml_loops(qtype):
    rng = np.random.default_rng(qtype + 100)
    blocks = _blocks(rng, qtype, 24)
    want = np.array([v for blk in blocks for v in GGML[qtype](blk)], np.float32)
    got = KQ.dequant(blocks, qtype)
    assert got.dtype == np.float32 and got.shape == want.shape
    assert np.array_equal(got, want)
