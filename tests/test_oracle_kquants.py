"""Pins the Q8_0 / Q4_K / Q5_K / Q6_K oracle (oracle/kquants.py, CPU only).

No reference vectors exist for these types, so the decoders are checked against
blocks built weight by weight by the packers (the inverse direction), with expected
values from the closed forms evaluated in float64 and rounded once: every product
is exact, so one fp32 rounding of the exact value is the only correct answer.
"""
import numpy as np
import pytest

from oracle import kquants as K


def _f16(v):
    return float(np.float16(v))


def test_q8_0_closed_form():
    rng = np.random.default_rng(0)
    for _ in range(20):
        d = _f16(rng.standard_normal() * 0.01)
        q = rng.integers(-128, 128, 32)
        y = K.dequant_q8_0(K.pack_q8_0(d, q))
        assert np.array_equal(y, np.float32(np.float64(d) * q))


def test_scale_min_packing_exhaustive():
    # every 6-bit (sc, m) value at every one of the 8 sub-block positions
    for s in range(8):
        for v in range(64):
            sc = [(v + 17 * j) % 64 for j in range(8)]
            m = [(v * 5 + 3 * j) % 64 for j in range(8)]
            sc[s] = v
            m[s] = 63 - v
            got_sc, got_m = K.scale_min_k4(K.pack_scale_min_k4(sc, m)[None, :])
            assert got_sc[0].tolist() == sc and got_m[0].tolist() == m


@pytest.mark.parametrize("five", [False, True])
def test_q4_q5_k_closed_form(five):
    rng = np.random.default_rng(1 + five)
    for _ in range(10):
        d, dmin = _f16(abs(rng.standard_normal()) * 1e-3), _f16(abs(rng.standard_normal()) * 1e-3)
        sc, m = rng.integers(0, 64, 8).tolist(), rng.integers(0, 64, 8).tolist()
        q = rng.integers(0, 32 if five else 16, 256)
        blk = K.pack_q4_k(d, dmin, sc, m, q, five=five)
        y = (K.dequant_q5_k if five else K.dequant_q4_k)(blk)
        want = [np.float32(np.float64(d) * sc[e // 32] * q[e] - np.float64(dmin) * m[e // 32]) for e in range(256)]
        assert np.array_equal(y, np.array(want, np.float32))


def test_q6_k_closed_form():
    rng = np.random.default_rng(3)
    for _ in range(10):
        d = _f16(rng.standard_normal() * 1e-3)
        sc = rng.integers(-128, 128, 16).tolist()
        q = rng.integers(-32, 32, 256)
        y = K.dequant_q6_k(K.pack_q6_k(d, sc, q))
        want = [np.float32(np.float64(d) * sc[e // 16] * q[e]) for e in range(256)]
        assert np.array_equal(y, np.array(want, np.float32))


def test_q6_k_every_value_every_position():
    # each 6-bit value at every weight position (a wrong nibble / bit-pair / byte index
    # moves a value to another weight and fails here)
    for v in range(-32, 32):
        q = np.full(256, v)
        q[::7] = -v - 1 if v < 31 else 0
        y = K.dequant_q6_k(K.pack_q6_k(1.0, [1] * 16, q))
        assert np.array_equal(y, q.astype(np.float32))


def test_q5_k_fifth_bit_positions():
    for e in range(256):
        q = np.zeros(256, np.int64)
        q[e] = 16
        y = K.dequant_q5_k(K.pack_q4_k(1.0, 0.0, [1] * 8, [0] * 8, q, five=True))
        assert np.flatnonzero(y).tolist() == [e] and y[e] == 16.0


def test_multi_block_and_errors():
    rng = np.random.default_rng(4)
    blocks = [K.pack_q6_k(_f16(rng.standard_normal()), rng.integers(-128, 128, 16).tolist(),
                          rng.integers(-32, 32, 256)) for _ in range(3)]
    y = K.dequant_q6_k(np.concatenate(blocks))
    for i, b in enumerate(blocks):
        assert np.array_equal(y[256 * i:256 * i + 256], K.dequant_q6_k(b))
    with pytest.raises(ValueError):
        K.dequant_q6_k(np.zeros(211, np.uint8))
    with pytest.raises(ValueError):
        K.dequant(np.zeros(34, np.uint8), 99)


def test_dequant_matrix_takes_kquant_rows():
    """oracle.quants.dequant_matrix (the OracleLayer's per-call expert dequant) hands
    K-quant rows to this module, row-major, and rejects a byte count that is not
    M x K / block weights blocks."""
    from npu_amd import synth
    from oracle import quants as Q
    g = np.random.default_rng(3)
    for q in (K.Q8_0, K.Q4_K, K.Q5_K, K.Q6_K):
        raw = synth.host_quant_matrix(g, q, 3, 512)
        m = Q.dequant_matrix(raw, q, 3, 512)
        assert m.shape == (3, 512) and np.isfinite(m).all()
        assert np.array_equal(m, K.dequant(raw.reshape(-1), q).reshape(3, 512))
        with pytest.raises(ValueError):
            Q.dequant_matrix(raw.reshape(-1)[:-1], q, 3, 512)
