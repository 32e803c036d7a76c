"""GGUF container: write -> read round trips, gguf-py's data shaping, errors, and the
TensorStore / build_config surface of qwen/model.py:95-277 (CPU only).

The byte layout checked here is the GGUF v3 container (magic, version, counts, typed
metadata, tensor infos, aligned data section).  The expected bytes of a header are built
by hand in ``test_header_bytes_by_hand`` so that a reader and writer sharing one mistake
would still fail it.
"""
import struct

import numpy as np
import pytest

from npu_amd import gguf_file as G
from npu_amd.gguf_types import GGMLQuantizationType as QT


def _rand_bytes(rng, n):
    return rng.integers(0, 256, n, dtype=np.uint8)


def test_header_bytes_by_hand(tmp_path):
    p = tmp_path / "h.gguf"
    G.write_gguf(p, {"a": G.Typed(7, G.UINT32)}, [("t", int(QT.F32), (4,), np.arange(4, dtype=np.float32))])
    b = p.read_bytes()
    want = b"GGUF" + struct.pack("<IQQ", 3, 1, 1)
    want += struct.pack("<Q", 1) + b"a" + struct.pack("<I", G.UINT32) + struct.pack("<I", 7)
    want += struct.pack("<Q", 1) + b"t" + struct.pack("<I", 1) + struct.pack("<Q", 4) + struct.pack("<IQ", 0, 0)
    assert b[:len(want)] == want
    data_at = (len(want) + 31) // 32 * 32
    assert b[len(want):data_at] == b"\0" * (data_at - len(want))
    assert np.array_equal(np.frombuffer(b[data_at:data_at + 16], np.float32), np.arange(4, dtype=np.float32))


@pytest.mark.parametrize("alignment", [32, 64])
def test_roundtrip(tmp_path, alignment):
    rng = np.random.default_rng(0)
    E, FF, D = 3, 8, 512
    iq4 = _rand_bytes(rng, E * FF * (D // 256) * 136).reshape(E, FF, (D // 256) * 136)
    iq3 = _rand_bytes(rng, FF * (D // 256) * 98).reshape(FF, (D // 256) * 98)
    q6 = _rand_bytes(rng, 2 * 210).reshape(2, 210)
    f32 = rng.standard_normal((FF, D)).astype(np.float32)
    f16 = rng.standard_normal(D).astype(np.float16)
    bf16 = rng.integers(0, 2 ** 16, (4, 64), dtype=np.uint16)
    kv = {"general.architecture": "qwen3next", "s": "héllo", "i": -5, "u": 2 ** 40, "f": 0.25, "b": True,
          "arr_i": [1, 2, 3], "arr_s": ["x", "yz"], "arr_np": np.array([1.5, -2.0], np.float32),
          "u8": G.Typed(200, G.UINT8), "i16": G.Typed(-3, G.INT16), "f64": G.Typed(0.1, G.FLOAT64)}
    tensors = [("blk.0.ffn_gate_exps.weight", int(QT.IQ4_XS), (D, FF, E), iq4),
               ("blk.0.ffn_down_shexp.weight", int(QT.IQ3_XXS), (D, FF), iq3),
               ("q6", int(QT.Q6_K), (256, 2), q6),
               ("dense", int(QT.F32), (D, FF), f32),
               ("vec", int(QT.F16), (D,), f16),
               ("bf", int(QT.BF16), (64, 4), bf16)]
    p = tmp_path / "m.gguf"
    G.write_gguf(p, kv, tensors, alignment=alignment)
    r = G.GGUFReader(p)
    assert r.version == 3 and r.alignment == alignment and r.data_offset % alignment == 0
    f = {k: v.contents() for k, v in r.fields.items()}
    assert f["s"] == "héllo" and f["i"] == -5 and f["u"] == 2 ** 40 and f["b"] is True
    assert f["f"] == 0.25 and f["u8"] == 200 and f["i16"] == -3 and f["f64"] == 0.1
    assert list(f["arr_i"]) == [1, 2, 3] and f["arr_s"] == ["x", "yz"]
    assert np.array_equal(f["arr_np"], np.array([1.5, -2.0], np.float32))
    assert r.fields["arr_s"].types == [G.ARRAY, G.STRING]
    by = {t.name: t for t in r.tensors}
    t = by["blk.0.ffn_gate_exps.weight"]
    assert t.tensor_type == QT.IQ4_XS and t.shape == (D, FF, E) and t.data.shape == (E, FF, 272)
    assert np.array_equal(t.data, iq4) and t.n_bytes == iq4.size and t.data_offset % alignment == 0
    assert np.array_equal(by["blk.0.ffn_down_shexp.weight"].data, iq3)
    assert by["q6"].data.shape == (2, 210) and np.array_equal(by["q6"].data, q6)
    assert by["dense"].data.dtype == np.float32 and np.array_equal(by["dense"].data, f32)
    assert by["vec"].data.dtype == np.float16 and np.array_equal(by["vec"].data, f16)
    assert by["bf"].data.shape == (4, 128) and np.array_equal(by["bf"].data.view(np.uint16), bf16)


def test_errors(tmp_path):
    p = tmp_path / "x.gguf"
    p.write_bytes(b"GGML" + b"\0" * 28)
    with pytest.raises(G.GGUFError, match="not a GGUF"):
        G.GGUFReader(p)
    p.write_bytes(b"GGUF" + struct.pack("<I", 1) + b"\0" * 24)
    with pytest.raises(G.GGUFError, match="version"):
        G.GGUFReader(p)
    G.write_gguf(p, {"k": "v"}, [("t", int(QT.F32), (8,), np.zeros(8, np.float32))])
    full = p.read_bytes()
    p.write_bytes(full[:-40])                                   # data cut short
    with pytest.raises(G.GGUFError):
        G.GGUFReader(p)
    p.write_bytes(full[:30])                                    # metadata cut short
    with pytest.raises(G.GGUFError, match="end of file"):
        G.GGUFReader(p)
    with pytest.raises(G.GGUFError, match="block size"):
        G.tensor_nbytes(QT.IQ4_XS, (100, 2))
    with pytest.raises(G.GGUFError, match="expected"):
        G.write_gguf(p, {}, [("t", int(QT.F32), (8,), np.zeros(7, np.float32))])


def test_nbytes_table():
    # a superblock of 256 weights: IQ4_XS 136 B, IQ3_XXS 98 B, Q6_K 210 B, Q5_K 176 B; Q8_0 34 B per 32
    assert G.tensor_nbytes(QT.IQ4_XS, (2048, 512)) == 8 * 512 * 136
    assert G.tensor_nbytes(QT.IQ3_XXS, (512, 2048, 4)) == 2 * 2048 * 4 * 98
    assert G.tensor_nbytes(QT.Q6_K, (256,)) == 210 and G.tensor_nbytes(QT.Q5_K, (256,)) == 176
    assert G.tensor_nbytes(QT.Q8_0, (64, 3)) == 6 * 34 and G.tensor_nbytes(QT.BF16, (5, 3)) == 30


def _moe_file(tmp_path, rng):
    D, FF, E = 256, 256, 4
    kv = {"general.architecture": "qwen3next", "qwen3next.block_count": 1, "qwen3next.embedding_length": D,
          "qwen3next.expert_count": E, "qwen3next.expert_used_count": 2,
          "qwen3next.expert_feed_forward_length": FF, "qwen3next.attention.layer_norm_rms_epsilon": 1e-6}
    router = rng.standard_normal((E, D)).astype(np.float32)
    gate_inp_sh = rng.standard_normal(D).astype(np.float16)
    bf = rng.integers(0, 2 ** 16, (FF, D), dtype=np.uint16)
    q6 = _rand_bytes(rng, D * 66).reshape(D, 66)
    tensors = [("blk.0.ffn_gate_inp.weight", int(QT.F32), (D, E), router),
               ("blk.0.ffn_gate_inp_shexp.weight", int(QT.F16), (D,), gate_inp_sh),
               ("blk.0.ffn_up_shexp.weight", int(QT.BF16), (D, FF), bf),
               ("blk.0.ffn_down_shexp.weight", int(QT.IQ2_XXS), (FF, D), q6)]
    p = tmp_path / "moe.gguf"
    G.write_gguf(p, kv, tensors)
    return p, router, gate_inp_sh, bf


def test_tensor_store_and_config(tmp_path):
    rng = np.random.default_rng(1)
    p, router, gate_inp_sh, bf = _moe_file(tmp_path, rng)
    ts = G.TensorStore(p)
    assert (ts.cfg.d_model, ts.cfg.n_expert, ts.cfg.n_expert_used, ts.cfg.d_expert_ff, ts.cfg.n_layer) == \
        (256, 4, 2, 256, 1)
    assert ts.cfg.rms_eps == pytest.approx(1e-6)
    assert ts.has("blk.0.ffn_gate_inp.weight") and not ts.has("nope")
    with pytest.raises(KeyError):
        ts.raw("nope")
    got = ts.get("blk.0.ffn_gate_inp.weight")
    assert got.shape == (4, 256) and np.array_equal(got, router)        # (out, in) = reversed ggml dims
    assert np.array_equal(ts.get("blk.0.ffn_gate_inp_shexp.weight"), gate_inp_sh.astype(np.float32))
    want_bf = (bf.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(ts.get("blk.0.ffn_up_shexp.weight").view(np.uint32), want_bf.view(np.uint32))
    assert ts.get("blk.0.ffn_up_shexp.weight", dtype="bf16").dtype == np.uint16
    assert ts.cache_bytes() > 0
    with pytest.raises(NotImplementedError, match="type 16"):
        ts.get("blk.0.ffn_down_shexp.weight")
    with pytest.raises(ValueError, match="stacked"):
        ts.get_expert("blk.0.ffn_gate_inp.weight", 0)


def test_config_needs_metadata(tmp_path):
    p = tmp_path / "c.gguf"
    G.write_gguf(p, {"general.architecture": "qwen3next"}, [])
    with pytest.raises(G.GGUFError, match="embedding_length"):
        G.TensorStore(p)
