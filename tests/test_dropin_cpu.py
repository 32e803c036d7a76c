"""Drop-in operator surface without a GPU: names, constants, validation errors.

Mirrors the reference's constructor contract (npu/quant_mv.py:366-397):
TypeError for a non-uint8 weight, ValueError for K % 256 or a wrong byte
count, ValueError / IndexError from the repack helpers.
"""
import numpy as np
import pytest

from npu_amd import quant_mv, quant_mv_iq4, quant_mv_iq4_packed, qwen_moe, synth
from npu_amd.gguf_types import GGMLQuantizationType as QT, QuantTensor


def test_module_constants():
    assert quant_mv.BLK == 256 and quant_mv.B_BYTES == 98
    assert quant_mv_iq4.BLK == 256 and quant_mv_iq4.RAW_B_BYTES == 136 and quant_mv_iq4.B_BYTES == 136
    assert quant_mv_iq4_packed.B_BYTES == 136
    # qwen/forward.py:542-549 derives row bytes from the module constants
    assert (2048 // quant_mv.BLK) * quant_mv.B_BYTES == 784


def test_constructor_errors():
    with pytest.raises(TypeError):
        quant_mv.NpuQuantMatVec(np.zeros(98 * 8, np.int8), 1, 2048)
    with pytest.raises(ValueError):
        quant_mv.NpuQuantMatVec(np.zeros(98, np.uint8), 1, 200)
    with pytest.raises(ValueError):
        quant_mv_iq4.NpuIQ4MatVec(np.zeros(135, np.uint8), 1, 256)
    op = quant_mv_iq4_packed.NpuIQ4PackedMatVec(np.zeros(136 * 2, np.uint8), 2, 256)
    assert op.in_features == 256 and op.out_features == 2


def _stack(qtype, E=3, M=4, K=512):
    g = np.random.Generator(np.random.PCG64(1))
    return QuantTensor("blk.0.ffn_gate_exps.weight", qtype, (K, M, E), synth.host_quant_matrix(g, qtype, M, K, E))


def test_repack_is_zero_copy_raw_rows():
    t = _stack(QT.IQ3_XXS)
    r = quant_mv.repack_iq3_xxs_per_expert(t, 2)
    assert r.shape == (4, 2 * 98) and np.shares_memory(r, t.data)
    assert np.array_equal(r, t.data[2])
    with pytest.raises(IndexError):
        quant_mv.repack_iq3_xxs_per_expert(t, 3)
    with pytest.raises(ValueError):
        quant_mv_iq4.repack_iq4_xs_per_expert(t, 0)       # wrong type
    t4 = _stack(QT.IQ4_XS)
    with pytest.raises(ValueError):
        quant_mv.repack_iq3_xxs_weight(t4)
    assert np.array_equal(quant_mv_iq4_packed.repack_iq4_xs_packed_per_expert(t4, 1), t4.data[1])


def test_enable_npu_rejects_unknown_ops():
    with pytest.raises(ValueError):
        qwen_moe.enable_npu([], ops=("router", "warp_drive"))


def test_quant_tensor_shape_validation():
    g = np.random.Generator(np.random.PCG64(2))
    data = synth.host_quant_matrix(g, QT.IQ4_XS, 4, 512, 2)
    with pytest.raises(ValueError):
        QuantTensor("x", QT.IQ4_XS, (512, 4, 3), data)
