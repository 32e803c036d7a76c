"""NpuLinear's host-side contract (npu/linear.py:147-244): shape bookkeeping and the
share_N_pad check, without a GPU (the weight goes to the device on the first call)."""
import pytest
import torch

from npu_amd.linear import NpuLinear


def test_shape_and_share_n_pad():
    W = torch.zeros(576, 1536)
    lin = NpuLinear(W, share_N_pad=3072)
    assert (lin.out_features, lin.in_features, lin.share_N_pad) == (576, 1536, 3072)
    with pytest.raises(ValueError):
        NpuLinear(W, share_N_pad=512)
    with pytest.raises(AssertionError):
        NpuLinear(torch.zeros(4, 4, 4))
    with pytest.raises(ValueError):
        NpuLinear(torch.zeros(8, 100))
