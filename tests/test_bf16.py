"""bf16 helpers (qwen/model.py:280-295) against torch's bf16 cast.

``synth.to_bf16`` rounds fp32 to bf16 bits to nearest even with a carry trick
(``(u + 0x7FFF + ((u >> 16) & 1)) >> 16``) and is used for every bf16 router and
shared-gate weight the tests and the GGUF writer make; ``oracle.moe.from_bf16``
widens them back.  Both are checked element by element against torch's own
conversion on halfway cases (both parities), values that round across a binade or up
to inf, +-0, +-inf, subnormals and NaNs with small and large payloads.
"""
import numpy as np
import torch

from npu_amd import synth
from oracle import moe as OM


def _bits(u32):
    return np.array(u32, dtype=np.uint32).view(np.float32)


def _torch_bf16(a):
    return torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def test_to_bf16_matches_torch_on_edge_cases():
    cases = [
        0x00000000, 0x80000000,                      # +-0
        0x7F800000, 0xFF800000,                      # +-inf
        0x3F808000, 0x3F818000,                      # exact halfway, even / odd upper half
        0x3F808001, 0x3F807FFF,                      # just above / below halfway
        0x3FFF8000, 0x3FFFFFFF,                      # rounds up across a binade
        0x7F7F8000, 0x7F7FFFFF, 0xFF7FFFFF,          # rounds up to +-inf
        0x00000001, 0x00008000, 0x00018000, 0x007FFFFF, 0x80008001,   # subnormals, halfway among them
        0x00800000, 0x80800000,                      # smallest normals
    ]
    a = _bits(cases)
    assert np.array_equal(synth.to_bf16(a), _torch_bf16(a))


def test_to_bf16_keeps_nan():
    nans = _bits([0x7FC00000, 0xFFC00000, 0x7F800001, 0xFF800001, 0x7F80FFFF, 0x7FFFFFFF])
    got = synth.to_bf16(nans)
    want = _torch_bf16(nans)
    for g, w in zip(got, want):      # torch writes one canonical NaN; only NaN-ness is fixed
        assert (g & 0x7FFF) > 0x7F80 and (w & 0x7FFF) > 0x7F80, (hex(g), hex(w))


def test_to_bf16_random_and_round_trip():
    g = np.random.default_rng(0)
    a = np.concatenate([g.standard_normal(100_000).astype(np.float32) * 10.0 ** g.integers(-30, 30, 100_000),
                        g.integers(0, 2 ** 32, 100_000, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    a = a[~np.isnan(a)]
    b = synth.to_bf16(a)
    assert np.array_equal(b, _torch_bf16(a))
    back = OM.from_bf16(b)
    assert np.array_equal(back, torch.from_numpy(a).to(torch.bfloat16).to(torch.float32).numpy())
    assert np.array_equal(synth.from_bf16(b), back)
