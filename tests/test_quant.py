"""The GPU-side HEX quantizer (blackhole_runtime.quant, used to build the benchmark layers)
against the oracle quantizer, run on CPU tensors: same expert scales and fp8 block codes, levels
equal up to float summation order, indices equal except at values within rounding of a
midpoint; its fp8 encoder and bit packing equal the oracle's exactly."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from blackhole_runtime import quant
from oracle import hex_oracle as O


@pytest.mark.parametrize("L,block,shape", [(16, 32, (3, 64, 256)), (8, 128, (2, 48, 512)), (16, 128, (2, 136, 1024))])
def test_quantizer_matches_oracle(L, block, shape):
    rng = np.random.default_rng(L + block)
    W = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    got = quant.quantize_experts(torch.from_numpy(W), L, block)
    bits = L.bit_length() - 1
    for e in range(shape[0]):
        q = O.quantize(W[e], L, block)
        assert got["expert_scale"][e].item() == np.float32(q["expert_scale"])
        assert np.array_equal(got["block_scale"][e].numpy(), q["block_scale"])
        np.testing.assert_allclose(got["levels"][e].numpy(), q["levels"], rtol=0, atol=2e-6)
        codes = O.unpack_bits(got["idx"][e].numpy().view(np.uint32), bits, shape[2])
        assert (codes == q["idx"]).mean() > 0.999


def test_fp8_encode_and_pack_exact():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(5000) * 100, rng.standard_normal(1000) * 1e-3]).astype(np.float32)
    assert np.array_equal(quant.fp8_encode(torch.from_numpy(x)).numpy(), O.fp8_encode(x))
    for bits in (3, 4):
        codes = rng.integers(0, 1 << bits, (3, 5, 96))
        assert np.array_equal(quant.pack(torch.from_numpy(codes), bits).numpy().view(np.uint32), O.pack(codes, bits))
