"""The HEX quantizer the benchmark builds its layers with (blackhole_runtime.quant, nearest
rounding), run on the GPU, against the CPU oracle quantizer: the same expert scales and fp8 block
codes, levels equal up to float summation order (float64 k-means sums on the device), indices
equal except at values within rounding of a midpoint; the device fp8 encoder and bit packing
equal the oracle's exactly."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from blackhole_runtime import quant
from oracle import hex_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("L,block,shape", [(16, 32, (3, 64, 256)), (8, 128, (2, 48, 512)),
                                           (16, 128, (2, 768, 2048)), (8, 128, (2, 2048, 768))])
def test_device_quantizer_matches_oracle(L, block, shape):
    """Includes the benchmark's own call at config 2/3 width (gate/up 768 x 2048 and down
    2048 x 768, fp8 scale per 128 inputs)."""
    print(f"device quantizer L={L} block={block} shape={shape}", flush=True)
    rng = np.random.default_rng(L + block + shape[1])
    W = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    got = quant.quantize_experts(torch.from_numpy(W).to(DEV), L, block)
    assert all(v.is_cuda for v in got.values())
    bits = L.bit_length() - 1
    for e in range(shape[0]):
        q = O.quantize(W[e], L, block)
        assert got["expert_scale"][e].item() == np.float32(q["expert_scale"])
        assert np.array_equal(got["block_scale"][e].cpu().numpy(), q["block_scale"])
        np.testing.assert_allclose(got["levels"][e].cpu().numpy(), q["levels"], rtol=0, atol=2e-6)
        codes = O.unpack_bits(got["idx"][e].cpu().numpy().view(np.uint32), bits, shape[2])
        assert (codes == q["idx"]).mean() > 0.999


def test_device_fp8_encode_and_pack_exact():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(5000) * 100, rng.standard_normal(1000) * 1e-3,
                        np.array([0.0, -0.0, 448.0, -448.0, 500.0, 1e-9], np.float32)]).astype(np.float32)
    assert np.array_equal(quant.fp8_encode(torch.from_numpy(x).to(DEV)).cpu().numpy(), O.fp8_encode(x))
    for bits in (3, 4):
        codes = rng.integers(0, 1 << bits, (3, 5, 96))
        got = quant.pack(torch.from_numpy(codes).to(DEV), bits).cpu().numpy().view(np.uint32)
        assert np.array_equal(got, O.pack(codes, bits))
