"""Write the golden vectors for the one oracle function that no closed form, invariant or
reference test pins: the HEX quantizer's exact output (table fit by quantile-started k-means,
fp8 block codes, nearest-level indices) of blackhole/anatomy/hex.py:207-227.

Run in the build container only (the reference checkout is not on the GPU box):

    python tests/golden/make_golden.py /root/reference

It imports blackhole.anatomy.hex (numpy only) from the reference checkout, quantizes a few
seeded matrices and writes tests/golden/quantize.npz: per case the SHA-256 of the input matrix
(regenerated from its seed by the test, which checks the hash), the levels, the expert scale,
the fp8 block codes and the packed index words. Only these data are committed.
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

# (name, out, in, levels, block, seed): N(0, 0.02) weights like the benchmark configs, a case
# above the k-means sample size (131072 values), a ragged width, and both block sizes.
CASES = [
    ("l16_b32", 64, 256, 16, 32, 0),
    ("l8_b32", 48, 128, 8, 32, 1),
    ("l16_b128", 64, 256, 16, 128, 2),
    ("l8_b128_big", 136, 1024, 8, 128, 3),
    ("l16_ragged", 8, 70, 16, 32, 4),
]


def weights(o: int, i: int, seed: int) -> np.ndarray:
    """The seeded N(0, 0.02) input matrix of a case."""
    return (np.random.default_rng(seed).standard_normal((o, i)) * 0.02).astype(np.float32)


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from blackhole.anatomy import hex as hx

    out = {}
    for name, o, i, L, block, seed in CASES:
        W = weights(o, i, seed)
        h = hx.quantize(W, L, block)
        out[f"{name}.W_sha256"] = np.frombuffer(hashlib.sha256(W.tobytes()).digest(), np.uint8)
        out[f"{name}.levels"] = h.levels.astype(np.float32)
        out[f"{name}.expert_scale"] = np.array([h.expert_scale], np.float64)
        out[f"{name}.block_scale"] = h.block_scale.astype(np.uint8)
        out[f"{name}.idx_words"] = hx.pack_bits(h.idx, h.bits, 32)
        out[f"{name}.meta"] = np.array([o, i, L, block, seed], np.int64)
    dst = Path(__file__).with_name("quantize.npz")
    np.savez_compressed(dst, **out)
    print(f"wrote {dst} ({dst.stat().st_size} bytes, {len(CASES)} cases)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
