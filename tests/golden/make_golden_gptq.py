"""Write golden vectors for the HEX producer with GPTQ rounding, the one producer function no
closed form or reference test pins: the per-expert parts that the pipeline's hexvllm stage writes
(harness/blackhole_pipeline/stages/hexvllm.py:75-96, hex_parts): header scales and Hessian-weighted
k-means levels (reaper/gpu_perf/headers.py:83-107), GPTQ rounding onto the table
(reaper/gpu_perf/gptq.py:134-141), table indices, fp8 block codes and the bit stream
(harness/blackhole_pipeline/pack.py:53-86, 104-110).

Run in the build container only (the reference checkout is not on the GPU box):

    python tests/golden/make_golden_gptq.py /root/reference

It imports those reference modules (torch only), runs hex_parts' sequence on a few seeded
problems on the CPU and writes tests/golden/gptq.npz: per case the SHA-256 of the weights and of
the Hessian (both regenerated from the seed by the test, which checks the hashes), and the
reference's levels, expert scales, fp8 block codes, packed index words and the GPTQ output Q.
Only these data are committed.
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

# (name, experts, out, in, levels, tokens, seed). tokens 0 for an expert = no calibration data.
CASES = [
    ("l16", 2, 32, 128, 16, 512, 0),
    ("l8", 2, 24, 256, 8, 384, 1),
    ("l16_dead", 3, 16, 96, 16, 256, 2),      # a zero weight column, a dead input channel, an empty Hessian
]


def problem(n: int, out: int, inp: int, tokens: int, seed: int):
    """Seeded weights W [n, out, in] N(0, 0.02) and Hessians H [n, in, in] = X^T X of N(0, 1)
    activations with a few heavy channels (float32). Case 'dead' variants are applied by the caller."""
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((n, out, inp)) * 0.02).astype(np.float32)
    H = np.zeros((n, inp, inp), np.float32)
    for e in range(n):
        X = rng.standard_normal((tokens, inp)).astype(np.float32)
        X[:, rng.integers(0, inp, 3)] *= 8.0
        H[e] = X.T @ X
    return W, H


def make_case(name: str, n: int, out: int, inp: int, tokens: int, seed: int):
    W, H = problem(n, out, inp, tokens, seed)
    if name.endswith("dead"):
        W[0, :, 5] = 0.0          # a weight column that is all zero
        H[1, 7, :] = 0.0          # an input channel no token activates
        H[1, :, 7] = 0.0
        H[2] = 0.0                # an expert no token reached
    return W, H


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main(ref: str) -> None:
    root = Path(ref)
    sys.path.insert(0, str(root / "reaper" / "gpu_perf"))
    sys.path.insert(0, str(root / "harness"))
    import torch
    from gptq import gptq_table
    from headers import header_parts

    from blackhole_pipeline.pack import block_codes, expert_scale, mlx_pack, table_indices

    out = {}
    for name, n, o, i, L, tokens, seed in CASES:
        W, H = make_case(name, n, o, i, tokens, seed)
        Wt, Ht = torch.from_numpy(W), torch.from_numpy(H)
        # the sequence of hexvllm.py:81-96 (hex_parts), block 32
        S, Lv = header_parts(Wt, "expert", L, 32, Ht.diagonal(dim1=-2, dim2=-1), False)
        Q = gptq_table(Wt, Ht, S, Lv)
        es = expert_scale(Wt)
        idx = table_indices(Q, S, Lv)
        codes = block_codes(S, es, 32)
        bits = L.bit_length() - 1
        words = mlx_pack(idx.long().reshape(n, o, i // 32, 32), bits).reshape(n, o, -1)
        out[f"{name}__w_sha"] = np.array(sha(W))
        out[f"{name}__h_sha"] = np.array(sha(H))
        out[f"{name}__levels"] = Lv.float().numpy()
        out[f"{name}__expert_scale"] = es.float().numpy()
        out[f"{name}__block_scale"] = codes.view(torch.uint8).numpy()
        out[f"{name}__idx"] = words.view(torch.int32).numpy()
        out[f"{name}__q"] = Q.float().numpy()
        print(name, "levels", Lv.shape, "idx", tuple(words.shape), "q", tuple(Q.shape))
    np.savez_compressed(Path(__file__).with_name("gptq.npz"), **out)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
