"""The HEX producer with GPTQ rounding (blackhole_runtime.gptq) against the golden vectors the
reference's own hexvllm sequence wrote (tests/golden/make_golden_gptq.py; hexvllm.py:75-96), on CPU
tensors: levels, expert scales, fp8 block codes, packed index words and the rounded weights equal
bit for bit. Plus the properties GPTQ promises: dead columns stay zero, every rounded weight is a
table level times its block scale, and the layer error under the Hessian is below plain rounding's."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from blackhole_runtime import gptq

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import make_golden_gptq as G  # noqa: E402  (the fixture script: seeds and shapes, no reference import)

GOLD = np.load(Path(__file__).resolve().parent / "golden" / "gptq.npz")


@pytest.mark.parametrize("case", G.CASES, ids=[c[0] for c in G.CASES])
def test_gptq_parts_match_reference(case):
    name, n, o, i, L, tokens, seed = case
    W, H = G.make_case(name, n, o, i, tokens, seed)
    assert G.sha(W) == str(GOLD[f"{name}__w_sha"]) and G.sha(H) == str(GOLD[f"{name}__h_sha"])
    got = gptq.quantize_experts_gptq(torch.from_numpy(W), torch.from_numpy(H), L)
    assert np.array_equal(got["levels"].numpy(), GOLD[f"{name}__levels"])
    assert np.array_equal(got["expert_scale"].numpy(), GOLD[f"{name}__expert_scale"])
    assert np.array_equal(got["block_scale"].numpy(), GOLD[f"{name}__block_scale"])
    assert np.array_equal(got["idx"].numpy(), GOLD[f"{name}__idx"])
    assert np.array_equal(got["q"].numpy(), GOLD[f"{name}__q"])


def test_gptq_properties():
    name, n, o, i, L, tokens, seed = G.CASES[2]            # the case with dead columns
    W, H = G.make_case(name, n, o, i, tokens, seed)
    got = gptq.quantize_experts_gptq(torch.from_numpy(W), torch.from_numpy(H), L)
    Q = got["q"]
    assert torch.count_nonzero(Q[0, :, 5]) == 0 and torch.count_nonzero(Q[1, :, 7]) == 0
    # every weight is a level times its block's dequant scale (fp8 code * expert scale)
    from oracle import hex_oracle as O
    bits = L.bit_length() - 1
    for e in range(n):
        deq = O.dequant(got["idx"][e:e + 1].numpy().view(np.uint32), got["block_scale"][e:e + 1].numpy(),
                        got["expert_scale"][e:e + 1].numpy(), got["levels"][e:e + 1].numpy(), bits, "R")[0]
        np.testing.assert_allclose(deq[:, (Q[e].abs().amax(0) > 0).numpy()],
                                   Q[e].numpy()[:, (Q[e].abs().amax(0) > 0).numpy()], rtol=2e-6, atol=0)
    # GPTQ beats plain rounding onto the same table under the Hessian (the layer output error)
    Wt, Ht = torch.from_numpy(W), torch.from_numpy(H)
    xn, blk, _ = gptq.block_headers(Wt)
    scale = blk.expand(-1, -1, -1, 32).reshape(Wt.shape)
    rtn = torch.gather(got["levels"], 1, gptq.nearest_index((Wt / scale).clamp(-1, 1), got["levels"]).reshape(n, -1)
                       ).view(Wt.shape) * scale
    for e in range(2):                                       # (expert 2 has no calibration data)
        err = lambda Qe: float(torch.einsum("oi,ij,oj->", (Wt[e] - Qe).double(), Ht[e].double(), (Wt[e] - Qe).double()))
        assert err(Q[e]) < err(rtn[e])
