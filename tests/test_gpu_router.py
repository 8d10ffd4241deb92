"""Routing on the GPU against the CPU oracle (reaper/reaper_pipeline/moe.py:141-168 restated):
bh_hex_route_select on given logits (both branches, correction bias, group-limited choice,
scaling), and bh_hex_route_gemm (the gate linear on the matrix cores, then the choice).

Ids are exact; weights within a few float32 ulp (the order of the k-term sum differs). The
router GEMM's logits accumulate in float32 on the device and are rounded to the activation dtype
as the gate linear's output is: against float64 products rounded the same way they are equal or
one unit of the activation dtype apart (a float32 sum near a rounding boundary), and the choice
is exact on the kernel's own logits."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from blackhole_runtime import hex_moe as hm
from oracle import hex_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = [
    dict(),
    dict(renormalize=False),
    dict(scoring="sigmoid"),
    dict(scoring="sigmoid", routed_scaling_factor=2.5),
    dict(bias=True, routed_scaling_factor=2.5),                       # DeepSeek-V3 / Kimi style gate
    dict(bias=True, n_group=8, topk_group=4, routed_scaling_factor=2.5),
    dict(scoring="sigmoid", n_group=4, topk_group=1),
    dict(bias=True, n_group=16, topk_group=16, renormalize=False),
]


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _opts(c, E, seed):
    o = {k: v for k, v in c.items() if k != "bias"}
    bias = None
    if c.get("bias"):
        bias = (np.random.default_rng(seed).standard_normal(E) * 0.5).astype(np.float32)
    return o, bias


def _oracle(lg, k, o, bias):
    return O.route_select(lg, k, o.get("scoring", "softmax"), o.get("renormalize", True), o.get("n_group", 1),
                          o.get("topk_group", 0), bias, o.get("routed_scaling_factor", 1.0))


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("T,E,k,dt", [(37, 128, 8, torch.float32), (16, 96, 8, torch.bfloat16),
                                      (5, 1024, 16, torch.float32), (300, 64, 6, torch.float16)])
def test_route_select(case, T, E, k, dt):
    c = CASES[case]
    if c.get("n_group", 1) > 1 and E % c["n_group"]:
        pytest.skip("groups do not divide the experts")
    say(f"route_select {c} T={T} E={E} k={k} {dt}")
    o, bias = _opts(c, E, case)
    lg = torch.randn(T, E, generator=torch.Generator().manual_seed(case * 100 + T)).to(dt)
    w, ids = hm.route_select(lg.to(DEV), k, correction_bias=None if bias is None else torch.from_numpy(bias), **o)
    w_ref, ids_ref = _oracle(lg.float().numpy(), k, o, bias)
    assert np.array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=2e-6, atol=1e-12)


@pytest.mark.parametrize("case", [0, 2, 4, 5])
@pytest.mark.parametrize("T,E,H,k,dt", [(1, 96, 2048, 8, torch.bfloat16), (16, 96, 2048, 8, torch.bfloat16),
                                        (300, 128, 4096, 8, torch.bfloat16), (33, 64, 1024, 4, torch.float16),
                                        (8, 1024, 512, 16, torch.bfloat16)])
def test_route_gemm(case, T, E, H, k, dt):
    c = CASES[case]
    if c.get("n_group", 1) > 1 and E % c["n_group"]:
        pytest.skip("groups do not divide the experts")
    say(f"route_gemm {c} T={T} E={E} H={H} k={k} {dt}")
    o, bias = _opts(c, E, case)
    g = torch.Generator().manual_seed(T * 7 + E)
    x = torch.randn(T, H, generator=g).to(dt)
    wr = (torch.randn(E, H, generator=g) * H ** -0.5).to(dt)
    w, ids, logits = hm.route(x.to(DEV), wr.to(DEV), k, correction_bias=None if bias is None else torch.from_numpy(bias), **o)
    lg = logits.cpu().numpy()
    want = O.router_logits(x.float().numpy(), wr.float().numpy(), "bf16" if dt == torch.bfloat16 else "f16")
    ulp = np.abs(want) * (2.0 ** -7 if dt == torch.bfloat16 else 2.0 ** -10) + 1e-30
    assert (np.abs(lg - want) <= ulp).all(), np.abs(lg - want).max()
    assert (lg == want).mean() > 0.98
    w_ref, ids_ref = _oracle(lg, k, o, bias)                      # the choice on the kernel's own logits
    assert np.array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=2e-6, atol=1e-12)


def test_route_gemm_graph_replays():
    """Captured with the layer after it (as a decode step), replayed with eager calls of other
    sizes between: the tile counters are left at zero, every replay equals the eager result."""
    say("route_gemm graph replays")
    E, H, I, k, T = 32, 512, 256, 4, 16
    parts = [O.random_parts(E, o, i, 4, seed=60 + q, block=32) for q, (o, i) in enumerate(((I, H), (I, H), (H, I)))]
    dp = lambda p: {"idx": torch.from_numpy(p["idx"].view(np.int32)).to(DEV), "block_scale": torch.from_numpy(p["block_scale"]).to(DEV),  # noqa: E731
                    "expert_scale": torch.from_numpy(p["expert_scale"]).to(DEV), "levels": torch.from_numpy(p["levels"]).to(DEV)}
    tier = hm.HexTier(4, torch.arange(E, dtype=torch.int32), *[dp(p) for p in parts]).prepare(E)
    ref = [{"bits": 4, "experts": np.arange(E), "gate_proj": parts[0], "up_proj": parts[1], "down_proj": parts[2]}]
    g = torch.Generator().manual_seed(3)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV)
    wr = (torch.randn(E, H, generator=g) * H ** -0.5).to(torch.bfloat16).to(DEV)
    bias = (torch.randn(E, generator=g) * 0.3).to(DEV)             # a device parameter, as in vLLM
    opts = dict(correction_bias=bias, routed_scaling_factor=1.5)
    eager = hm.moe_layer(x, wr, [tier], k, **opts)
    w, ids, lg = hm.route(x, wr, k, **opts)
    want = O.moe_reference(x.float().cpu().numpy(), w.cpu().numpy(), ids.cpu().numpy(), ref, "bf16")
    assert O.rel_err(eager.float().cpu().numpy(), want) < 1e-2
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        hm.moe_layer(x, wr, [tier], k, **opts)
    torch.cuda.current_stream().wait_stream(s)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        out = hm.moe_layer(x, wr, [tier], k, **opts)
    for i in range(3):
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        hm.route(torch.randn(40 + i, H, device=DEV).to(torch.bfloat16), wr, k, **opts)   # other sizes between
        torch.cuda.synchronize()


def test_route_argument_checks():
    say("route argument checks")
    lg = torch.randn(4, 96, device=DEV)
    with pytest.raises(ValueError, match="n_group"):
        hm.route_select(lg, 8, "sigmoid", n_group=5)
    with pytest.raises(ValueError, match="topk_group"):
        hm.route_select(lg, 8, "sigmoid", n_group=8, topk_group=9)
    with pytest.raises(ValueError, match="kept groups"):
        hm.route_select(lg, 8, "sigmoid", n_group=32, topk_group=1)
    with pytest.raises(ValueError, match="correction_bias"):
        hm.route_select(lg, 8, correction_bias=torch.zeros(95))
    g = torch.cuda.CUDAGraph()
    with pytest.raises(ValueError, match="on the GPU when the routing is captured"):
        with torch.cuda.graph(g):
            hm.route_select(lg, 8, correction_bias=torch.zeros(96))
    with pytest.raises(NotImplementedError, match="multiple of 32"):
        hm.route(torch.zeros(2, 48, dtype=torch.bfloat16, device=DEV), torch.zeros(96, 48, dtype=torch.bfloat16, device=DEV), 8)
