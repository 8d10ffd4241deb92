"""The two matrix-vector launches of a few-token layer (bh_hex_moe_gemv) against the CPU oracle
(runtime/blackhole_runtime/hex_ref.py:77-94 restated) and against the expert-block kernels on
the same inputs.

Layer outputs: max relative error <= 1e-2 against the oracle's float32 layer (the north-star
bound). Against the block kernels the only differences are the float32 summation order and the
roundings of act and out it shifts: <= 4e-3 relative to the largest output. Exact operands
(levels k/8, power-of-two scales, integer activations) pin the code, scale, slot and weight
mappings: the gate/up sums are exact in float32, so act equals the float64 statement rounded to
the activation dtype up to SiLU's last bit, and out equals the float64 down projection of the
device's own act within one unit of the activation dtype."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from blackhole_runtime import _lib
from blackhole_runtime import hex_moe as hm
from oracle import hex_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def dev_parts(p: dict) -> dict:
    return {"idx": torch.from_numpy(np.ascontiguousarray(p["idx"]).view(np.int32)).to(DEV),
            "block_scale": torch.from_numpy(np.ascontiguousarray(p["block_scale"])).to(DEV),
            "expert_scale": torch.from_numpy(np.ascontiguousarray(p["expert_scale"], np.float32)).to(DEV),
            "levels": torch.from_numpy(np.ascontiguousarray(p["levels"], np.float32)).to(DEV)}


def make_tier(E, H, I, bits, block, seed, experts=None):
    experts = np.arange(E) if experts is None else np.asarray(experts)
    n = len(experts)
    parts = {proj: O.random_parts(n, o, i, bits, seed=seed + q, block=block)
             for q, (proj, (o, i)) in enumerate((("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))))}
    ref = {"bits": bits, "experts": experts, **parts}
    tier = hm.HexTier(bits, torch.from_numpy(experts.astype(np.int32)),
                      *[dev_parts(parts[p]) for p in ("gate_proj", "up_proj", "down_proj")]).prepare(E)
    return ref, tier


def inputs(T, E, H, k, dt, seed):
    rng = np.random.default_rng(seed)
    w, ids = O.route_topk(rng.standard_normal((T, E)).astype(np.float32), k)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(dt)
    return x, w, ids


def act_name(dt):
    return {torch.bfloat16: "bf16", torch.float16: "f16"}[dt]


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bits,block", [(4, 128), (3, 128), (4, 32)])
@pytest.mark.parametrize("T", [1, 2, 4, 8, 10])
def test_gemv_config2_widths(T, bits, block, dt):
    """96 experts, hidden 2048, intermediate 768, top-8 (the decode configurations' layer)."""
    say(f"gemv T={T} bits={bits} block={block} {dt}")
    E, H, I, k = 96, 2048, 768, 8
    ref, tier = make_tier(E, H, I, bits, block, seed=bits * 10 + block)
    x, w, ids = inputs(T, E, H, k, dt, seed=T)
    want = O.moe_reference(x.float().numpy(), w, ids, [ref], act_name(dt))
    xd, wd, idd = x.to(DEV), torch.from_numpy(w).to(DEV), torch.from_numpy(ids).to(DEV)
    got = hm.hex_moe_gemv(xd, wd, idd, tier)
    assert got.dtype == dt and got.shape == (T, H)
    g = got.float().cpu().numpy()
    assert O.rel_err(g, want) < 1e-2
    blocks = hm.hex_moe_fused(xd, wd, idd, [tier], {"BLOCK_M": 16}).float().cpu().numpy()
    assert O.rel_err(g, blocks) < 4e-3
    # the dispatcher takes this path for a single tier at these batches
    if hm.gemv_prefer(T, k, H, I, tier):
        assert torch.equal(hm.hex_moe_fused(xd, wd, idd, [tier]), got)


def _exact_parts(E, H, I, bits, block, seed):
    rng = np.random.default_rng(seed)
    L = 1 << bits
    parts = {}
    for proj, (o, i) in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
        parts[proj] = {"idx": O.pack(rng.integers(0, L, (E, o, i)), bits),
                       "block_scale": rng.choice(np.array([0x30, 0x38, 0x40], np.uint8), (E, o, i // block)),
                       "expert_scale": np.ones(E, np.float32),
                       "levels": ((np.arange(L) - L // 2) / 8.0).astype(np.float32)[None].repeat(E, 0)}
    return parts


def _round(a, dt):
    return torch.from_numpy(np.asarray(a, np.float32)).to(dt).float().numpy()


@pytest.mark.parametrize("bits,block", [(4, 32), (3, 128), (4, 128)])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_gemv_exact_operands(bits, block, dt):
    """Pins which code, scale, slot, expert and top-k weight each term takes: act against the
    float64 gate/up + SiLU, out against the float64 down projection and k-slot sum of the device's
    act; ids of int32 and int64 give the same bits."""
    say(f"gemv exact bits={bits} block={block} {dt}")
    E, H, I, k, T = 6, 256, 128, 3, 3
    parts = _exact_parts(E, H, I, bits, block, seed=bits + block)
    tier = hm.HexTier(bits, torch.arange(E, dtype=torch.int32),
                      *[dev_parts(parts[p]) for p in ("gate_proj", "up_proj", "down_proj")]).prepare(E)
    rng = np.random.default_rng(5)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    tw = np.array([[0.5, 0.25, 0.125]] * T, np.float32)
    x = rng.integers(-3, 4, (T, H)).astype(np.float32)
    W = {p: O.dequant(parts[p]["idx"], parts[p]["block_scale"], parts[p]["expert_scale"], parts[p]["levels"], bits,
                      "R").astype(np.float64) for p in parts}
    xd = torch.from_numpy(x).to(dt).to(DEV)
    act = torch.full((T * k, I), float("nan"), dtype=dt, device=DEV)
    out = torch.full((T, H), float("nan"), dtype=dt, device=DEV)
    lib = _lib.load()
    outs = []
    for idt in (torch.int32, torch.int64):
        idd = torch.from_numpy(ids).to(idt).to(DEV).reshape(-1)
        wd = torch.from_numpy(tw).to(DEV).reshape(-1)
        c = _lib.dtype_code(dt)
        _lib.check(lib.bh_hex_moe_gemv(
            xd.data_ptr(), c, H, act.data_ptr(), I, out.data_ptr(), c, H, tier.struct("gate_proj"),
            tier.struct("up_proj"), tier.struct("down_proj"), bits, H, I, idd.data_ptr(), _lib.dtype_code(idt),
            wd.data_ptr(), tier.lookup.data_ptr(), E, T, k, _lib.stream_of(xd)), "bh_hex_moe_gemv")
        torch.cuda.synchronize()
        outs.append(out.clone())
    assert torch.equal(outs[0], outs[1])
    a_dev = act.float().cpu().numpy()
    o_dev = outs[0].float().cpu().numpy()
    flat = ids.reshape(-1)
    g = np.stack([W["gate_proj"][flat[s]] @ x[s // k] for s in range(T * k)])
    u = np.stack([W["up_proj"][flat[s]] @ x[s // k] for s in range(T * k)])
    h = _round(g / (1.0 + np.exp(-g)) * u, dt)
    ulp = 2.0 ** (-8 if dt == torch.bfloat16 else -11)
    assert (np.abs(a_dev - h) <= np.abs(h) * 2 * ulp + 1e-30).all()
    assert (a_dev == h).mean() > 0.99
    o64 = np.zeros((T, H))
    for s in range(T * k):
        o64[s // k] += tw.reshape(-1)[s] * (W["down_proj"][flat[s]] @ a_dev[s].astype(np.float64))
    want = _round(o64, dt)
    assert (np.abs(o_dev - want) <= np.abs(want) * 2 * ulp + 1e-30).all()
    assert (o_dev == want).mean() > 0.95


def test_gemv_invalid_ids_and_partial_tier():
    """Ids -1 and E, and a tier holding only some experts: those slots contribute nothing (as the
    reference's sum over the tiers' experts)."""
    say("gemv invalid ids")
    E, H, I, k, T = 16, 512, 256, 4, 3
    ref, tier = make_tier(E, H, I, 4, 128, seed=3, experts=np.arange(0, E, 2))
    x, w, ids = inputs(T, E, H, k, torch.bfloat16, seed=9)
    ids = ids.copy()
    ids[0, 1] = -1
    ids[1, 3] = E
    ids[2, 0] = E + 7
    want = O.moe_reference(x.float().numpy(), w, ids, [ref], "bf16")
    got = hm.hex_moe_gemv(x.to(DEV), torch.from_numpy(w).to(DEV), torch.from_numpy(ids).to(DEV), tier)
    assert O.rel_err(got.float().cpu().numpy(), want) < 1e-2


def test_gemv_graph_replays():
    """Captured in a hipGraph (no workspace, nothing to clear): replays equal the eager result,
    with eager calls of other sizes between them."""
    say("gemv graph replays")
    E, H, I, k, T = 96, 2048, 768, 8, 2
    _, tier = make_tier(E, H, I, 4, 128, seed=1)
    x, w, ids = inputs(T, E, H, k, torch.bfloat16, seed=4)
    xd, wd, idd = x.to(DEV), torch.from_numpy(w).to(DEV), torch.from_numpy(ids).to(DEV)
    eager = hm.hex_moe_gemv(xd, wd, idd, tier)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        hm.hex_moe_gemv(xd, wd, idd, tier)
    torch.cuda.current_stream().wait_stream(s)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        out = hm.hex_moe_gemv(xd, wd, idd, tier)
    for i in range(3):
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        x2, w2, i2 = inputs(1 + i, E, H, k, torch.bfloat16, seed=20 + i)
        hm.hex_moe_gemv(x2.to(DEV), torch.from_numpy(w2).to(DEV), torch.from_numpy(i2).to(DEV), tier)
        torch.cuda.synchronize()


def test_gemv_limits():
    say("gemv limits")
    E, H, I = 8, 256, 128
    _, tier = make_tier(E, H, I, 4, 32, seed=2)
    x = torch.zeros(1, H, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(NotImplementedError, match="k <= 16"):
        hm.hex_moe_gemv(x, torch.ones(1, 17, device=DEV), torch.zeros(1, 17, dtype=torch.long, device=DEV), tier)
    with pytest.raises(NotImplementedError, match="bf16 or f16"):
        hm.hex_moe_gemv(x.float(), torch.ones(1, 2, device=DEV), torch.zeros(1, 2, dtype=torch.long, device=DEV), tier)
    assert hm.hex_moe_gemv(x[:0], torch.ones(0, 2, device=DEV), torch.zeros(0, 2, dtype=torch.long, device=DEV),
                           tier).shape == (0, H)
    assert not hm.gemv_fits(8, 2048, 4096) and hm.gemv_fits(8, 4096, 1536) and not hm.gemv_fits(8, 4128, 768)
    assert hm.gemv_fits(16, 2048, 2048) and not hm.gemv_fits(8, 2048, 2080)
