"""HIP kernels against the CPU oracle on the same seeded inputs (called through the C ABI).

Bit-exact: dequant (each association order, every output dtype, every fp8 code), align, direct,
routing ids. Tolerance: routing weights (2 ulp), layer outputs (max|got - ref| / max|ref| <= 1e-2
with bf16/f16 activations, the north-star bound; 1e-4 for float32 activations on the dequant
path, the reference's own bound at runtime/tests/test_hex_moe.py:81)."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from blackhole_runtime import hex_moe as hm
from oracle import hex_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL_16 = 1e-2


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def dev_parts(p: dict) -> dict:
    return {"idx": torch.from_numpy(np.ascontiguousarray(p["idx"]).view(np.int32)).to(DEV),
            "block_scale": torch.from_numpy(np.ascontiguousarray(p["block_scale"])).to(DEV),
            "expert_scale": torch.from_numpy(np.ascontiguousarray(p["expert_scale"], np.float32)).to(DEV),
            "levels": torch.from_numpy(np.ascontiguousarray(p["levels"], np.float32)).to(DEV)}


def make_layer(E, H, I, split, bits=(4, 3), seed=0, block=32, quantized=False):
    """(oracle tiers with numpy parts, prepared HexTiers on the GPU)."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(E)
    groups = [perm[:split], perm[split:]] if split else [perm]
    ref, tiers = [], []
    for j, (ids, b) in enumerate(zip(groups, bits)):
        n = len(ids)
        if n == 0:
            continue
        parts = {}
        for q, (proj, (o, i)) in enumerate((("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I)))):
            if quantized:
                W = (np.random.default_rng(seed * 100 + 10 * j + q).standard_normal((n, o, i)) * 0.02).astype(np.float32)
                parts[proj] = O.quantize_stack(W, 1 << b, block)
            else:
                parts[proj] = O.random_parts(n, o, i, b, seed=seed * 100 + 10 * j + q, block=block)
        ref.append({"bits": b, "experts": ids, **parts})
        tiers.append(hm.HexTier(b, torch.from_numpy(ids.astype(np.int32)),
                                *[dev_parts(parts[p]) for p in ("gate_proj", "up_proj", "down_proj")]).prepare(E))
    return ref, tiers


def routing(T, E, k, seed=0, skew=False):
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    if skew:
        p = 1.0 / np.arange(1, E + 1) ** 1.1
        logits = logits + np.log(p / p.sum())[rng.permutation(E)].astype(np.float32)
    w, ids = O.route_topk(logits, k)
    return w, ids


# --------------------------------------------------------------------------- dequant


@pytest.mark.parametrize("bits", [3, 4])
@pytest.mark.parametrize("block", [32, 128])
@pytest.mark.parametrize("order", ["R", "D", "T"])
def test_dequant_bit_exact(bits, block, order):
    say(f"dequant bits={bits} block={block} order={order}")
    p = O.random_parts(3, 40, 256, bits, seed=bits * 7 + block, block=block)
    # every fp8 code, including subnormals, zero and +-480
    p["block_scale"] = (np.arange(p["block_scale"].size) % 256).astype(np.uint8).reshape(p["block_scale"].shape)
    want = O.dequant(p["idx"], p["block_scale"], p["expert_scale"], p["levels"], bits, order)
    d = dev_parts(p)
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        got = hm.hex_dequant(d["idx"], d["block_scale"], d["expert_scale"], d["levels"], bits, order, dt).cpu()
        exp = torch.from_numpy(want).to(dt)
        assert torch.equal(got.view(torch.int16 if dt != torch.float32 else torch.int32),
                           exp.view(torch.int16 if dt != torch.float32 else torch.int32)), dt


def test_dequant_all_places_experts():
    say("dequant_all placement")
    ref, tiers = make_layer(7, 64, 32, 3, seed=9)
    w13, w2 = hm.dequant_all(tiers, torch.float32)
    w13, w2 = w13.cpu().numpy(), w2.cpu().numpy()
    for t in ref:
        for local, e in enumerate(t["experts"].tolist()):
            for proj, got in (("gate_proj", w13[e, :32]), ("up_proj", w13[e, 32:]), ("down_proj", w2[e])):
                q = t[proj]
                want = O.dequant(q["idx"][local:local + 1], q["block_scale"][local:local + 1],
                                 q["expert_scale"][local:local + 1], q["levels"][local:local + 1], t["bits"], "D")[0]
                assert np.array_equal(got, want), (e, proj)


# --------------------------------------------------------------------------- routing and plans


@pytest.mark.parametrize("S,n,bm,skew,idt", [(0, 8, 16, False, torch.int64), (1, 96, 16, False, torch.int64),
                                             (8, 4, 4, False, torch.int32), (37, 5, 4, False, torch.int64),
                                             (128, 96, 16, False, torch.int64), (512, 96, 16, False, torch.int32),
                                             (2048, 96, 32, True, torch.int64), (3000, 1000, 16, False, torch.int64),
                                             (32768, 96, 64, False, torch.int64), (40000, 128, 16, True, torch.int32),
                                             (4096, 96, 128, False, torch.int64), (4097, 96, 128, True, torch.int64),
                                             (33000, 96, 128, True, torch.int32), (20000, 1000, 128, True, torch.int64),
                                             (65536, 128, 128, False, torch.int64)])
def test_align_bit_exact(S, n, bm, skew, idt):
    say(f"align S={S} n={n} bm={bm} skew={skew} {idt}")
    rng = np.random.default_rng(S + n + bm)
    p = None
    if skew:
        p = 1.0 / np.arange(1, n + 1) ** 1.1
        p /= p.sum()
    ids = rng.choice(n, S, p=p) if S else np.zeros(0, np.int64)
    want = O.align(ids, n, bm)
    # above 4096 slots: counted per chunk into a workspace, and without one
    for chunked in ((True, False) if S > 4096 else (True,)):
        got = hm.align(torch.from_numpy(ids).to(idt).to(DEV), n, bm, _chunked=chunked)
        for g, w in zip(got, want):
            assert np.array_equal(g.cpu().numpy(), w), chunked


@pytest.mark.parametrize("S,n,bm", [(128, 96, 16), (2048, 96, 32), (9000, 96, 128), (40000, 128, 64), (50, 8, 16)])
def test_align_tier_bit_exact(S, n, bm):
    """A tier's plan places only the slots of experts it holds: the oracle's align of that subset
    of slots, its positions mapped back to the original slot numbers, padded to the full plan's
    length (S as padding, -1 past the last block). Both align paths (one workgroup up to 4096
    slots, plan + placement above)."""
    say(f"align_tier S={S} n={n} bm={bm}")
    rng = np.random.default_rng(S + bm)
    ids = rng.integers(0, n, S)
    lookup = np.full(n, -1, np.int32)
    held = rng.permutation(n)[: n // 2]
    lookup[held] = np.arange(held.size)
    sub = np.nonzero(lookup[ids] >= 0)[0]
    s_sub, e_sub, npp_sub = O.align(ids[sub], n, bm)
    mb = -(-S // bm) + min(n, S)
    want_sid = np.full(mb * bm, S, np.int32)
    want_sid[: s_sub.size] = np.where(s_sub < sub.size, sub[np.minimum(s_sub, max(sub.size - 1, 0))], S)
    want_eid = np.full(mb, -1, np.int32)
    want_eid[: e_sub.size] = e_sub
    for chunked in ((True, False) if S > 4096 else (True,)):
        sid, eid, npp = hm.align(torch.from_numpy(ids).to(DEV), n, bm, torch.from_numpy(lookup).to(DEV), chunked)
        assert np.array_equal(sid.cpu().numpy(), want_sid), chunked
        assert np.array_equal(eid.cpu().numpy(), want_eid), chunked
        assert npp.item() == int(npp_sub[0]), chunked


def test_align_reference_example():
    say("align reference example")
    ids = torch.tensor([2, 0, 0, 2, 2, 1, 3, 0], device=DEV)
    sid, eid, npp = hm.align(ids, 4, 4)
    assert sid.tolist() == [1, 2, 7, 8, 5, 8, 8, 8, 0, 3, 4, 8, 6, 8, 8, 8] + [8] * 8
    assert eid.tolist() == [0, 1, 2, 3, -1, -1] and npp.tolist() == [16]


@pytest.mark.parametrize("S,bm", [(1, 16), (8, 16), (32, 16), (5, 4)])
def test_direct_bit_exact(S, bm):
    say(f"direct S={S} bm={bm}")
    ids = np.random.default_rng(S).integers(0, 96, S)
    got = hm.direct(torch.from_numpy(ids).to(DEV), bm)
    for g, w in zip(got, O.direct(ids, bm)):
        assert np.array_equal(g.cpu().numpy(), w)


@pytest.mark.parametrize("T,E,k,dt", [(1, 8, 2, torch.float32), (16, 96, 8, torch.float32),
                                      (300, 128, 8, torch.bfloat16), (7, 1000, 4, torch.float32),
                                      (4, 7, 7, torch.float16)])
def test_route_topk(T, E, k, dt):
    say(f"route_topk T={T} E={E} k={k} {dt}")
    g = torch.Generator().manual_seed(T + E)
    logits = torch.randn(T, E, generator=g).to(dt)
    w_ref, i_ref = O.route_topk(logits.float().numpy(), k)
    w, ids = hm.route_topk(logits.to(DEV), k)
    assert np.array_equal(ids.cpu().numpy(), i_ref)
    np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=5e-7, atol=0)
    w2, ids2 = hm.route_topk(logits.to(DEV), k, renormalize=False, ids_dtype=torch.int32)
    assert np.array_equal(ids2.cpu().numpy(), i_ref)
    p = torch.softmax(logits.float(), -1).gather(1, torch.from_numpy(i_ref)).numpy()
    np.testing.assert_allclose(w2.cpu().numpy(), p, rtol=5e-7, atol=1e-12)


# --------------------------------------------------------------------------- the fused layer


def run_fused(ref, tiers, T, E, k, H, dt=torch.bfloat16, seed=1, config=None, align_mode="auto", skew=False,
              path="fused"):
    w, ids = routing(T, E, k, seed=seed, skew=skew)
    x = torch.from_numpy(np.random.default_rng(seed + 1).standard_normal((T, H)).astype(np.float32)).to(dt)
    act_round = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: None}[dt]
    want = O.moe_reference(x.float().numpy(), w, ids, ref, act_round)
    xd, wd, idd = x.to(DEV), torch.from_numpy(w).to(DEV), torch.from_numpy(ids).to(DEV)
    if path == "fused":
        got = hm.hex_moe_fused(xd, wd, idd, tiers, config, align_mode)
    else:
        got = hm.hex_moe(xd, wd, idd, tiers, config, path)
    assert got.dtype == dt and got.shape == (T, H)
    return O.rel_err(got.float().cpu().numpy(), want)


@pytest.mark.parametrize("T,split,bits", [(1, 0, (3,)), (3, 5, (4, 3)), (40, 4, (4, 3)), (4, 0, (4,)),
                                          (16, 6, (4, 3)), (64, 0, (4,))])
def test_reference_suite_shapes(T, split, bits):
    """runtime/tests/test_hex_moe.py:64-81's shapes (E=12, H=128, I=64, k=4) in bf16 through the
    fused kernels with both plans; float32 through the dequant path at the reference's 1e-4."""
    say(f"reference shapes T={T} split={split} bits={bits}")
    E, H, I, k = 12, 128, 64, 4
    ref, tiers = make_layer(E, H, I, split, bits, seed=T)
    for mode in ("auto", "direct", "torch"):
        err = run_fused(ref, tiers, T, E, k, H, seed=T, align_mode=mode)
        assert err < TOL_16, (mode, err)
    small = {"BLOCK_M": 16, "BLOCK_N": 32, "BLOCK_K": 32, "num_warps": 4, "num_stages": 1}
    assert run_fused(ref, tiers, T, E, k, H, seed=T, config=small) < TOL_16
    assert run_fused(ref, tiers, T, E, k, H, dt=torch.float32, seed=T, path="dequant") < 1e-4
    assert run_fused(ref, tiers, T, E, k, H, dt=torch.float32, seed=T, path="auto") < 1e-4


@pytest.mark.parametrize("bm", [16, 32, 64, 128])
@pytest.mark.parametrize("block", [32, 128])
def test_tiles(bm, block):
    say(f"tiles bm={bm} block={block}")
    E, H, I, k = 16, 256, 128, 4
    ref, tiers = make_layer(E, H, I, 8, (4, 3), seed=bm, block=block)
    cfg = {"BLOCK_M": bm}
    for T in (1, 24, 70):
        err = run_fused(ref, tiers, T, E, k, H, seed=T, config=cfg)
        assert err < TOL_16, (T, err)


@pytest.mark.parametrize("T", [1, 3, 16, 40])
def test_items_split_between_workgroups(T):
    """Wide inputs and few blocks: each (block, row tile) item's 128-input steps are spread over
    several workgroups, which exchange partial sums (gate/up over 2048 inputs in 16 steps, down
    over 1024 in 8); twice in a row, so the arrival counters must have been left at zero."""
    say(f"split items T={T}")
    E, H, I, k = 8, 2048, 1024, 2
    ref, tiers = make_layer(E, H, I, 0, (4,), seed=11, block=128)
    for _ in range(2):
        assert run_fused(ref, tiers, T, E, k, H, seed=T) < TOL_16


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("block", [32, 128])
def test_prefill_kernels(dt, block):
    """The 128-slot prefill kernels at batches where each expert fills several blocks (plus a
    partly filled one): two tiers (4 and 3 bits), down outputs (384) not a multiple of the
    256-row tile, Zipf-skewed routing; twice in a row."""
    say(f"prefill kernels {dt} block={block}")
    E, H, I, k = 8, 384, 256, 2
    ref, tiers = make_layer(E, H, I, 3, (4, 3), seed=31, block=block)
    for T, skew in ((600, False), (700, True), (600, False)):
        err = run_fused(ref, tiers, T, E, k, H, dt=dt, seed=T, config={"BLOCK_M": 128}, skew=skew)
        assert err < TOL_16, (T, err)
    # and chosen by default at that batch (more than 64 slots per expert)
    assert hm.default_config(1200, I, H, True, E)["BLOCK_M"] == 128


@pytest.mark.parametrize("bits", [3, 4])
def test_prefill_scale_extremes(bits):
    """The 128-slot kernels with one scale per 128 inputs keep each accumulator in units of the
    current block's scale. Zero scales (in a row's first block, its last block, or every
    block), the smallest subnormal scale (0x01) next to the largest (0x7E = 448), and 0x7F
    (480) must all give the oracle's layer. (bf16 only: with 448 and 480 scales the intermediate
    activations pass f16's 65504, and the float32 oracle's f16 rounding of them overflows too.)"""
    say(f"prefill scale extremes bits={bits}")
    E, H, I, k = 4, 512, 256, 2
    ref, tiers = make_layer(E, H, I, 0, (bits,), seed=41, block=128)
    for t_ref, t in zip(ref, tiers):
        for proj in ("gate_proj", "up_proj", "down_proj"):
            bs = t_ref[proj]["block_scale"]            # [n, out, in / 128]
            nb = bs.shape[2]
            bs[:, 0::5, 0] = 0x00                      # first block zero
            bs[:, 1::5, nb - 1] = 0x80                 # last block -0
            bs[:, 2::13, :] = 0x00                     # the whole row zero
            bs[:, 3::5, 0::2] = 0x01                   # 2^-9 next to 448
            bs[:, 3::5, 1::2] = 0x7E
            bs[:, 4::7, nb // 2] = 0x7F
            getattr(t, proj)["block_scale"].copy_(torch.from_numpy(bs))
    for T in (300, 129):
        err = run_fused(ref, tiers, T, E, k, H, seed=T, config={"BLOCK_M": 128})
        assert err < TOL_16, (T, err)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bits", [3, 4])
def test_quantized_layer(dt, bits):
    """Weights from the HEX quantizer (N(0, 0.02)), as the benchmark configs are built."""
    say(f"quantized layer {dt} bits={bits}")
    E, H, I, k = 8, 256, 128, 2
    ref, tiers = make_layer(E, H, I, 0, (bits,), seed=3, quantized=True)
    for T in (1, 16):
        assert run_fused(ref, tiers, T, E, k, H, dt=dt, seed=T) < TOL_16


def test_skewed_routing_and_odd_widths():
    """Zipf-skewed routing (hot experts over several blocks); widths 160 and 96, not multiples of
    the 128-input step or the 64-row tile."""
    say("skewed routing, odd widths")
    E, H, I, k = 10, 160, 96, 3
    ref, tiers = make_layer(E, H, I, 5, (4, 3), seed=21)
    for T, cfg in ((200, None), (200, {"BLOCK_M": 64}), (33, {"BLOCK_M": 32}), (33, {"BLOCK_M": 16})):
        assert run_fused(ref, tiers, T, E, k, H, seed=T, config=cfg, skew=True) < TOL_16


def test_fp8_special_codes_in_fused_path():
    """Scale codes 0x7F / 0xFF decode to +-480 (the reference formula) in the fused kernels too."""
    say("fp8 0x7F in fused path")
    E, H, I, k = 4, 128, 64, 2
    ref, tiers = make_layer(E, H, I, 0, (4,), seed=5)
    for t_ref, t in zip(ref, tiers):
        for proj in ("gate_proj", "up_proj", "down_proj"):
            bs = t_ref[proj]["block_scale"]
            bs.reshape(-1)[::7] = 0x7F
            bs.reshape(-1)[3::11] = 0xFF
            getattr(t, proj)["block_scale"].copy_(torch.from_numpy(bs))
    assert run_fused(ref, tiers, 3, E, k, H, seed=2) < TOL_16


def _exact_layer(E, H, I, bits):
    """Parts whose dequantized weights, activations and all partial sums are exact in float32:
    levels k/8, power-of-two block scales, unit expert scales."""
    rng = np.random.default_rng(bits)
    L = 1 << bits
    parts = {}
    for proj, (o, i) in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
        parts[proj] = {"idx": O.pack(rng.integers(0, L, (E, o, i)), bits),
                       "block_scale": rng.choice(np.array([0x30, 0x38, 0x40], np.uint8), (E, o, i // 32)),
                       "expert_scale": np.ones(E, np.float32),
                       "levels": ((np.arange(L) - L // 2) / 8.0).astype(np.float32)[None].repeat(E, 0)}
    return parts


@pytest.mark.parametrize("bits", [3, 4])
def test_down_kernel_exact(bits):
    """With exactly representable operands the down kernel's y must equal the float64 sum bit
    for bit: pins the code -> input mapping, the block -> scale mapping and the slot rows."""
    say(f"down exact bits={bits}")
    E, H, I, k, T = 6, 64, 128, 2, 5
    parts = _exact_layer(E, H, I, bits)
    tier = hm.HexTier(bits, torch.arange(E, dtype=torch.int32),
                      *[dev_parts(parts[p]) for p in ("gate_proj", "up_proj", "down_proj")]).prepare(E)
    rng = np.random.default_rng(7)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    S = T * k
    act = rng.integers(-4, 5, (S, I)).astype(np.float32)
    tw = np.full(S, 0.5, np.float32)
    Wd = O.dequant(parts["down_proj"]["idx"], parts["down_proj"]["block_scale"], parts["down_proj"]["expert_scale"],
                   parts["down_proj"]["levels"], bits, "R").astype(np.float64)
    want = np.stack([Wd[ids.reshape(-1)[s]] @ act[s].astype(np.float64) * 0.5 for s in range(S)])
    for bm in (16, 32, 64, 128):
        sid, eid, npp = hm.plan(torch.from_numpy(ids).to(DEV).reshape(-1), E, bm, "torch")
        y = torch.full((S, H), float("nan"), device=DEV)
        hm._launch_down(torch.from_numpy(act).to(torch.bfloat16).to(DEV), y, tier, sid, eid, npp, S,
                        torch.from_numpy(tw).to(DEV), bm)
        assert np.array_equal(y.cpu().numpy(), want.astype(np.float32)), bm
        # y in the activation dtype: the same float32 value, rounded once (to nearest even)
        y16 = torch.full((S, H), float("nan"), dtype=torch.bfloat16, device=DEV)
        hm._launch_down(torch.from_numpy(act).to(torch.bfloat16).to(DEV), y16, tier, sid, eid, npp, S,
                        torch.from_numpy(tw).to(DEV), bm)
        assert torch.equal(y16.cpu(), torch.from_numpy(want.astype(np.float32)).to(torch.bfloat16)), bm


@pytest.mark.parametrize("T", [3, 9, 24])
def test_repeated_experts_within_a_token(T, monkeypatch):
    """Routing ids that repeat an expert within a token (the reference's align takes any ids): one
    expert can then hold more slots than tokens (up to T * k), so its run spans several 16-slot
    blocks. Through the matrix-vector launches and through the expert-block kernels (both plans),
    against the oracle, which sums every slot."""
    say(f"repeated experts T={T}")
    E, H, I, k = 8, 256, 128, 4
    ref, tiers = make_layer(E, H, I, 0, (4,), seed=31)
    rng = np.random.default_rng(T)
    ids = np.where(rng.random((T, k)) < 0.6, 2, rng.integers(0, E, (T, k))).astype(np.int64)
    ids[:, 0] = 5                                    # expert 5 once per token, expert 2 often repeated
    w = rng.random((T, k)).astype(np.float32)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16)
    want = O.moe_reference(x.float().numpy(), w, ids, ref, "bf16")
    xd, wd, idd = x.to(DEV), torch.from_numpy(w).to(DEV), torch.from_numpy(ids).to(DEV)
    assert T < 24 or (ids == 2).sum() > 32            # (T = 24: expert 2 spans three blocks)
    gemv = hm.hex_moe_gemv(xd, wd, idd, tiers[0])
    assert O.rel_err(gemv.float().cpu().numpy(), want) < TOL_16
    monkeypatch.setattr(hm, "GEMV_MAX", 0)
    for mode in ("auto", "vllm"):
        got = hm.hex_moe_fused(xd, wd, idd, tiers, {"BLOCK_M": 16}, mode)
        assert O.rel_err(got.float().cpu().numpy(), want) < TOL_16, mode
    got = hm.hex_moe_fused(xd, wd, idd, tiers)
    assert O.rel_err(got.float().cpu().numpy(), want) < TOL_16


def test_uncovered_experts_contribute_nothing():
    say("uncovered experts")
    E, H, I, k = 8, 64, 32, 2
    ref, tiers = make_layer(E, H, I, 3, (4, 3), seed=4)
    ref, tiers = ref[:1], tiers[:1]          # experts of the second tier have no weights
    assert run_fused(ref, tiers, 9, E, k, H, seed=3) < TOL_16


def test_width_mismatch_and_dtype_errors():
    say("errors")
    E, H, I, k = 4, 64, 32, 2
    _, tiers = make_layer(E, H, I, 0, (4,), seed=1)
    x = torch.zeros(2, 96, dtype=torch.bfloat16, device=DEV)
    w = torch.full((2, k), 0.5, device=DEV)
    ids = torch.zeros(2, k, dtype=torch.long, device=DEV)
    with pytest.raises(AssertionError, match="input width"):
        hm.hex_moe_fused(x, w, ids, tiers)
    with pytest.raises(NotImplementedError, match="bf16 or f16"):
        hm.hex_moe_fused(torch.zeros(2, H, device=DEV), w, ids, tiers)


@pytest.mark.parametrize("bm,split", [(None, 8), (128, 8), (128, 0)])
def test_graph_capture_replays_match_eager(bm, split):
    """The fused path captured in a hipGraph: several replays, with eager work between them,
    each equal to the eager result (default tiles, and the 128-slot prefill kernels). Two tiers
    (the second on the side stream), or one tier (with the prefill kernels, its two halves by
    expert on the two streams)."""
    say(f"graph capture bm={bm} split={split}")
    E, H, I, k, T = 16, 256, 128, 4, 8 if bm is None else 300
    cfg = None if bm is None else {"BLOCK_M": bm}
    ref, tiers = make_layer(E, H, I, split, (4, 3), seed=12)
    if bm == 128 and split == 0:
        assert len(tiers) == 1 and tiers[0]._parts and hm.SPLIT > 1
        assert run_fused(ref, tiers, T, E, k, H, seed=5, config=cfg) < TOL_16
    w, ids = routing(T, E, k, seed=5)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16).to(DEV)
    wd, idd = torch.from_numpy(w).to(DEV), torch.from_numpy(ids).to(DEV)
    eager = hm.hex_moe_fused(x, wd, idd, tiers, cfg)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        hm.hex_moe_fused(x, wd, idd, tiers, cfg)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = hm.hex_moe_fused(x, wd, idd, tiers, cfg)
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        _ = hm.hex_moe_fused(x * 2, wd, idd, tiers, cfg)      # unrelated eager work between replays
        torch.cuda.synchronize()


def test_three_tiers_on_three_streams():
    """Three tiers (4, 3 and 4 bits): the second and third run on side streams of their own,
    eager and captured in a hipGraph, decode and prefill tiles."""
    say("three tiers")
    E, H, I, k = 12, 256, 128, 3
    perm = np.random.default_rng(51).permutation(E)
    ref, tiers = [], []
    for j, (ids, b) in enumerate(zip(np.split(perm, 3), (4, 3, 4))):
        parts = {proj: O.random_parts(len(ids), o, i, b, seed=510 + 10 * j + q, block=128)
                 for q, (proj, (o, i)) in enumerate((("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))))}
        ref.append({"bits": b, "experts": ids, **parts})
        tiers.append(hm.HexTier(b, torch.from_numpy(ids.astype(np.int32)),
                                *[dev_parts(parts[p]) for p in ("gate_proj", "up_proj", "down_proj")]).prepare(E))
    for T, cfg in ((20, None), (500, {"BLOCK_M": 128})):
        assert run_fused(ref, tiers, T, E, k, H, seed=T, config=cfg) < TOL_16, T
        w, ids = routing(T, E, k, seed=T)
        x = torch.randn(T, H, generator=torch.Generator().manual_seed(T)).to(torch.bfloat16).to(DEV)
        wd, idd = torch.from_numpy(w).to(DEV), torch.from_numpy(ids).to(DEV)
        eager = hm.hex_moe_fused(x, wd, idd, tiers, cfg)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = hm.hex_moe_fused(x, wd, idd, tiers, cfg)
        for i in range(2):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), (T, i)
            _ = hm.hex_moe_fused(x * 2, wd, idd, tiers, cfg)
            torch.cuda.synchronize()


# --------------------------------------------------------------------------- the kernels' own plan


@pytest.mark.parametrize("bm", [16, 32, 64])
def test_kernel_plan_equals_align_plan(bm):
    """The decode kernels sorting the slots themselves (bh_hex_moe_*_ids) give the outputs of the
    align kernel's plan bit for bit (the same blocks, so the same unit ranges), and match the
    oracle: one tier and two tiers, int32 and int64 ids, ids outside [0, E) and slots of experts
    no tier holds, from 1 slot to the 1024-slot limit with up to 1000 experts."""
    say(f"kernel plan bm={bm}")
    cases = [(40, 256, 256, 4, 13, 1, False), (40, 256, 256, 4, 13, 5, True), (40, 256, 256, 4, 0, 33, False),
             (40, 256, 256, 4, 0, 256, True), (1000, 256, 256, 8, 0, 128, False), (16, 512, 256, 2, 5, 7, True)]
    for E, H, I, k, split, T, skew in cases:
        ref, tiers = make_layer(E, H, I, split, (4, 3), seed=70 + T, block=128)
        w, ids = routing(T, E, k, seed=T, skew=skew)
        ids = ids.copy()
        ids[0, 0] = -1
        if T > 1:
            ids[-1, -1] = E + 3
        if E == 16:                      # a tier that does not hold every expert
            ref, tiers = ref[:1], tiers[:1]
        x = torch.randn(T, H, generator=torch.Generator().manual_seed(T)).to(torch.bfloat16).to(DEV)
        wd = torch.from_numpy(w).to(DEV)
        cfg = {"BLOCK_M": bm}
        want = O.moe_reference(x.float().cpu().numpy(), w, ids, ref, "bf16")
        for idt in (torch.int64, torch.int32):
            idd = torch.from_numpy(ids).to(idt).to(DEV)
            assert hm.KERNEL_PLAN_MAX >= T * k
            own = hm.hex_moe_fused(x, wd, idd, tiers, cfg)
            # align_mode "vllm" takes the align kernel at every batch (auto would take the direct
            # plan up to 32 slots, whose different blocks split items differently)
            aligned = hm.hex_moe_fused(x, wd, idd, tiers, cfg, align_mode="vllm")
            assert torch.equal(own, aligned), (E, T, idt)
            assert O.rel_err(own.float().cpu().numpy(), want) < TOL_16, (E, T, idt)


def test_kernel_plan_limits():
    """More than 1024 slots, or block_m 128, are refused by the _ids entry points (the Python
    layer then launches the align kernel); 1024 slots are taken."""
    say("kernel plan limits")
    E, H, I, k = 8, 256, 128, 8
    ref, tiers = make_layer(E, H, I, 0, (4,), seed=71, block=128)
    t = tiers[0]
    x = torch.zeros(129, H, dtype=torch.bfloat16, device=DEV)
    act = torch.empty(129 * k, I, dtype=torch.bfloat16, device=DEV)
    ids = torch.zeros(129 * k, dtype=torch.long, device=DEV)
    code = 4
    with pytest.raises(NotImplementedError, match="1024 slots"):
        hm._launch_glu_ids(x, act, t, ids, code, 129 * k, k, 16)
    with pytest.raises(NotImplementedError, match="block_m 128"):
        hm._launch_glu_ids(x, act, t, ids[:1024], code, 1024, k, 128)
    hm._launch_glu_ids(x[:128], act[:1024], t, ids[:1024], code, 1024, k, 16)
    torch.cuda.synchronize()
    assert run_fused(ref, tiers, 128, E, k, H, seed=3) < TOL_16       # 1024 slots through the kernels' plan


# --------------------------------------------------------------------------- workspaces


def _ws_key(stream, kind="moe"):
    return (torch.device(DEV).index or 0, stream.cuda_stream, kind)


def test_capture_records_no_fill(monkeypatch):
    """A decode layer captured on a stream that never ran it eagerly: its workspace counters
    come from the zeroed arena, so the capture calls no torch.zeros (no fill kernel replays with
    the layer), and every replay equals the eager result."""
    say("capture records no fill")
    monkeypatch.setattr(hm, "GEMV_MAX", 0)   # the expert-block kernels, whose workspace this is about
    E, H, I, k, T = 16, 512, 256, 4, 24
    ref, tiers = make_layer(E, H, I, 0, (4,), seed=60, block=128)
    w, ids = routing(T, E, k, seed=60)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(60)).to(torch.bfloat16).to(DEV)
    wd, idd = torch.from_numpy(w).to(DEV), torch.from_numpy(ids).to(DEV)
    eager = hm.hex_moe_fused(x, wd, idd, tiers)
    want = O.moe_reference(x.float().cpu().numpy(), w, ids, ref, "bf16")
    assert O.rel_err(eager.float().cpu().numpy(), want) < TOL_16
    torch.cuda.synchronize()

    def no_zeros(*a, **kw):
        raise AssertionError("torch.zeros called while capturing the layer")
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    assert _ws_key(s) not in hm._WORKSPACES
    with torch.cuda.graph(g, stream=s):
        with monkeypatch.context() as m:
            m.setattr(torch, "zeros", no_zeros)
            out = hm.hex_moe_fused(x, wd, idd, tiers)
    assert _ws_key(s) in hm._WORKSPACES
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        _ = hm.hex_moe_fused(x * 2, wd, idd, tiers)
        torch.cuda.synchronize()


def test_workspace_kept_alive_when_it_grows(monkeypatch):
    """Warm-up and capture on one stream, then an eager call on that stream whose workspace must
    grow: the graph's buffers stay allocated (nothing else is given their memory), and replays
    still equal the eager result."""
    say("workspace kept alive when it grows")
    E, H, I, k = 16, 512, 256, 4
    ref, tiers = make_layer(E, H, I, 0, (4,), seed=61, block=128)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())

    def inputs(T, seed):
        w, ids = routing(T, E, k, seed=seed)
        x = torch.randn(T, H, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16).to(DEV)
        return x, torch.from_numpy(w).to(DEV), torch.from_numpy(ids).to(DEV)
    monkeypatch.setattr(hm, "GEMV_MAX", 0)   # the expert-block kernels (their workspaces) at every batch
    xs, ws_, ids_s = inputs(5, 61)          # 20 slots: a small workspace
    xb, wb, idb = inputs(64, 62)            # 256 slots on 32-slot blocks: a larger one
    with torch.cuda.stream(s):
        eager = hm.hex_moe_fused(xs, ws_, ids_s, tiers)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = hm.hex_moe_fused(xs, ws_, ids_s, tiers)
    torch.cuda.synchronize()
    before = [t.data_ptr() for t in hm._WORKSPACES[_ws_key(s)]]
    with torch.cuda.stream(s):
        big = hm.hex_moe_fused(xb, wb, idb, tiers)
    torch.cuda.synchronize()
    after = [t.data_ptr() for t in hm._WORKSPACES[_ws_key(s)]]
    assert after[1] != before[1], "the partials did not grow: the test does not exercise growth"
    kept = {t.data_ptr() for t in hm._RETIRED}
    assert before[1] in kept
    # fresh allocations with other contents: none may take the graph's old workspace
    junk = [torch.full((1 << 20,), 7, dtype=torch.int32, device=DEV) for _ in range(8)]
    _, idsb_np = routing(64, E, k, seed=62)
    want_big = O.moe_reference(xb.float().cpu().numpy(), wb.cpu().numpy(), idsb_np, ref, "bf16")
    assert O.rel_err(big.float().cpu().numpy(), want_big) < TOL_16
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
    del junk
