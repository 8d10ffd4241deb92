"""The CPU oracle, pinned: each function against something other than its own formula
(torch's conversions, brute force, bit-by-bit packing, exact float64 arithmetic with explicit
rounding, independent sequential constructions, the reference's own tests and the golden
vectors written from the reference quantizer)."""

from __future__ import annotations

import hashlib
import math
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import hex_oracle as O

GOLDEN = Path(__file__).with_name("golden")


# --------------------------------------------------------------------------- fp8 / bf16


def test_fp8_decode_matches_torch_e4m3fn_and_480():
    codes = np.arange(256, dtype=np.uint8)
    ours = O.fp8_decode(codes)
    theirs = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    finite = np.isfinite(theirs)
    assert finite.sum() == 254
    assert np.array_equal(ours[finite].view(np.uint32), theirs[finite].view(np.uint32))   # incl. -0.0
    assert ours[0x7F] == 480.0 and ours[0xFF] == -480.0      # the kernels' formula, hex_moe.py:42-48


def test_fp8_codec_kats():
    """tests/test_hex.py:13-19 restated."""
    x = np.array([0.0, 1.0, -1.5, 3.14159, 0.0625, 448.0, -0.0078125], np.float32)
    f = O.fp8_table_st()[O.fp8_encode(x)]
    assert np.allclose(f, x, rtol=0.13) and f[0] == 0 and f[-1] == -0.0078125
    assert np.isnan(O.fp8_table_st()[0x7F]) and np.isnan(O.fp8_table_st()[0xFF])


def test_fp8_encode_brute_force():
    rng = np.random.default_rng(0)
    table = O.fp8_table_st()
    finite = [c for c in range(256) if np.isfinite(table[c])]
    vals = sorted({float(table[c]) for c in finite})
    mids = [(a + b) / 2 for a, b in zip(vals[:-1], vals[1:])]
    x = np.concatenate([rng.standard_normal(2000) * 50, rng.standard_normal(500) * 1e-3, np.array(mids),
                        np.array([0.0, -0.0, 448.0, -448.0, 500.0, -1e9, 1e-12, -1e-12])]).astype(np.float32)
    got = O.fp8_encode(x)
    for xi, c in zip(x.tolist(), got.tolist()):
        xc = min(max(xi, -448.0), 448.0)
        best = min(finite, key=lambda k: (abs(float(table[k]) - xc), float(table[k]), k != 0))
        # ties go to the lower value; among equal values (+0 / -0) the one that sorts first
        assert float(table[c]) == float(table[best]), (xi, c, best)


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32),
                        (rng.integers(0, 2 ** 31, 5000, dtype=np.int64).astype(np.uint32)).view(np.float32),
                        # exact ties: low 16 bits 0x8000, both parities of bit 16
                        ((rng.integers(0, 2 ** 15, 2000).astype(np.uint32) << 17) | 0x8000).view(np.float32),
                        ((rng.integers(0, 2 ** 15, 2000).astype(np.uint32) << 17) | 0x18000).view(np.float32)])
    x = x[np.isfinite(x)]
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(O.bf16_round(x).view(np.uint32), want.view(np.uint32))


# --------------------------------------------------------------------------- bit stream


def _pack_bitwise(codes: np.ndarray, bits: int, block: int = 32) -> np.ndarray:
    """Bit-by-bit packing with Python integers: value i of a block at stream bits i*bits..."""
    out, n = codes.shape
    nblk = -(-n // block)
    words = np.zeros((out, nblk * block * bits // 32), np.uint32)
    for o in range(out):
        for b in range(nblk):
            stream = 0
            for i in range(block):
                j = b * block + i
                v = int(codes[o, j]) if j < n else 0
                stream |= v << (i * bits)
            for w in range(block * bits // 32):
                words[o, b * block * bits // 32 + w] = (stream >> (32 * w)) & 0xFFFFFFFF
    return words


@pytest.mark.parametrize("bits", [3, 4])
def test_pack_bits_bitwise_and_roundtrip(bits):
    rng = np.random.default_rng(bits)
    L = 1 << bits
    # every code value at every position of a block, plus random rows and a ragged width
    sweep = np.array([[(c + i) % L for i in range(64)] for c in range(L)], np.uint8)
    rnd = rng.integers(0, L, (7, 96)).astype(np.uint8)
    for codes in (sweep, rnd, rnd[:, :70]):
        w = O.pack_bits(codes, bits)
        assert np.array_equal(w, _pack_bitwise(codes, bits))
        assert np.array_equal(O.unpack_bits(w, bits, codes.shape[1]), codes)


def test_pack_shapes_and_straddle():
    """tests/test_hex.py:53-57: in=70 pads to 96, words (5, 3*bits); 3-bit values 10 and 21
    straddle word boundaries (hex.py:147-149)."""
    rng = np.random.default_rng(7)
    for bits in (3, 4):
        idx = rng.integers(0, 2 ** bits, (5, 70)).astype(np.uint8)
        words = O.pack_bits(idx, bits)
        assert words.dtype == np.uint32 and words.shape == (5, 3 * bits)
        assert np.array_equal(O.unpack_bits(words, bits, 70), idx)
    for j, expect in ((10, [(0, 30, 2), (1, 0, 1)]), (21, [(1, 31, 1), (2, 0, 2)])):
        codes = np.zeros((1, 32), np.uint8)
        codes[0, j] = 7
        w = O.pack_bits(codes, 3)[0]
        for word, shift, nbits in expect:
            assert (int(w[word]) >> shift) & ((1 << nbits) - 1) == (1 << nbits) - 1


def test_stacked_pack_kat():
    """runtime/tests/test_hex_moe.py:36-44: levels = arange, fp8 0x38 = 1.0, es = 1 -> W == codes."""
    rng = np.random.default_rng(0)
    for bits in (3, 4):
        codes = rng.integers(0, 2 ** bits, (2, 5, 64))
        words = O.pack(codes, bits)
        assert words.shape == (2, 5, 64 // 32 * bits)
        lv = np.broadcast_to(np.arange(2 ** bits, dtype=np.float32), (2, 2 ** bits)).copy()
        bs = np.full((2, 5, 2), 0x38, np.uint8)
        for order in ("R", "D", "T"):
            W = O.dequant(words, bs, np.ones(2, np.float32), lv, bits, order)
            assert np.array_equal(W, codes.astype(np.float32))


# --------------------------------------------------------------------------- dequant


def _exact_orders(parts, bits):
    """float64 products (exact for these widths) rounded once to float32 per product."""
    codes = O.unpack(parts["idx"], bits).astype(np.int64)
    n = codes.shape[0]
    lv = parts["levels"].astype(np.float64)
    v = np.take_along_axis(lv.reshape(n, 1, -1), codes.reshape(n, 1, -1), 2).reshape(codes.shape)
    B = codes.shape[-1] // parts["block_scale"].shape[-1]
    f8 = np.repeat(O.fp8_decode(parts["block_scale"]).astype(np.float64), B, -1)
    es = parts["expert_scale"].astype(np.float64).reshape(n, 1, 1)
    r = (v * (f8 * es).astype(np.float32).astype(np.float64)).astype(np.float32)
    d = ((v * f8).astype(np.float32).astype(np.float64) * es).astype(np.float32)
    t = torch.from_numpy((v * f8).astype(np.float32)).to(torch.bfloat16).float().numpy()
    return {"R": r, "D": d, "T": t}


@pytest.mark.parametrize("bits,block", [(4, 32), (3, 32), (4, 128), (3, 128)])
def test_dequant_orders_exact(bits, block):
    parts = O.random_parts(3, 16, 256, bits, seed=bits + block, block=block)
    # every fp8 code, including subnormals and +-480
    parts["block_scale"] = np.arange(parts["block_scale"].size, dtype=np.int64).reshape(
        parts["block_scale"].shape).astype(np.uint8)
    want = _exact_orders(parts, bits)
    got = {o: O.dequant(parts["idx"], parts["block_scale"], parts["expert_scale"], parts["levels"], bits, o)
           for o in "RDT"}
    for o in "RDT":
        assert np.array_equal(got[o].view(np.uint32), want[o].view(np.uint32)), o
    assert not np.array_equal(got["R"], got["D"])    # the orders differ, so the test can tell them apart


def test_dequant_elementwise_loop():
    """Index mapping (expert, row, block, position in the stream) by per-element Python loops."""
    bits, n, out, inp = 3, 2, 3, 64
    parts = O.random_parts(n, out, inp, bits, seed=11)
    W = O.dequant(parts["idx"], parts["block_scale"], parts["expert_scale"], parts["levels"], bits, "R")
    for e in range(n):
        for o in range(out):
            for i in range(inp):
                blk, pos = divmod(i, 32)
                stream = 0
                for w in range(bits):
                    stream |= int(parts["idx"][e, o, blk * bits + w]) << (32 * w)
                code = (stream >> (pos * bits)) & 7
                c = int(parts["block_scale"][e, o, blk])
                ex, mt = (c >> 3) & 15, c & 7
                f8 = (mt / 512.0) if ex == 0 else (1 + mt / 8) * 2.0 ** (ex - 7)
                f8 = -f8 if c & 128 else f8
                want = np.float32(parts["levels"][e, code]) * (np.float32(f8) * np.float32(parts["expert_scale"][e]))
                assert W[e, o, i] == want


# --------------------------------------------------------------------------- slot plans


def test_align_reference_example():
    """runtime/tests/test_hex_moe.py:47-61's input, with its outputs worked out by hand."""
    ids = np.array([2, 0, 0, 2, 2, 1, 3, 0])
    sid, eid, npp = O.align(ids, 4, 4)
    S = 8
    assert sid.tolist() == [1, 2, 7, S, 5, S, S, S, 0, 3, 4, S, 6, S, S, S] + [S] * 8
    assert eid.tolist() == [0, 1, 2, 3, -1, -1] and npp.tolist() == [16]


def _align_sequential(ids, n, bm):
    S = len(ids)
    rows, experts = [], []
    for e in range(n):
        slots = [s for s in range(S) if ids[s] == e]
        nb = -(-len(slots) // bm)
        rows += slots + [S] * (nb * bm - len(slots))
        experts += [e] * nb
    max_blocks = -(-S // bm) + min(n, S)
    npp = len(rows)
    rows += [S] * (max_blocks * bm - len(rows))
    experts += [-1] * (max_blocks - len(experts))
    return rows, experts, npp


@pytest.mark.parametrize("S,n,bm,skew", [(0, 8, 16, 0), (1, 96, 16, 0), (37, 5, 4, 0), (128, 96, 16, 0),
                                         (300, 12, 32, 1), (513, 96, 64, 1), (64, 200, 16, 0)])
def test_align_matches_sequential(S, n, bm, skew):
    rng = np.random.default_rng(S + n)
    p = None
    if skew:
        p = 1.0 / np.arange(1, n + 1) ** 1.1
        p /= p.sum()
    ids = rng.choice(n, S, p=p) if S else np.zeros(0, np.int64)
    sid, eid, npp = O.align(ids, n, bm)
    rows, experts, want_npp = _align_sequential(ids.tolist(), n, bm)
    assert sid.tolist() == rows and eid.tolist() == experts and int(npp[0]) == want_npp
    # the reference test's invariants
    seen = []
    for b, e in enumerate(eid.tolist()):
        if b * bm >= int(npp[0]):
            assert e < 0
            continue
        for r in sid[b * bm:(b + 1) * bm].tolist():
            if r < S:
                assert ids[r] == e
                seen.append(r)
    assert sorted(seen) == list(range(S))


def test_direct_closed_form():
    ids = np.array([5, 1, 1, 0])
    sid, eid, npp = O.direct(ids, 4)
    assert sid.tolist() == [0, 4, 4, 4, 1, 4, 4, 4, 2, 4, 4, 4, 3, 4, 4, 4]
    assert eid.tolist() == [5, 1, 1, 0] and eid.dtype == np.int32 and npp.tolist() == [16]


# --------------------------------------------------------------------------- routing


@pytest.mark.parametrize("T,E,k", [(1, 8, 2), (16, 96, 8), (33, 128, 8), (5, 7, 7)])
def test_route_topk_matches_torch(T, E, k):
    g = torch.Generator().manual_seed(T * E)
    logits = torch.randn(T, E, generator=g)
    w_ref, i_ref = torch.softmax(logits, -1).topk(k, -1)
    w_ref = w_ref / w_ref.sum(-1, keepdim=True)
    w, ids = O.route_topk(logits.numpy(), k)
    assert np.array_equal(ids, i_ref.numpy())
    np.testing.assert_allclose(w, w_ref.numpy(), rtol=2.5e-7 * 4, atol=0)


# --------------------------------------------------------------------------- the layer


def _brute_force(x, tw, ids, tiers, act_round=None):
    """float64 per (token, slot) loops over explicit float64 weights from exact products."""
    T, k = ids.shape
    H = x.shape[1]
    out = np.zeros((T, H))
    for t in tiers:
        Ws = {p: _exact_orders(t[p], t["bits"])["R"].astype(np.float64) for p in ("gate_proj", "up_proj", "down_proj")}
        for local, e in enumerate(t["experts"].tolist()):
            for tok in range(T):
                for s in range(k):
                    if ids[tok, s] != e:
                        continue
                    a = x[tok].astype(np.float64)
                    g = Ws["gate_proj"][local] @ a
                    u = Ws["up_proj"][local] @ a
                    h = g / (1 + np.exp(-g)) * u
                    if act_round == "bf16":
                        h = torch.from_numpy(h.astype(np.float32)).to(torch.bfloat16).double().numpy()
                    out[tok] += (Ws["down_proj"][local] @ h) * float(tw[tok, s])
    return out


def _tiny_layer(E=6, H=64, I=32, split=2, seed=0):
    rng = np.random.default_rng(seed)
    perm = rng.permutation(E)
    tiers = []
    for j, (ids, bits) in enumerate(((perm[:split], 4), (perm[split:], 3))):
        n = len(ids)
        tiers.append({"bits": bits, "experts": ids,
                      "gate_proj": O.random_parts(n, I, H, bits, seed=seed * 10 + 3 * j + 1),
                      "up_proj": O.random_parts(n, I, H, bits, seed=seed * 10 + 3 * j + 2),
                      "down_proj": O.random_parts(n, H, I, bits, seed=seed * 10 + 3 * j + 3)})
    return tiers


@pytest.mark.parametrize("act_round", [None, "bf16"])
def test_moe_reference_brute_force(act_round):
    tiers = _tiny_layer()
    rng = np.random.default_rng(5)
    T, k = 4, 3
    x = rng.standard_normal((T, 64)).astype(np.float32)
    ids = np.stack([rng.permutation(6)[:k] for _ in range(T)])
    tw = rng.random((T, k)).astype(np.float32)
    got = O.moe_reference(x, tw, ids, tiers, act_round)
    want = _brute_force(x, tw, ids, tiers, act_round)
    assert O.rel_err(got, want) < (1e-5 if act_round is None else 1e-2)
    # sensitivity: dropping the top-k weight is caught
    assert O.rel_err(O.moe_reference(x, np.ones_like(tw), ids, tiers, act_round), want) > 0.05


def test_rel_err_definition():
    assert O.rel_err(np.array([1.0, 2.5]), np.array([1.0, 2.0])) == pytest.approx(0.25)


# --------------------------------------------------------------------------- quantizer


def _golden_cases():
    sys.path.insert(0, str(GOLDEN))
    from make_golden import CASES, weights
    return CASES, weights


def test_quantize_matches_reference_golden():
    cases, weights = _golden_cases()
    d = np.load(GOLDEN / "quantize.npz")
    for name, o, i, L, block, seed in cases:
        W = weights(o, i, seed)
        assert hashlib.sha256(W.tobytes()).digest() == d[f"{name}.W_sha256"].tobytes(), name
        q = O.quantize(W, L, block)
        bits = int(np.log2(L))
        assert np.array_equal(q["levels"], d[f"{name}.levels"]), name
        assert q["expert_scale"] == float(d[f"{name}.expert_scale"][0]), name
        assert np.array_equal(q["block_scale"], d[f"{name}.block_scale"]), name
        assert np.array_equal(O.pack_bits(q["idx"], bits), d[f"{name}.idx_words"]), name


def test_quantize_stack_layout():
    rng = np.random.default_rng(2)
    Ws = (rng.standard_normal((3, 16, 128)) * 0.02).astype(np.float32)
    p = O.quantize_stack(Ws, 16, 32)
    assert p["idx"].shape == (3, 16, 16) and p["idx"].dtype == np.uint32
    assert p["block_scale"].shape == (3, 16, 4) and p["levels"].shape == (3, 16)
    W = O.dequant(p["idx"], p["block_scale"], p["expert_scale"], p["levels"], 4, "R")
    assert np.abs(W - Ws).max() < 0.2 * np.abs(Ws).max()


def test_random_parts_ranges():
    p = O.random_parts(4, 8, 64, 3, seed=1)
    assert p["idx"].shape == (4, 8, 6) and p["block_scale"].min() >= 40 and p["block_scale"].max() < 70
    assert np.all(np.diff(p["levels"], axis=-1) >= 0) and np.all(np.abs(p["levels"]) <= 1)
    assert np.all((p["expert_scale"] >= 0.01) & (p["expert_scale"] <= 0.03))


# --------------------------------------------------------------------------- routing from logits


def _logits(T, E, seed):
    return np.random.default_rng(seed).standard_normal((T, E)).astype(np.float32)


def test_route_select_softmax_branch_is_route_topk():
    lg = _logits(32, 96, 1)
    for renorm in (True, False):
        w, ids = O.route_select(lg, 8, renormalize=renorm)
        w2, ids2 = O.route_topk(lg, 8, renorm)
        assert np.array_equal(ids, ids2)
        np.testing.assert_allclose(w, w2, rtol=1e-6)


def test_route_select_sigmoid_properties():
    lg = _logits(64, 96, 2)
    k = 8
    # sigmoid and softmax are both monotone in the logits: the same experts, in the same order
    w, ids = O.route_select(lg, k, "sigmoid", renormalize=False)
    assert np.array_equal(ids, O.route_select(lg, k)[1])
    sig = 1.0 / (1.0 + np.exp(-lg.astype(np.float64)))
    np.testing.assert_allclose(w, np.take_along_axis(sig, ids, -1), rtol=1e-6)
    # renormalised weights sum to the scaling factor
    w, _ = O.route_select(lg, k, "sigmoid", routed_scaling_factor=2.5)
    np.testing.assert_allclose(w.sum(-1), 2.5, rtol=1e-5)
    # a correction bias that strongly favours k experts picks exactly them; the weights stay the
    # unbiased scores of those experts
    fav = np.array([3, 17, 40, 41, 60, 77, 90, 95])
    bias = np.zeros(96, np.float32)
    bias[fav] = 10.0
    w, ids = O.route_select(lg, k, correction_bias=bias, renormalize=False)
    assert all(sorted(r) == sorted(fav.tolist()) for r in ids.tolist())
    np.testing.assert_allclose(w, np.take_along_axis(sig, ids, -1), rtol=1e-6)
    # the bias alone switches to the sigmoid branch (scoring left at "softmax")
    assert np.array_equal(O.route_select(lg, k, correction_bias=np.zeros(96))[1], O.route_select(lg, k, "sigmoid")[1])


def _groups_brute(choice_row, n_group, topk_group, k):
    """Pure-Python group-limited top-k of one token."""
    E = len(choice_row)
    G = E // n_group
    gs = []
    for q in range(n_group):
        vals = sorted((float(v) for v in choice_row[q * G:(q + 1) * G]), reverse=True)
        gs.append((-(np.float32(vals[0]) + np.float32(vals[1])), q))
    kept = {q for _, q in sorted(gs)[:topk_group]}
    cand = sorted((-float(choice_row[e]), e) for e in range(E) if e // G in kept)
    return [e for _, e in cand[:k]]


def test_route_select_groups():
    lg = _logits(40, 64, 3)
    bias = (np.random.default_rng(4).standard_normal(64) * 0.3).astype(np.float32)
    k = 6
    base = O.route_select(lg, k, "sigmoid", correction_bias=bias)
    assert np.array_equal(O.route_select(lg, k, "sigmoid", n_group=1, correction_bias=bias)[1], base[1])
    assert np.array_equal(O.route_select(lg, k, "sigmoid", n_group=8, topk_group=8, correction_bias=bias)[1], base[1])
    for n_group, topk_group in ((8, 3), (4, 2), (16, 5)):
        w, ids = O.route_select(lg, k, "sigmoid", n_group=n_group, topk_group=topk_group, correction_bias=bias)
        choice = (1.0 / (1.0 + np.exp(-lg))).astype(np.float32) + bias
        for t in range(lg.shape[0]):
            assert ids[t].tolist() == _groups_brute(choice[t], n_group, topk_group, k), (n_group, t)


def test_route_select_kimi_toy_gate():
    """The reference test's DeepSeek-V3 style gate (reaper/tests/test_pipeline_moe.py:196-211),
    restated in torch: sigmoid scores, correction bias for the choice only, renormalised and scaled."""
    import torch
    g = torch.Generator().manual_seed(0)
    E, H, k, scale = 6, 16, 2, 2.0
    weight = torch.randn(E, H, generator=g)
    bias = torch.randn(E, generator=g) * 0.3
    x = torch.randn(15, H, generator=g)
    s = torch.nn.functional.linear(x, weight).sigmoid()
    idx = (s + bias).topk(k, dim=-1)[1]
    w = s.gather(1, idx)
    w = w / w.sum(-1, keepdim=True) * scale
    logits = torch.nn.functional.linear(x, weight).numpy()
    w2, ids2 = O.route_select(logits, k, correction_bias=bias.numpy(), routed_scaling_factor=scale)
    assert np.array_equal(ids2, idx.numpy())
    np.testing.assert_allclose(w2, w.numpy(), rtol=2e-6)


def test_router_logits_dot_products():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 40)).astype(np.float32)
    W = rng.standard_normal((5, 40)).astype(np.float32)
    got = O.router_logits(x, W, None)
    for t in range(3):
        for e in range(5):
            acc = math.fsum(float(x[t, i]) * float(W[e, i]) for i in range(40))
            assert got[t, e] == np.float32(acc)
    assert np.array_equal(O.router_logits(x, W, "bf16"), O.bf16_round(got))
