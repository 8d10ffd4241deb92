"""numpy restatement of the reference's HEX fused-MoE path. TEST INFRASTRUCTURE ONLY.

Imported only by `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py`.

HEX layout, per tier (stacked over the tier's n experts) and per projection W [out, in]
(blackhole/anatomy/hex.py:21-31, runtime/blackhole_runtime/hex_ref.py:5-11):
  idx           uint32 [n, out, in / 32 * bits]  one little-endian bit stream per 32 inputs
  block_scale   uint8  [n, out, in / B]          fp8 e4m3 code per block of B inputs
  expert_scale  float32 [n]
  levels        float32 [n, 2**bits]
  weight[e, o, i] = levels[e, code] * fp8(block_scale[e, o, i // B]) * expert_scale[e]
The reference fixes B = 32 (hex.py:44); here B is read from the shapes (B = in / nblocks), so the
same functions cover B = 128. The index stream does not depend on B.

What pins each function (tests/test_oracle.py):
  fp8_decode        all 256 codes against torch.float8_e4m3fn (every finite code) and the
                    closed form 0x7F/0xFF -> +-480; KATs of tests/test_hex.py:13-19.
  fp8_encode        brute force nearest-value search over the finite table; KATs.
  bf16_round        torch's float32 -> bfloat16 conversion on random and edge values.
  pack_bits /       bit-by-bit pure-Python packing on small cases (every code at every
  unpack_bits       position, the straddling fields of 3-bit), roundtrip, the shapes of
                    tests/test_hex.py:53-57, the words of the torch pack (hex_ref.py:49-61).
  dequant           float64 products checked to round to the float32 results in the named
                    order; KAT of runtime/tests/test_hex_moe.py:36-44 (levels = arange,
                    scale 1.0 -> W == codes); order-R equality with a per-element loop.
  align / direct    invariants of runtime/tests/test_hex_moe.py:47-61 plus an independent
                    pure-Python sequential construction; the reference's worked example.
  route_topk        torch.softmax + torch.topk (an independent implementation).
  route_select      properties that a dropped term or a wrong branch breaks: the softmax branch
                    equals route_topk; sigmoid ids equal softmax ids (both monotone in the
                    logits) without bias or groups; weights are the unbiased scores of the chosen
                    ids and sum to the scaling factor when renormalised; a correction bias that
                    strongly favours k experts selects exactly them; groups: n_group = 1 or
                    topk_group = n_group change nothing, and the kept groups equal a pure-Python
                    brute force over every group's top-2 sum; the reference's toy Kimi gate
                    (reaper/tests/test_pipeline_moe.py:196-211) restated in torch.
  router_logits     float64 products rounded once (a pure-Python dot product on small cases).
  moe_reference     float64 brute force (per-token, per-slot loops) on tiny shapes.
  quantize          golden fixtures written from the reference quantizer in
                    tests/golden/make_golden.py (blackhole.anatomy.hex.quantize).
"""

from __future__ import annotations

import math

import numpy as np

HEX_BLOCK = 32          # inputs per bit stream (hex.py:44, hex_ref.py:21)
FP8_MAX = 448.0         # largest finite e4m3fn value (hex.py:43)


# --------------------------------------------------------------------------- scalar codecs


def fp8_decode(codes) -> np.ndarray:
    """e4m3 codes -> float32 by the kernels' formula (hex_moe.py:42-48; hex.py:199-203;
    hex_ref.py:41-45): ex = (c >> 3) & 15, mt = c & 7; ex == 0 -> mt * 2^-9, else
    (1 + mt / 8) * 2^(ex - 7); negative when bit 7 is set. Codes 0x7F / 0xFF give +-480 (the
    safetensors table of st.py:43 gives NaN there; the quantizer never writes them)."""
    c = np.asarray(codes).astype(np.int64) & 0xFF
    ex = (c >> 3) & 15
    mt = (c & 7).astype(np.float64)
    s = np.where(ex == 0, mt * 2.0 ** -9, (1.0 + mt / 8.0) * np.exp2(ex - 7.0))
    s = np.where((c & 128) != 0, -s, s)
    return s.astype(np.float32)


def fp8_table_st() -> np.ndarray:
    """The 256-entry e4m3fn table of blackhole/anatomy/st.py:35-53 (NaN at 0x7F and 0xFF)."""
    t = fp8_decode(np.arange(256))
    t[0x7F] = np.nan
    t[0xFF] = np.nan
    return t


def fp8_encode(x) -> np.ndarray:
    """float -> e4m3fn code, nearest finite value, ties to the lower value
    (blackhole/anatomy/st.py:74-86, F8_E4M3 branch)."""
    table = fp8_table_st()
    finite = np.where(np.isfinite(table))[0]
    order = finite[np.argsort(table[finite], kind="stable")]
    vals = table[order]
    lim = float(vals[-1])
    xc = np.clip(np.ascontiguousarray(x, dtype=np.float32), -lim, lim)
    i = np.clip(np.searchsorted(vals, xc), 1, len(vals) - 1)
    pick = np.where(np.abs(vals[i - 1] - xc) <= np.abs(vals[i] - xc), i - 1, i)
    return order[pick].astype(np.uint8)


def bf16_round(x) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), returned as float32 values
    (blackhole/anatomy/st.py:66-71; torch's .to(torch.bfloat16))."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u >> 16) & 1) + 0x7FFF
    out = (((u + r) >> 16) & 0xFFFF).astype(np.uint32)
    out = np.where(np.isnan(x), np.uint32(0x7FC0), out)
    return (out << 16).astype(np.uint32).view(np.float32)


# --------------------------------------------------------------------------- the bit stream


def pack_bits(idx, bits: int, block: int = HEX_BLOCK) -> np.ndarray:
    """[out, in] codes < 2**bits -> uint32 [out, ceil(in / block) * block * bits / 32]: per block
    one little-endian stream, value i at bits i*bits .. i*bits+bits-1 (hex.py:136-150)."""
    idx = np.asarray(idx)
    out, n = idx.shape
    pad = -n % block
    x = np.pad(idx.astype(np.uint64), ((0, 0), (0, pad))).reshape(out, -1, block)
    nwords = block * bits // 32
    words = np.zeros((out, x.shape[1], nwords), np.uint64)
    for i in range(block):
        off = i * bits
        wi, sh = divmod(off, 32)
        words[:, :, wi] |= (x[:, :, i] << np.uint64(sh)) & np.uint64(0xFFFFFFFF)
        if sh + bits > 32:
            words[:, :, wi + 1] |= x[:, :, i] >> np.uint64(32 - sh)
    return words.reshape(out, -1).astype(np.uint32)


def unpack_bits(words, bits: int, n: int, block: int = HEX_BLOCK) -> np.ndarray:
    """Inverse of pack_bits: uint32 [out, nblocks * block * bits / 32] -> uint8 [out, n]
    (hex.py:153-166)."""
    words = np.asarray(words)
    out = words.shape[0]
    nwords = block * bits // 32
    w = words.reshape(out, -1, nwords).astype(np.uint64)
    vals = []
    for i in range(block):
        off = i * bits
        wi, sh = divmod(off, 32)
        v = w[:, :, wi] >> np.uint64(sh)
        if sh + bits > 32:
            v = v | (w[:, :, wi + 1] << np.uint64(32 - sh))
        vals.append(v & np.uint64((1 << bits) - 1))
    return np.stack(vals, -1).reshape(out, -1)[:, :n].astype(np.uint8)


def pack(codes, bits: int) -> np.ndarray:
    """Stacked [..., in] codes (in a multiple of 32) -> [..., in / 32 * bits] uint32
    (runtime/blackhole_runtime/hex_ref.py:49-61)."""
    codes = np.asarray(codes)
    lead, n = codes.shape[:-1], codes.shape[-1]
    flat = codes.reshape(-1, n)
    return pack_bits(flat, bits).reshape(*lead, n // HEX_BLOCK * bits)


def unpack(idx, bits: int) -> np.ndarray:
    """Stacked words [..., out, in / 32 * bits] -> codes uint8 [..., out, in]
    (the unpack of hex.py:185-196)."""
    idx = np.asarray(idx)
    if idx.dtype != np.uint32:
        idx = idx.view(np.uint32)
    lead, nw = idx.shape[:-1], idx.shape[-1]
    n = nw // bits * HEX_BLOCK
    return unpack_bits(idx.reshape(-1, nw), bits, n).reshape(*lead, n)


# --------------------------------------------------------------------------- dequant


def block_size(idx_shape, bs_shape, bits: int) -> int:
    """Scale block size from the tensor shapes: in / nblocks, with in = words / bits * 32."""
    n_in = idx_shape[-1] // bits * HEX_BLOCK
    nblk = bs_shape[-1]
    if nblk == 0 or n_in % nblk:
        raise ValueError(f"block_scale width {nblk} does not divide the input width {n_in}")
    return n_in // nblk


def dequant(idx, block_scale, expert_scale, levels, bits: int, order: str = "R") -> np.ndarray:
    """Weights [n, out, in] float32 from stacked HEX parts, in a named association order:

    "R"  level * (fp8 * es)     torch/numpy source of truth (hex.py:180-204 and hex.py:116-123;
                                hex_ref.py:24-46)
    "D"  (level * fp8) * es     the Triton dequant kernel (hex_moe.py:154-168, 163-164)
    "T"  bf16(level * fp8)      the operand the Triton fused kernel feeds tl.dot, expert scale
                                left for the accumulator (hex_moe.py:105, 140, 144-147)
    Each product is one float32 rounding (numpy float32 arithmetic is IEEE round-to-nearest)."""
    idx = np.asarray(idx)
    bs = np.asarray(block_scale)
    es = np.asarray(expert_scale, np.float32).reshape(-1)
    lv = np.asarray(levels, np.float32)
    n = lv.shape[0]
    B = block_size(idx.shape, bs.shape, bits)
    codes = unpack(idx, bits).astype(np.int64)                       # [n, out, in]
    v = np.take_along_axis(lv.reshape(n, 1, -1), codes.reshape(n, 1, -1), axis=2).reshape(codes.shape)
    f8 = np.repeat(fp8_decode(bs), B, axis=-1)                       # [n, out, in]
    e3 = es.reshape(n, 1, 1)
    if order == "R":
        return v * (f8 * e3)
    if order == "D":
        return (v * f8) * e3
    if order == "T":
        return bf16_round(v * f8)
    raise ValueError(f"unknown dequant order {order!r}")


# --------------------------------------------------------------------------- slot alignment


def align(ids, n: int, block_m: int):
    """Group slots by expert, each expert's run padded to block_m (hex_moe.py:201-222).
    Returns (sorted slot ids int32 [max_blocks * block_m] with S as padding, the expert of each
    block int32 [max_blocks] with -1 past the end, padded length int32 [1])."""
    e = np.asarray(ids).reshape(-1).astype(np.int64)
    S = e.size
    counts = np.bincount(e, minlength=n) if S else np.zeros(n, np.int64)
    nblk = (counts + block_m - 1) // block_m
    max_blocks = -(-S // block_m) + min(n, S)
    blk_end = np.cumsum(nblk)
    start = (blk_end - nblk) * block_m
    order = np.argsort(e, kind="stable")
    se = e[order]
    first = np.cumsum(counts) - counts
    pos = start[se] + np.arange(S) - first[se]
    sorted_ids = np.full(max_blocks * block_m, S, np.int32)
    sorted_ids[pos] = order
    b = np.arange(max_blocks)
    last = int(blk_end[-1]) if n else 0
    expert_ids = np.where(b < last, np.searchsorted(blk_end, b, side="right"), -1).astype(np.int32)
    return sorted_ids, expert_ids, np.array([last * block_m], np.int32)


def direct(ids, block_m: int):
    """One block per slot, no sorting (hex_moe.py:228-237): slot s at row s * block_m, S in
    the other rows; block experts = the ids; padded length S * block_m."""
    e = np.asarray(ids).reshape(-1)
    S = e.size
    s = np.full((S, block_m), S, np.int32)
    s[:, 0] = np.arange(S, dtype=np.int32)
    return s.reshape(-1), e.astype(np.int32), np.array([S * block_m], np.int32)


# --------------------------------------------------------------------------- routing


def route_topk(logits, k: int, renormalize: bool = True):
    """Softmax routing (reaper/reaper_pipeline/moe.py:161-166, softmax branch): probabilities
    of fp32 logits, the k largest in descending order (ties to the lower expert id), divided
    by their sum. Returns (weights float32 [T, k], ids int64 [T, k])."""
    lg = np.asarray(logits, np.float32)
    m = lg.max(-1, keepdims=True)
    ex = np.exp(lg - m)
    p = ex / ex.sum(-1, keepdims=True)
    ids = np.argsort(-p, axis=-1, kind="stable")[:, :k]
    w = np.take_along_axis(p, ids, -1)
    if renormalize:
        w = w / w.sum(-1, keepdims=True)
    return w.astype(np.float32), ids.astype(np.int64)


def _topk_desc(v: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest values of each row, in descending order, ties to the lower index."""
    return np.argsort(-v, axis=-1, kind="stable")[..., :k]


def route_select(logits, k: int, scoring: str = "softmax", renormalize: bool = True, n_group: int = 1,
                 topk_group: int = 0, correction_bias=None, routed_scaling_factor: float = 1.0):
    """Expert choice from router logits [T, E] (reaper/reaper_pipeline/moe.py:141-168,
    route_from_logits), in float32:
      sigmoid branch (taken when a correction bias is given or scoring == "sigmoid"):
        scores = sigmoid(logits); choice = scores + bias; with n_group > 1 each group of E/n_group
        consecutive experts scores the sum of its two largest choices, only the topk_group best
        groups stay (0: all), the others' choices are -inf; ids = the k largest choices, weights =
        their unbiased scores, divided by (their sum + 1e-20) when renormalize;
      softmax branch: probabilities, the k largest, divided by their sum when renormalize;
    then weights * routed_scaling_factor. Ties go to the lower expert / group id.
    Returns (weights float32 [T, k], ids int64 [T, k])."""
    lg = np.asarray(logits, np.float32)
    T, E = lg.shape
    if correction_bias is not None or scoring == "sigmoid":
        scores = (np.float32(1.0) / (np.float32(1.0) + np.exp(-lg))).astype(np.float32)
        choice = scores + np.asarray(correction_bias, np.float32) if correction_bias is not None else scores.copy()
        if n_group > 1:
            G = E // n_group
            grp = np.sort(choice.reshape(T, n_group, G), axis=-1)[..., ::-1]
            gs = (grp[..., 0] + grp[..., 1]).astype(np.float32)
            keep = _topk_desc(gs, topk_group or n_group)
            mask = np.zeros((T, n_group), bool)
            np.put_along_axis(mask, keep, True, axis=-1)
            choice = np.where(np.repeat(mask, G, axis=-1), choice, np.float32(-np.inf))
        ids = _topk_desc(choice, k)
        w = np.take_along_axis(scores, ids, -1)
        if renormalize:
            w = w / (w.sum(-1, keepdims=True, dtype=np.float32) + np.float32(1e-20))
    else:
        m = lg.max(-1, keepdims=True)
        ex = np.exp(lg - m)
        p = (ex / ex.sum(-1, keepdims=True)).astype(np.float32)
        ids = _topk_desc(p, k)
        w = np.take_along_axis(p, ids, -1)
        if renormalize:
            w = w / w.sum(-1, keepdims=True, dtype=np.float32)
    w = (w * np.float32(routed_scaling_factor)).astype(np.float32)
    return w, ids.astype(np.int64)


def router_logits(x, w_router, round_to: str | None = "bf16") -> np.ndarray:
    """Router logits [T, E] = x [T, H] @ w_router [E, H]^T (the model's gate linear, no bias),
    accumulated in float64 and rounded to the activation dtype (round_to "bf16" / "f16" / None for
    float32), as a bf16 gate linear hands them to the routing."""
    acc = np.asarray(x, np.float64) @ np.asarray(w_router, np.float64).T
    if round_to == "bf16":
        return bf16_round(acc.astype(np.float32))
    if round_to == "f16":
        return acc.astype(np.float16).astype(np.float32)
    return acc.astype(np.float32)


# --------------------------------------------------------------------------- the MoE layer


def _silu(a: np.ndarray) -> np.ndarray:
    return a / (np.float32(1.0) + np.exp(-a))


def moe_reference(x, topk_weights, topk_ids, tiers, act_round=None) -> np.ndarray:
    """Routed-expert output [T, H] float32 of a SwiGLU MoE over HEX tiers
    (runtime/blackhole_runtime/hex_ref.py:77-94): per expert, float32 dequant (order R) and
    matmul, silu(a Wg^T) * (a Wu^T), the activation rounded to the model dtype (act_round:
    "bf16", "f16" or None for float32), then (h Wd^T) * topk weight added to the token's row.
    Experts are dequantized one at a time so memory stays bounded at large shapes.
    tiers: [{"bits", "experts" [n], "gate_proj"/"up_proj"/"down_proj": {idx, block_scale,
    expert_scale, levels}}] with numpy arrays."""
    xf = np.asarray(x, np.float32)
    ids = np.asarray(topk_ids)
    tw = np.asarray(topk_weights, np.float32)
    T = ids.shape[0]
    out = np.zeros((T, xf.shape[1]), np.float32)
    for t in tiers:
        bits = int(t["bits"])
        for local, e in enumerate(np.asarray(t["experts"]).reshape(-1).tolist()):
            tok, slot = np.nonzero(ids == e)
            if tok.size == 0:
                continue
            W = {}
            for p in ("gate_proj", "up_proj", "down_proj"):
                q = t[p]
                W[p] = dequant(np.asarray(q["idx"])[local:local + 1], np.asarray(q["block_scale"])[local:local + 1],
                               np.asarray(q["expert_scale"]).reshape(-1)[local:local + 1],
                               np.asarray(q["levels"])[local:local + 1], bits, "R")[0]
            a = xf[tok]
            h = _silu(a @ W["gate_proj"].T) * (a @ W["up_proj"].T)
            if act_round == "bf16":
                h = bf16_round(h)
            elif act_round == "f16":
                h = h.astype(np.float16).astype(np.float32)
            np.add.at(out, tok, (h @ W["down_proj"].T) * tw[tok, slot][:, None])
    return out


def rel_err(got, ref) -> float:
    """max|got - ref| / max|ref| (runtime/tests/test_hex_moe.py:80; hex_check.py:116)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


# --------------------------------------------------------------------------- the quantizer


def block_scales(W, block: int):
    """(expert scale, fp8-rounded dequant block scales [out, nblocks], block-normalised W)
    (blackhole/anatomy/hex.py:60-70). The expert scale stays a Python float, as there; it
    enters float32 arithmetic as float32(es)."""
    W = np.asarray(W, np.float32)
    out, n = W.shape
    pad = -n % block
    x = np.pad(W, ((0, 0), (0, pad))).reshape(out, -1, block)
    amax = np.abs(x).max(-1)
    es = max(float(amax.max()) / FP8_MAX, 1e-30)
    es32 = np.float32(es)
    blk = fp8_table_st()[fp8_encode(np.minimum(amax / es32, np.float32(FP8_MAX)))] * es32
    blk = np.where(blk > 0, blk, np.float32(1.0)).astype(np.float32)
    xn = np.clip(x / blk[..., None], -1, 1).reshape(out, -1)[:, :n]
    return es, blk, xn


def fit_table(xn, L: int, iters: int = 20, sample: int = 1 << 17, seed: int = 0) -> np.ndarray:
    """Unweighted 1-D k-means (Lloyd) on block-normalised values: quantile start, `iters`
    rounds, empty clusters keep their level, L sorted float32 levels (hex.py:73-90, weights
    None). Above `sample` values, a seeded sample of indices is used, as there."""
    x = np.asarray(xn).ravel().astype(np.float32)
    if x.size > sample:
        x = x[np.random.default_rng(seed).integers(0, x.size, sample)]
    w = np.ones_like(x)
    lev = np.quantile(x, np.linspace(0, 1, L + 2)[1:-1]).astype(np.float32)
    for _ in range(iters):
        a = np.searchsorted((lev[1:] + lev[:-1]) / 2, x)
        num = np.bincount(a, weights=x * w, minlength=L)
        den = np.bincount(a, weights=w, minlength=L)
        lev = np.sort(np.where(den > 0, num / np.maximum(den, 1e-30), lev)).astype(np.float32)
    return lev


def nearest(xn, levels) -> np.ndarray:
    """Index of the nearest level (midpoint search) of each block-normalised value (hex.py:93-95)."""
    levels = np.asarray(levels, np.float32)
    return np.searchsorted((levels[1:] + levels[:-1]) / 2, np.clip(xn, -1, 1)).astype(np.uint8)


def quantize(W, L: int = 8, block: int = HEX_BLOCK) -> dict:
    """HEX-quantize one [out, in] matrix with nearest rounding (hex.py:207-227 with energy and
    H both None). Returns {"levels", "expert_scale" (Python float), "block_scale" uint8
    [out, nblocks], "idx" uint8 [out, in]}."""
    W = np.asarray(W, np.float32)
    if W.ndim != 2:
        raise ValueError(f"HEX quantizes 2-D matrices, got shape {W.shape}")
    es, blk, xn = block_scales(W, block)
    levels = fit_table(xn, L)
    idx = nearest(xn, levels)
    codes = fp8_encode(np.minimum(blk / np.float32(es), np.float32(FP8_MAX)))
    return {"levels": levels, "expert_scale": es, "block_scale": codes, "idx": idx}


def quantize_stack(Ws, L: int, block: int = HEX_BLOCK) -> dict:
    """Quantize n matrices [n, out, in] into one tier projection's stacked parts
    (idx uint32 [n, out, in/32*bits], block_scale uint8, expert_scale float32 [n], levels)."""
    bits = int(math.log2(L))
    qs = [quantize(W, L, block) for W in np.asarray(Ws, np.float32)]
    return {"idx": np.stack([pack_bits(q["idx"], bits) for q in qs]),
            "block_scale": np.stack([q["block_scale"] for q in qs]),
            "expert_scale": np.array([q["expert_scale"] for q in qs], np.float32),
            "levels": np.stack([q["levels"] for q in qs])}


def random_parts(n: int, out: int, inp: int, bits: int, seed: int = 0, block: int = HEX_BLOCK) -> dict:
    """Random but well-formed HEX parts for one projection of n experts, distributed as those of
    hex_ref.py:64-74 (uniform codes, fp8 codes 40..69 ~ 0.1..1, expert scale 0.01..0.03, sorted
    uniform levels in [-1, 1]) from a numpy generator (its stream is not the reference's)."""
    g = np.random.default_rng(seed)
    codes = g.integers(0, 2 ** bits, (n, out, inp))
    return {"idx": pack(codes, bits),
            "block_scale": g.integers(40, 70, (n, out, inp // block)).astype(np.uint8),
            "expert_scale": (g.random(n) * 0.02 + 0.01).astype(np.float32),
            "levels": np.sort(g.random((n, 2 ** bits)) * 2 - 1, axis=-1).astype(np.float32)}
