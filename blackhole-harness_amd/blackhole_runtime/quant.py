"""HEX quantizer on the GPU (nearest rounding), batched over a stack of expert matrices.

Follows blackhole/anatomy/hex.py's quantize() without an input Hessian (hex.py:207-227):
  expert scale  es = max|W| / 448 (float64, used as float32)
  block scales  fp8 e4m3 of max|w_block| / es (nearest, ties to the lower value; st.py:74-86),
                dequant scale fp8 * es, zero blocks scaled by 1.0
  levels        L sorted levels by 1-D k-means on the block-normalised weights: quantiles as the
                start, 20 Lloyd rounds, empty clusters keep their level, a seeded sample of
                2^17 values when there are more (the same numpy draw as hex.py:78-80)
  indices       nearest level (midpoint search), packed into the HEX bit stream
The k-means sums here are float64 reductions on the GPU and torch's quantile interpolates in
float32, so levels can differ from the numpy quantizer's in the last bits; the benchmark uses
this to build its synthetic layers, the tests compare it with the CPU oracle.
"""

from __future__ import annotations

import numpy as np
import torch

FP8_MAX = 448.0
HEX_BLOCK = 32


def _fp8_values(device) -> torch.Tensor:
    """Decoded value of every e4m3 code by the kernels' formula (0x7F / 0xFF: +-480)."""
    c = torch.arange(256, device=device)
    ex = (c >> 3) & 15
    mt = (c & 7).double()
    s = torch.where(ex == 0, mt * 2.0 ** -9, (1.0 + mt / 8.0) * torch.exp2((ex - 7).double()))
    return torch.where((c & 128) != 0, -s, s).float()


def fp8_encode(x: torch.Tensor) -> torch.Tensor:
    """Nearest finite e4m3fn code, ties to the lower value (st.py:74-86)."""
    vals = _fp8_values(x.device)
    finite = torch.tensor([c for c in range(256) if c not in (0x7F, 0xFF)], device=x.device)
    fv = vals[finite]
    order = finite[torch.sort(fv, stable=True).indices]
    sv = vals[order]
    xc = x.float().clamp(-FP8_MAX, FP8_MAX).contiguous()
    i = torch.searchsorted(sv, xc).clamp(1, sv.numel() - 1)
    lo, hi = sv[i - 1], sv[i]
    pick = torch.where((lo - xc).abs() <= (hi - xc).abs(), i - 1, i)
    return order[pick].to(torch.uint8)


def pack(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """[..., in] codes (in a multiple of 32) -> int32 [..., in / 32 * bits] HEX bit stream
    (value i of a block at bits i*bits .. i*bits+bits-1, little endian)."""
    lead, n = codes.shape[:-1], codes.shape[-1]
    x = codes.to(torch.int64).reshape(*lead, n // HEX_BLOCK, HEX_BLOCK)
    words = torch.zeros(*lead, n // HEX_BLOCK, bits, dtype=torch.int64, device=codes.device)
    for j in range(HEX_BLOCK):
        wi, sh = divmod(j * bits, 32)
        words[..., wi] |= (x[..., j] << sh) & 0xFFFFFFFF
        if sh + bits > 32:
            words[..., wi + 1] |= x[..., j] >> (32 - sh)
    words = torch.where(words >= 2 ** 31, words - 2 ** 32, words)
    return words.to(torch.int32).reshape(*lead, n // HEX_BLOCK * bits)


def fit_tables(xn: torch.Tensor, L: int, iters: int = 20, sample: int = 1 << 17, seed: int = 0) -> torch.Tensor:
    """Per-matrix k-means levels [n, L] (float32, sorted) of block-normalised values xn [n, m]."""
    n, m = xn.shape
    if m > sample:
        idx = torch.from_numpy(np.random.default_rng(seed).integers(0, m, sample)).to(xn.device)
        xs = xn[:, idx]
    else:
        xs = xn
    q = torch.linspace(0, 1, L + 2, dtype=torch.float64, device=xn.device)[1:-1]
    lev = torch.quantile(xs.double(), q, dim=1).T.float().contiguous()          # [n, L]
    x64 = xs.double()
    for _ in range(iters):
        mids = ((lev[:, 1:] + lev[:, :-1]) / 2).contiguous()
        a = torch.searchsorted(mids, xs.contiguous())
        num = torch.zeros(n, L, dtype=torch.float64, device=xn.device).scatter_add_(1, a, x64)
        den = torch.zeros(n, L, dtype=torch.float64, device=xn.device).scatter_add_(1, a, torch.ones_like(x64))
        lev = torch.sort(torch.where(den > 0, num / den.clamp(min=1e-30), lev.double()), dim=1).values.float()
    return lev


def quantize_experts(W: torch.Tensor, L: int = 16, block: int = HEX_BLOCK) -> dict:
    """HEX parts of a stack of matrices W [n, out, in] (in a multiple of `block`, block a multiple
    of 32): {"idx" int32 [n, out, in/32*bits], "block_scale" uint8 [n, out, in/block],
    "expert_scale" float32 [n], "levels" float32 [n, L]}."""
    if W.dim() != 3:
        raise ValueError(f"quantize_experts takes [n, out, in], got {tuple(W.shape)}")
    n, out, inp = W.shape
    if inp % block or block % HEX_BLOCK:
        raise ValueError(f"input width {inp} must be a multiple of the block {block} (a multiple of 32)")
    bits = int(L).bit_length() - 1
    if L != 1 << bits or bits not in (3, 4):
        raise ValueError("HEX tables have 8 or 16 levels")
    W = W.float()
    x = W.reshape(n, out, inp // block, block)
    amax = x.abs().amax(-1)                                                     # [n, out, nblk]
    es = (amax.reshape(n, -1).amax(1).double() / FP8_MAX).clamp(min=1e-30)
    es32 = es.float()[:, None, None]
    vals = _fp8_values(W.device)
    blk = vals[fp8_encode(torch.minimum(amax / es32, torch.tensor(FP8_MAX, device=W.device))).long()] * es32
    blk = torch.where(blk > 0, blk, torch.ones_like(blk))
    xn = (x / blk[..., None]).clamp(-1, 1).reshape(n, out, inp)
    levels = fit_tables(xn.reshape(n, -1), L)
    mids = ((levels[:, 1:] + levels[:, :-1]) / 2).contiguous()
    codes = torch.searchsorted(mids, xn.reshape(n, -1).contiguous()).reshape(n, out, inp)
    bs = fp8_encode(torch.minimum(blk / es32, torch.tensor(FP8_MAX, device=W.device)))
    return {"idx": pack(codes, bits), "block_scale": bs.contiguous(), "expert_scale": es.float().contiguous(),
            "levels": levels.contiguous()}


def random_parts(n: int, out: int, inp: int, bits: int, device="cuda", seed: int = 0, block: int = HEX_BLOCK) -> dict:
    """Random but well-formed HEX parts (uniform codes, fp8 codes 40..69 ~ 0.1..1, expert scale
    0.01..0.03, sorted uniform levels in [-1, 1]; distributed as runtime/blackhole_runtime/
    hex_ref.py:64-74) from a seeded torch generator."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    codes = torch.randint(0, 2 ** bits, (n, out, inp), generator=g)
    return {"idx": pack(codes.to(device), bits),
            "block_scale": torch.randint(40, 70, (n, out, inp // block), generator=g, dtype=torch.int32)
            .to(torch.uint8).to(device),
            "expert_scale": (torch.rand(n, generator=g) * 0.02 + 0.01).to(device),
            "levels": torch.sort(torch.rand(n, 2 ** bits, generator=g) * 2 - 1, dim=-1).values.to(device)}
