"""Reference MoE for HEX experts, on the GPU (runtime/blackhole_runtime/hex_ref.py).

The layer computed the plain way: every tier's weights dequantized to float32 by this
library's dequant kernel, in the association order of the HEX source of truth
(level * (fp8 * expert_scale), blackhole/anatomy/hex.py:180-204), then torch float32 products per
routed expert. The folder checker compares the fused kernels with it. It shares no code with
the fused kernels beyond the tensor layout, and it has no CPU path: like every operator of this
package it refuses CPU tensors.

Layout per tier and projection [out, in] (in a multiple of 32; hex_ref.py:4-11):
  idx           uint32 / int32 [n, out, in / 32 * bits]
  block_scale   uint8 [n, out, in / B]      (B = 32 in the reference's writers; any multiple of 32)
  expert_scale  float32 [n]
  levels        float32 [n, 2**bits]
"""

from __future__ import annotations

import torch

from . import hex_moe as _hm
from .quant import HEX_BLOCK, pack, random_parts  # noqa: F401  (the reference module's names)

_PARTS = ("idx", "block_scale", "expert_scale", "levels")
_PROJS = ("gate_proj", "up_proj", "down_proj")


def hex_dequant(idx, block_scale, expert_scale, levels, bits: int) -> torch.Tensor:
    """Float32 weights [n, out, in] of stacked HEX parts on the GPU (hex_ref.py:25-45), in
    order R: level * (fp8 * expert_scale)."""
    return _hm.hex_dequant(idx, block_scale, expert_scale, levels, bits, order="R", dtype=torch.float32)


def moe_reference(x, topk_weights, topk_ids, tiers: list[dict]) -> torch.Tensor:
    """Routed-expert output [T, H] float32 of a SwiGLU MoE whose experts are split over HEX tiers
    (hex_ref.py:77-94). Each tier: {"bits", "experts": int ids [n], "gate_proj" / "up_proj" /
    "down_proj": parts}, on the device of x. The activation handed to the down product is
    rounded to x.dtype, as the kernels hand it over."""
    _hm._lib.require_gpu(x, topk_weights, topk_ids)
    T = topk_ids.shape[0]
    out = torch.zeros(T, x.shape[1], dtype=torch.float32, device=x.device)
    xf = x.float()
    ids = topk_ids.long()
    for t in tiers:
        W = {p: hex_dequant(*(t[p][q] for q in _PARTS), t["bits"]) for p in _PROJS}
        for local, e in enumerate(t["experts"].tolist()):
            tok, slot = (ids == e).nonzero(as_tuple=True)
            if tok.numel() == 0:
                continue
            a = xf[tok]
            h = torch.nn.functional.silu(a @ W["gate_proj"][local].T) * (a @ W["up_proj"][local].T)
            h = h.to(x.dtype).float()
            out.index_add_(0, tok, (h @ W["down_proj"][local].T) * topk_weights[tok, slot, None].float())
    return out
