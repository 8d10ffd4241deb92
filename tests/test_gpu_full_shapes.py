"""The fused layer at BASELINE's full shapes, where the CPU oracle would take minutes per call
(marked gpu).

The reference here is hex_ref.moe_reference: this library's dequant kernel (order R, bit-exact
against the oracle's dequant) and torch float32 products on the GPU, which test_gpu_folder.py pins
to the oracle's moe_reference at 1e-5. The parts are random but well-formed and generated on the
device (any 32-bit word is a valid packed stream of 3- or 4-bit codes), so that config 5's
2.4 G codes per layer never pass through host memory. Bound: the north star's 1e-2 (max|got -
ref| / max|ref|, bf16 activations), as runtime/tests/test_hex_moe.py:80 measures it."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from blackhole_runtime import hex_moe as hm
from blackhole_runtime import hex_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL_16 = 1e-2


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def device_parts(n: int, out: int, inp: int, bits: int, block: int, g: torch.Generator) -> dict:
    """HEX parts of n experts drawn as hex_ref.py:64-74 draws them (uniform codes, fp8 codes
    40..69, expert scales 0.01..0.03, sorted uniform levels in [-1, 1]), on the GPU."""
    return {"idx": torch.randint(-(2 ** 31), 2 ** 31 - 1, (n, out, inp // 32 * bits), generator=g, device=DEV,
                                 dtype=torch.int32),
            "block_scale": torch.randint(40, 70, (n, out, inp // block), generator=g, device=DEV,
                                         dtype=torch.int32).to(torch.uint8),
            "expert_scale": torch.rand(n, generator=g, device=DEV) * 0.02 + 0.01,
            "levels": torch.sort(torch.rand(n, 2 ** bits, generator=g, device=DEV) * 2 - 1, dim=-1).values}


def rel_err(got: torch.Tensor, want: torch.Tensor) -> float:
    return ((got.float() - want).abs().max() / want.abs().max()).item()


# (name, E, H, I, k, tiers as (experts, bits), T, zipf) at 128-input scale blocks, as BASELINE
# states them, at every batch the benchmark reports: config 2's decode sweep (16-slot blocks, the
# kernels sorting the slots themselves), config 3's prefill (3-bit, the 128-slot kernels),
# config 4's two REAQ tiers under Zipf routing, config 5's sweep (T=256: 32-slot blocks behind
# the align kernel; T=8192: 65,536 slots through the chunked align and the prefill kernels).
SHAPES = [
    ("config2-T1", 96, 2048, 768, 8, ((96, 4),), 1, 0.0),
    ("config2-T4", 96, 2048, 768, 8, ((96, 4),), 4, 0.0),
    ("config2-T16", 96, 2048, 768, 8, ((96, 4),), 16, 0.0),
    ("config2-T64", 96, 2048, 768, 8, ((96, 4),), 64, 0.0),
    ("config3", 96, 2048, 768, 8, ((96, 3),), 4096, 0.0),
    ("config4", 96, 2048, 768, 8, ((48, 4), (48, 3)), 256, 1.1),
    ("config5-T1", 128, 4096, 1536, 8, ((128, 4),), 1, 0.0),
    ("config5-T4", 128, 4096, 1536, 8, ((128, 4),), 4, 0.0),
    ("config5-decode", 128, 4096, 1536, 8, ((128, 4),), 16, 0.0),
    ("config5-T256", 128, 4096, 1536, 8, ((128, 4),), 256, 0.0),
    ("config5-prefill", 128, 4096, 1536, 8, ((128, 4),), 2048, 0.0),
    ("config5-T8192", 128, 4096, 1536, 8, ((128, 4),), 8192, 0.0),
]


@pytest.mark.parametrize("name,E,H,I,k,groups,T,zipf", SHAPES, ids=[s[0] for s in SHAPES])
def test_full_shape_layer(name, E, H, I, k, groups, T, zipf, monkeypatch):
    say(f"full shape {name}: E={E} H={H} I={I} k={k} tiers={groups} T={T}")
    block = 128
    g = torch.Generator(device=DEV).manual_seed(E + T)
    perm = np.random.default_rng(E + T).permutation(E)
    tiers, ref_tiers, c0 = [], [], 0
    for n, bits in groups:
        ids = torch.from_numpy(np.sort(perm[c0:c0 + n]).astype(np.int32))
        c0 += n
        parts = {p: device_parts(n, o, i, bits, block, g)
                 for p, (o, i) in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I)))}
        ref_tiers.append({"bits": bits, "experts": ids, **parts})
        tiers.append(hm.HexTier(bits, ids, parts["gate_proj"], parts["up_proj"], parts["down_proj"]).prepare(E))
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(DEV)
    logits = torch.randn(T, E, generator=torch.Generator().manual_seed(2))
    if zipf:
        p = 1.0 / np.arange(1, E + 1) ** zipf
        logits = logits + torch.from_numpy(np.log(p / p.sum())[perm]).float()
    w, ids = hm.route_topk(logits.to(DEV), k)
    want = hex_ref.moe_reference(x, w, ids, ref_tiers)
    fused = hm.hex_moe_fused(x, w, ids, tiers)
    assert fused.dtype == torch.bfloat16 and fused.shape == (T, H)
    err = rel_err(fused, want)
    say(f"  fused: {err:.2e}")
    assert err < TOL_16, err
    deq = hm.hex_moe(x, w, ids, tiers, path="dequant")
    err = rel_err(deq, want)
    say(f"  dequant: {err:.2e}")
    assert err < TOL_16, err
    if hm.DEQUANT_MIN > T * k:
        # path="auto" keeps to the fused kernels at every batch unless BLACKHOLE_HEX_DEQUANT_MIN
        # is set (the fused results do not depend on timing, so they are equal bit for bit)
        assert torch.equal(hm.hex_moe(x, w, ids, tiers), fused)
    blocks = fused
    if len(tiers) == 1 and hm.gemv_prefer(T, k, H, I, tiers[0]):
        # the layer ran as the two matrix-vector launches; now through the expert-block kernels
        monkeypatch.setattr(hm, "GEMV_MAX", 0)
        blocks = hm.hex_moe_fused(x, w, ids, tiers)
        err = rel_err(blocks, want)
        say(f"  expert-block kernels: {err:.2e}")
        assert err < TOL_16, err
        monkeypatch.undo()
    if T * k <= hm.KERNEL_PLAN_MAX:
        # the kernels' own slot plan equals the align kernel's (align_mode "vllm" maps to the align
        # kernel at every batch), so the outputs are equal bit for bit
        assert torch.equal(hm.hex_moe_fused(x, w, ids, tiers, align_mode="vllm"), blocks)
    if T * k <= hm.DIRECT_MAX:
        # the reference's direct plan (one block per slot) at full width
        err = rel_err(hm.hex_moe_fused(x, w, ids, tiers, align_mode="direct"), want)
        say(f"  direct plan: {err:.2e}")
        assert err < TOL_16, err
