"""The folder checker's kernel check and the GPU reference MoE it compares with (marked gpu).

hex_ref.moe_reference (this library's dequant kernel, order R, and torch float32 products) is
pinned to the CPU oracle's moe_reference on the same parts (both float32; 1e-5 relative). The
checker then passes good folders of both scale-block sizes with the fused kernels within the
north-star bound (1e-2 with bf16 activations), as runtime/tests/test_folder.py:38-47 does on the
CPU, and still reports a folder whose tiers miss an expert."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from blackhole_runtime import check_folder as cf
from blackhole_runtime import hex_ref
from blackhole_runtime.quant import random_parts
from oracle import hex_oracle as O
from test_folder import write_folder

pytestmark = pytest.mark.gpu
DEV = "cuda"


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("block", [32, 128])
def test_gpu_reference_equals_oracle(block):
    say(f"hex_ref.moe_reference vs oracle, block {block}")
    E, H, I, k, T = 6, 256, 128, 2, 9
    tiers, ora = [], []
    for bits, ids in ((4, [0, 2, 4]), (3, [1, 3, 5])):
        parts = {p: random_parts(len(ids), o, i, bits, device=DEV, seed=bits * 7 + j, block=block)
                 for j, (p, (o, i)) in enumerate((("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))))}
        tiers.append({"bits": bits, "experts": torch.tensor(ids), **parts})
        ora.append({"bits": bits, "experts": np.array(ids),
                    **{p: {"idx": v["idx"].cpu().numpy().view(np.uint32), "block_scale": v["block_scale"].cpu().numpy(),
                           "expert_scale": v["expert_scale"].cpu().numpy(), "levels": v["levels"].cpu().numpy()}
                       for p, v in parts.items()}})
    g = torch.Generator().manual_seed(block)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    w = torch.softmax(torch.randn(T, k, generator=g), -1)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    got = hex_ref.moe_reference(x.to(DEV), w.to(DEV), ids.to(DEV), tiers).cpu().numpy()
    want = O.moe_reference(x.float().numpy(), w.numpy(), ids.numpy(), ora, "bf16")
    assert O.rel_err(got, want) < 1e-5


@pytest.mark.parametrize("block", [32, 128])
def test_check_folder_kernel_check(tmp_path, block):
    say(f"check_folder on a GPU, block {block}")
    write_folder(tmp_path, E=8, H=256, I=128, hot=4, block=block)
    r = cf.check(tmp_path, DEV, tokens=7)
    say(f"  {r}")
    assert r["ok"] and r["layers"] == 2 and r["checked"] == 2, r
    assert r["kernel_rel"] < 1e-2
    r = cf.check(tmp_path, DEV, n_layers=1)
    assert r["ok"] and r["checked"] == 1, r
    bad = tmp_path / "bad"
    bad.mkdir()
    write_folder(bad, E=8, H=256, I=128, hot=4, block=block, drop=5)
    r = cf.check(bad, DEV)
    assert not r["ok"] and "expected each of 0..7 once" in r["problems"][0] and r["checked"] == 0, r
