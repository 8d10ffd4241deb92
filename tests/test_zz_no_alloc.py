"""bh_hex_moe_glu_ids_noalloc (workspace in the library's static device array) against
bh_hex_moe_glu_ids (workspace allocated by the caller), both called through the C ABI.

The two run the same kernel over the same plan, and the split items' partial sums are added in
workgroup order either way, so the outputs must be equal bit for bit. Two calls in a row, the
second with fewer tokens (the array keeps the first call's contents), then a launch too large
for the array, which must be refused with a clear error."""

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


def _tier(E, H, I, bits, seed):
    parts = []
    for q, (o, i) in enumerate(((I, H), (I, H), (H, I))):
        p = O.random_parts(E, o, i, bits, seed=seed + q, block=128)
        parts.append({"idx": torch.from_numpy(np.ascontiguousarray(p["idx"]).view(np.int32)).to(DEV),
                      "block_scale": torch.from_numpy(p["block_scale"]).to(DEV),
                      "expert_scale": torch.from_numpy(p["expert_scale"].astype(np.float32)).to(DEV),
                      "levels": torch.from_numpy(p["levels"].astype(np.float32)).to(DEV)})
    return hm.HexTier(bits, torch.arange(E, dtype=torch.int32), *parts).prepare(E)


def _noalloc(x, act, t, ids, code, S, k, bm):
    lib = _lib.load()
    n_out = t.gate_proj["idx"].shape[1]
    n_in = hm._n_in(t.gate_proj, t.bits)
    tile = _lib.HexTile(bm, 256, 1)
    _lib.check(lib.bh_hex_moe_glu_ids_noalloc(
        x.data_ptr(), _lib.dtype_code(x.dtype), x.stride(0), act.data_ptr(), act.stride(0),
        t.struct("gate_proj"), t.struct("up_proj"), t.bits, n_out, n_in, ids.data_ptr(), code, t.lookup.data_ptr(),
        t.lookup.numel(), S, k, tile, _lib.stream_of(x)), "bh_hex_moe_glu_ids_noalloc")


@pytest.mark.parametrize("bits", [4, 3])
def test_noalloc_equals_workspace_entry_point(bits):
    E, H, I, k = 12, 2048, 768, 8
    t = _tier(E, H, I, bits, seed=40 + bits)
    for T in (16, 1):                          # the second call is smaller
        say(f"noalloc bits={bits} E={E} H={H} I={I} k={k} T={T}")
        S = T * k
        g = torch.Generator().manual_seed(T)
        x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV)
        ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(DEV)
        flat, code = hm._ids_arg(ids)
        want = torch.full((S, I), -1.0, dtype=torch.bfloat16, device=DEV)
        got = torch.full((S, I), 7.0, dtype=torch.bfloat16, device=DEV)
        hm._launch_glu_ids(x, want, t, flat, code, S, k, 16)
        _noalloc(x, got, t, flat, code, S, k, 16)
        torch.cuda.synchronize()
        assert torch.isfinite(want.float()).all()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"T={T}: outputs differ"


def test_noalloc_refuses_launches_beyond_its_scratch():
    say("noalloc size limit")
    E, k = 1024, 8
    t = _tier(8, 128, 128, 4, seed=3)
    lk = torch.zeros(E, dtype=torch.int32, device=DEV)
    x = torch.zeros(128, 128, dtype=torch.bfloat16, device=DEV)
    act = torch.zeros(8, 8192, dtype=torch.bfloat16, device=DEV)   # (never read: the call is refused first)
    ids = torch.zeros(1024, dtype=torch.int64, device=DEV)
    lib = _lib.load()
    # 1088 blocks x 32 row tiles x 16 counters per item: beyond the array's 2^18 counters
    rc = lib.bh_hex_moe_glu_ids_noalloc(x.data_ptr(), _lib.BF16, 128, act.data_ptr(), 8192, t.struct("gate_proj"),
                                        t.struct("up_proj"), 4, 8192, 128, ids.data_ptr(), _lib.I64, lk.data_ptr(), E,
                                        1024, k, _lib.HexTile(16, 256, 1), _lib.stream_of(x))
    assert rc == _lib.ERR_UNSUPPORTED
    assert b"static scratch" in lib.bh_hex_last_error()
