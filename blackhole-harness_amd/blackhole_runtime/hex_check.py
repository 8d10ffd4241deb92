"""Check and time the HEX MoE layer on the GPU (the counterpart of runtime/blackhole_runtime/hex_check.py).

    python -m blackhole_runtime.hex_check                    # the reference's default shape (176 experts)
    python -m blackhole_runtime.hex_check --experts 128 --hidden 2048 --inter 768 --topk 8
    python -m blackhole_runtime.hex_check --sweep            # also time each slot-block size

1. Numbers: the fused HIP kernels (and the dequant path) against hex_ref.moe_reference (every
   tier dequantized to float32 by this library's dequant kernel, then float32 products) for one
   token, a few tokens and a prompt, with a 4-bit and a 3-bit tier, in bf16. Passes below the
   reference's 2e-2 relative error (hex_check.py:116-118); the error against the 1e-2 bound of
   this build's parity tests is printed too.
2. Speed per MoE layer (gate + up + down for every routed slot, and the k-slot sum), hipGraph
   replays where the call allows capture: decode batches of 1 / 8 / 32 / 128 tokens and 1024-
   and 4096-token prompts, through the fused kernels, the dequant path, and path="auto". vLLM's
   fused MoE is timed beside them when vLLM is importable (it is not on this image).
Memory: a few hundred MB of random experts (1 GB more for the dequant path's bf16 stacks at the
default shape), no model download.
"""

from __future__ import annotations

import argparse
import time

import torch

from blackhole_runtime.hex_moe import HexTier, hex_moe, hex_moe_fused
from blackhole_runtime.hex_ref import moe_reference
from blackhole_runtime.quant import random_parts

TOL_REFERENCE = 2e-2     # hex_check.py:118
TOL_BUILD = 1e-2         # this build's bound (max relative error, bf16 activations)


def build(E: int, H: int, I: int, hot: int, dev, seed: int = 0):
    """(prepared HexTiers, reference tier dicts): a 4-bit tier of `hot` experts and a 3-bit tier
    of the rest, random well-formed parts (hex_check.py:32-44)."""
    perm = torch.randperm(E, generator=torch.Generator().manual_seed(seed))
    tiers, ref = [], []
    for i, (ids, bits) in enumerate(((perm[:hot], 4), (perm[hot:], 3))):
        if len(ids) == 0:
            continue
        parts = [random_parts(len(ids), o, n, bits, dev, seed + 10 * i + j)
                 for j, (o, n) in enumerate(((I, H), (I, H), (H, I)))]
        ids32 = ids.to(torch.int32).to(dev)
        ref.append({"bits": bits, "experts": ids32, "gate_proj": dict(parts[0]), "up_proj": dict(parts[1]),
                    "down_proj": dict(parts[2])})
        tiers.append(HexTier(bits, ids32, *[dict(p) for p in parts]).prepare(E))
    return tiers, ref


def routing(T: int, E: int, k: int, dev, seed: int = 0):
    """k distinct experts per token and softmax weights (hex_check.py:47-51)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    ids = torch.argsort(torch.rand(T, E, generator=g), -1)[:, :k].to(dev).to(torch.int32)
    w = torch.softmax(torch.randn(T, k, generator=g), -1).to(dev)
    return ids, w


def timeit(fn, iters: int = 50) -> float:
    """Microseconds per call: hipGraph replays when the call can be captured (the decode path),
    else eager calls (hex_check.py:54-74)."""
    for _ in range(5):
        fn()
    torch.cuda.synchronize()
    run = fn
    try:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        run = g.replay
    except Exception:  # noqa: BLE001  (the dequant path reads back the routed experts: not capturable)
        torch.cuda.synchronize()
        run = fn
    run()
    torch.cuda.synchronize()
    t = time.perf_counter()
    for _ in range(iters):
        run()
    torch.cuda.synchronize()
    return (time.perf_counter() - t) / iters * 1e6


def vllm_baselines(E: int, H: int, I: int, dev) -> dict:
    """{name: fn(x, w, ids)} for vLLM's fused MoE on bf16 experts, when vLLM is importable."""
    try:
        from vllm.model_executor.layers.fused_moe.fused_moe import fused_experts
    except Exception as e:  # noqa: BLE001
        print(f"  (vLLM fused MoE not importable here: {type(e).__name__}; HEX timings only)")
        return {}
    w1 = torch.randn(E, 2 * I, H, device=dev, dtype=torch.bfloat16) * 0.02
    w2 = torch.randn(E, H, I, device=dev, dtype=torch.bfloat16) * 0.02
    return {"vLLM bf16": lambda x, w, ids: fused_experts(x, w1, w2, w, ids)}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--experts", type=int, default=176)
    ap.add_argument("--hidden", type=int, default=2048)
    ap.add_argument("--inter", type=int, default=512)
    ap.add_argument("--topk", type=int, default=8)
    ap.add_argument("--hot", type=float, default=0.10, help="share of experts in the 4-bit tier")
    ap.add_argument("--sweep", action="store_true", help="also time each slot-block size per batch size")
    ap.add_argument("--tokens", default="1,8,32,128,1024,4096", help="token batches to time (comma list)")
    ap.add_argument("--iters", type=int, default=0, help="timed calls per point (default 100, 20 above 512 tokens)")
    a = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("hex_check needs a ROCm GPU; the CPU tests are in tests/ (pytest -m 'not gpu')")
    dev = "cuda"
    E, H, I, k = a.experts, a.hidden, a.inter, a.topk
    hot = int(round(E * a.hot))
    print(f"{torch.cuda.get_device_name()} · {E} experts ({hot} 4-bit, {E - hot} 3-bit), hidden {H}, "
          f"expert width {I}, top-{k}")
    tiers, ref = build(E, H, I, hot, dev)
    ok = True
    for T, path in ((1, "fused"), (7, "fused"), (300, "fused"), (300, "dequant")):
        ids, w = routing(T, E, k, dev, seed=T)
        x = (torch.randn(T, H, device=dev) * 0.5).to(torch.bfloat16)
        got = hex_moe(x, w, ids, tiers, path=path).float()
        r = moe_reference(x, w, ids, ref)
        err = float((got - r).abs().max() / r.abs().max())
        print(f"  {T:4d} tokens, {path:7s}: max rel error vs reference {err:.2e}"
              f"{'' if err < TOL_BUILD else '  (above the 1e-2 build bound)'}")
        ok &= err < TOL_REFERENCE

    base = vllm_baselines(E, H, I, dev)
    gb = 3 * H * I * (3.25 * (E - hot) + 4.25 * hot) / E / 8 / 1e9   # bytes per routed expert (hex_check.py:121)
    print("  per MoE layer, microseconds (lower is better); 'auto' is what serving uses:")
    print(f"  {'tokens':>7} {'HEX auto':>9} {'HEX fused':>10} {'HEX dequant':>12} " + " ".join(f"{n:>16}" for n in base))
    for T in (int(t) for t in a.tokens.split(",") if t):
        ids, w = routing(T, E, k, dev, seed=T)
        x = (torch.randn(T, H, device=dev) * 0.5).to(torch.bfloat16)
        n_it = a.iters or (20 if T > 512 else 100)
        t = {p: timeit(lambda p=p: hex_moe(x, w, ids, tiers, path=p), iters=n_it) for p in ("auto", "fused", "dequant")}
        row = f"  {T:7d} {t['auto']:9.1f} {t['fused']:10.1f} {t['dequant']:12.1f} "
        for fn in base.values():
            try:
                row += f"{timeit(lambda: fn(x, w, ids), iters=n_it):16.1f} "
            except Exception as e:  # noqa: BLE001
                row += f"{'err ' + type(e).__name__:>16} "
        if T == 1:
            row += f"   HEX weight traffic {k * gb / (t['fused'] * 1e-6):.0f} GB/s"
        print(row)
        if a.sweep:
            best = []
            for bm in (16, 32, 64, 128):
                try:
                    best.append((timeit(lambda bm=bm: hex_moe_fused(x, w, ids, tiers, {"BLOCK_M": bm}), iters=20), bm))
                except Exception:  # noqa: BLE001
                    pass
            best.sort()
            print("          fused, slot-block sizes BLOCK_M: " + ", ".join(f"{bm} {v:.1f}" for v, bm in best))
    print("HEX HIP kernels OK" if ok else "HEX HIP kernels MISMATCH: send this output")
    return 0 if ok else 1


if __name__ == "__main__":
    raise SystemExit(main())
