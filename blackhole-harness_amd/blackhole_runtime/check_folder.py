"""Check a "blackhole-hex" folder before serving it (runtime/blackhole_runtime/check_folder.py).

Every MoE layer's HEX tiers must load, cover every expert exactly once, and have consistent
shapes (with each other and with config.json where it states them); then, on a GPU, the fused
HEX kernels on them must equal the float32 reference MoE computed from the dequantized tiers
(hex_ref.moe_reference) for a few random tokens and routings per layer.

    python -m blackhole_runtime.check_folder <hex folder> [--device cuda] [--layers 4] [--tokens 5]

Tensors are found by name, <...>.experts.tier<L>.{experts | <proj>.<part>} (the layout of the
pipeline's hexvllm stage, harness/blackhole_pipeline/stages/hexvllm.py:19-21), so any MoE
architecture works. Prints one JSON line at the end; exit code 1 on any problem. There is no CPU
path for the kernels: with a CPU device the structure is checked and the kernel check is
reported as skipped.
"""

from __future__ import annotations

import argparse
import json
import re
import sys
from pathlib import Path

import torch

# <prefix>.tier<L>.experts | <prefix>.tier<L>.<proj>.<part>  (check_folder.py:24-25)
_NAME = re.compile(r"^(?P<pre>.+)\.tier(?P<L>\d+)\.(?:experts|(?P<proj>gate_proj|up_proj|down_proj)\."
                   r"(?P<part>idx|block_scale|expert_scale|levels))$")
_PROJS = ("gate_proj", "up_proj", "down_proj")
_PARTS = ("idx", "block_scale", "expert_scale", "levels")


def _natural(s: str) -> list:
    return [int(p) if p.isdigit() else p for p in re.split(r"(\d+)", s)]


def tiers_by_layer(folder: Path) -> dict[str, dict[int, dict]]:
    """{experts prefix: {levels L: {"experts": ids, proj: {part: tensor}}}} of every HEX tier in
    the folder's safetensors files (check_folder.py:28-44). Tensors stay on the CPU."""
    from safetensors import safe_open
    out: dict = {}
    for f in sorted(Path(folder).glob("*.safetensors")):
        with safe_open(str(f), "pt") as h:
            for name in h.keys():
                m = _NAME.match(name)
                if not m:
                    continue
                tier = out.setdefault(m["pre"], {}).setdefault(int(m["L"]), {})
                if m["proj"]:
                    tier.setdefault(m["proj"], {})[m["part"]] = h.get_tensor(name)
                else:
                    tier["experts"] = h.get_tensor(name)
    return out


def _shape_problems(pre: str, tiers: dict[int, dict], H_cfg: int | None, I_cfg: int | None) -> list[str]:
    """What is missing or inconsistent in one layer's tiers (empty when the kernels can take them)."""
    probs, dims = [], set()
    for L, t in sorted(tiers.items(), reverse=True):
        bits = L.bit_length() - 1
        name = f"{pre}.tier{L}"
        if L != 1 << bits or bits not in (3, 4):
            probs.append(f"{name}: HEX tables have 8 or 16 levels, not {L}")
            continue
        missing = (["experts"] if "experts" not in t else []) + [f"{p}.{q}" for p in _PROJS for q in _PARTS
                                                                 if q not in t.get(p, {})]
        if missing:
            probs.append(f"{name}: missing {', '.join(missing[:4])}")
            continue
        n = t["experts"].numel()
        outs = {}
        for p in _PROJS:
            idx, bs, es, lv = (t[p][q] for q in _PARTS)
            if idx.dim() != 3 or idx.shape[0] != n or idx.shape[2] % bits:
                probs.append(f"{name}.{p}.idx: shape {tuple(idx.shape)} is not [{n}, out, in/32*{bits}]")
                continue
            out, n_in = idx.shape[1], idx.shape[2] // bits * 32
            if bs.dim() != 3 or tuple(bs.shape[:2]) != (n, out) or bs.shape[2] == 0 or n_in % bs.shape[2] \
                    or (n_in // bs.shape[2]) % 32:
                probs.append(f"{name}.{p}.block_scale: shape {tuple(bs.shape)} does not fit idx {tuple(idx.shape)}")
            if es.numel() != n:
                probs.append(f"{name}.{p}.expert_scale: {es.numel()} values for {n} experts")
            if tuple(lv.shape) != (n, L):
                probs.append(f"{name}.{p}.levels: shape {tuple(lv.shape)}, expected ({n}, {L})")
            outs[p] = (out, n_in)
        if len(outs) == 3:
            (I_g, H_g), (I_u, H_u), (H_d, I_d) = outs["gate_proj"], outs["up_proj"], outs["down_proj"]
            if not (I_g == I_u == I_d and H_g == H_u == H_d):
                probs.append(f"{name}: gate {outs['gate_proj']}, up {outs['up_proj']} and down {outs['down_proj']} "
                             "(out, in) do not describe one SwiGLU expert")
            else:
                dims.add((H_g, I_g))
    if len(dims) > 1:
        probs.append(f"{pre}: tiers disagree on (hidden, intermediate): {sorted(dims)}")
    elif dims:
        H, I = dims.pop()
        if H_cfg and H != H_cfg:
            probs.append(f"{pre}: hidden size {H}, config.json says {H_cfg}")
        if I_cfg and I != I_cfg:
            probs.append(f"{pre}: expert intermediate size {I}, config.json says {I_cfg}")
    return probs


def check(folder: Path, device: str = "cuda", n_layers: int = 0, tokens: int = 5) -> dict:
    """Check one folder (check_folder.py:47-99): {"layers", "checked", "kernel_rel", "problems",
    "ok"}. n_layers > 0 kernel-checks only the first n layers; the kernel check runs on a GPU
    device only ("kernel_rel" None otherwise)."""
    folder = Path(folder)
    cfg = json.loads((folder / "config.json").read_text())
    q = cfg.get("quantization_config") or {}
    problems = []
    if q.get("quant_method") != "blackhole-hex":
        problems.append(f"config.json quantization_config.quant_method is {q.get('quant_method')!r}, "
                        "not 'blackhole-hex'")
    tc = cfg.get("text_config") or cfg
    E = next((tc[key] for key in ("num_experts", "num_local_experts", "n_routed_experts")
              if isinstance(tc.get(key), int)), None)
    k = int(tc.get("num_experts_per_tok") or 2)
    H_cfg = tc.get("hidden_size") if isinstance(tc.get("hidden_size"), int) else None
    I_cfg = tc.get("moe_intermediate_size") if isinstance(tc.get("moe_intermediate_size"), int) else None
    layers = tiers_by_layer(folder)
    if not layers:
        problems.append("no HEX tiers (<...>.experts.tier<L>.*) in the safetensors files")
    dev = torch.device(device)
    gpu = dev.type == "cuda"
    worst, checked = 0.0, 0
    for li, (pre, tiers) in enumerate(sorted(layers.items(), key=lambda kv: _natural(kv[0]))):
        shape = _shape_problems(pre, tiers, H_cfg, I_cfg)
        if shape:
            problems.extend(shape)
            continue
        seen = torch.cat([t["experts"].reshape(-1).long() for t in tiers.values()])
        n_exp = E or (int(seen.max()) + 1 if seen.numel() else 0)
        if sorted(seen.tolist()) != list(range(n_exp)):
            problems.append(f"{pre}: tiers hold experts {sorted(seen.tolist())[:6]}..., expected each of "
                            f"0..{n_exp - 1} once")
            continue
        if not gpu or (n_layers and checked >= n_layers):
            continue
        worst = max(worst, _kernel_rel(tiers, n_exp, k, tokens, li, dev))
        checked += 1
    tol = 2e-2        # bf16 activations (check_folder.py:90)
    if gpu and checked and worst >= tol:
        problems.append(f"HEX kernel differs from the reference MoE by {worst:.1e} (tolerance {tol:.0e})")
    return {"layers": len(layers), "checked": checked, "kernel_rel": worst if gpu else None,
            "problems": problems, "ok": not problems}


def _kernel_rel(tiers: dict[int, dict], n_exp: int, k: int, tokens: int, seed: int, dev: torch.device) -> float:
    """max|fused - reference| / max|reference| on one layer, for `tokens` seeded tokens and routings."""
    from .hex_moe import HexTier, hex_moe
    from .hex_ref import moe_reference
    ref_tiers, run_tiers = [], []
    for L, t in sorted(tiers.items(), reverse=True):
        bits = L.bit_length() - 1
        parts = {p: {q: t[p][q].to(dev) for q in _PARTS} for p in _PROJS}
        ids = t["experts"].reshape(-1).to(torch.int32)
        ref_tiers.append({"bits": bits, "experts": ids.long(), **parts})
        run_tiers.append(HexTier(bits, ids.to(dev), *(parts[p] for p in _PROJS)).prepare(n_exp))
    H = ref_tiers[0]["gate_proj"]["idx"].shape[-1] * 32 // ref_tiers[0]["bits"]
    g = torch.Generator().manual_seed(seed)
    topk = torch.stack([torch.randperm(n_exp, generator=g)[:min(k, n_exp)] for _ in range(tokens)])
    w = torch.softmax(torch.randn(tokens, topk.shape[1], generator=g), -1)
    x = torch.randn(tokens, H, generator=g).to(torch.bfloat16).to(dev)
    want = moe_reference(x, w.to(dev), topk.to(dev), ref_tiers)
    got = hex_moe(x, w.to(dev), topk.to(dev), run_tiers).float()
    return float((got - want).abs().max() / (want.abs().max() + 1e-12))


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("folder", type=Path)
    ap.add_argument("--device", default="cuda" if torch.cuda.is_available() else "cpu")
    ap.add_argument("--layers", type=int, default=0, help="kernel-check only the first N layers (0 = all)")
    ap.add_argument("--tokens", type=int, default=5)
    a = ap.parse_args(argv)
    res = check(a.folder, a.device, a.layers, a.tokens)
    for p in res["problems"]:
        print(f"problem: {p}", file=sys.stderr)
    rel = "skipped (no GPU)" if res["kernel_rel"] is None else f"max rel diff {res['kernel_rel']:.1e}"
    print(f"{res['layers']} HEX layers, {res['checked']} kernel-checked, {rel} ({'OK' if res['ok'] else 'PROBLEMS'})",
          file=sys.stderr)
    print(json.dumps(res))
    return 0 if res["ok"] else 1


if __name__ == "__main__":
    raise SystemExit(main())
