"""HEX MoE layer benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps 400] [--warmup 40] [--config 2] [--tokens 16]
                    [--no-sweep] [--no-cpu-baseline] [--copy-calibration]
    python bench.py --rocprof-summary DIR [DIR ...]     (summarise rocprofv3 CSV output)

A step is one HEX MoE layer call (hex_moe through the fused HIP kernels: slot plan, gate/up +
SiLU, down + top-k weight, k-slot sum) on one batch of synthetic tokens with inputs resident
in HBM. Eight copies of the layer's weights stay resident and the steps cycle through them, so
weights stream from HBM rather than the 256 MB Infinity Cache; the eight calls are captured in
one hipGraph (as a serving engine captures its layers) and replayed. The timed region is
bracketed by torch.cuda.synchronize(); one JSON line goes to stdout, progress to stderr.

Synthetic data (no checkpoints): weights N(0, 0.02) quantized to HEX on the GPU (16 levels
rounded to fp16 for 4-bit, 8 for 3-bit; fp8 scale per 128 inputs), activations bf16 N(0, 1),
router logits N(0, 1) through the softmax top-k routing kernel. Seeds: weights 0, activations 1,
logits 2, REAQ tiering 3.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "blackhole-harness_amd"))

CONFIGS = {
    1: dict(name="config1 tiny: E=8 H=256 I=128 top-2, HEX 4-bit", E=8, H=256, I=128, k=2, bits=4, T=16),
    2: dict(name="config2 decode: Qwen3-30B-A3B after 25% REAP, E=96 H=2048 I=768 top-8, HEX 4-bit",
            E=96, H=2048, I=768, k=8, bits=4, T=16),
    3: dict(name="config3 prefill: E=96 H=2048 I=768 top-8, HEX 3-bit (3.25 bpw)", E=96, H=2048, I=768, k=8,
            bits=3, T=4096),
    4: dict(name="config4 REAQ: 48x4-bit + 48x3-bit, Zipf(1.1) routing", E=96, H=2048, I=768, k=8, bits=4,
            T=256, reaq=48, zipf=1.1),
    5: dict(name="config5: Qwen3-235B-A22B shape, E=128 H=4096 I=1536 top-8, HEX 4-bit", E=128, H=4096, I=1536,
            k=8, bits=4, T=16),
}
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
# Untimed warm-up before every timed point: at least --warmup layer calls, and replays for at
# least this long, so the GPU's clocks have settled whatever the batch size (a point timed after
# three replays of a long prefill layer measured 16% slower than after forty).
WARMUP_FLOOR_S = 0.3


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def proj_bytes(out: int, inp: int, bits: int, block: int) -> int:
    """HBM bytes of one expert projection: idx + block scales + expert scale + levels."""
    return out * inp * bits // 8 + out * inp // block + 4 + 4 * (1 << bits)


def build_tiers(cfg, block, copies, dev):
    """`copies` independent copies of one layer's HexTiers (weights quantized once on the GPU)."""
    import torch

    from blackhole_runtime import hex_moe as hm
    from blackhole_runtime import quant
    E, H, I = cfg["E"], cfg["H"], cfg["I"]
    g = torch.Generator(device=dev).manual_seed(0)
    if cfg.get("reaq"):
        score = torch.rand(E, generator=torch.Generator().manual_seed(3))
        order = torch.argsort(score, descending=True)
        groups = [(order[:cfg["reaq"]], 4), (order[cfg["reaq"]:], 3)]
    else:
        groups = [(torch.arange(E), cfg["bits"])]
    base = []
    for ids, bits in groups:
        parts = {}
        for proj, (o, i) in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
            chunks = []
            for c0 in range(0, len(ids), 16):
                n = min(16, len(ids) - c0)
                W = torch.randn(n, o, i, generator=g, device=dev) * 0.02
                chunks.append(quant.quantize_experts(W, 1 << bits, block))
                del W
            p = {q: torch.cat([c[q] for c in chunks]) for q in chunks[0]}
            if bits == 4:
                p["levels"] = p["levels"].half().float()       # 16-level fp16 tables
            parts[proj] = p
        base.append((ids.to(torch.int32), bits, parts))
    out = []
    for c in range(copies):
        tiers = []
        for ids, bits, parts in base:
            cp = {proj: {q: (t if c == 0 else t.clone()) for q, t in p.items()} for proj, p in parts.items()}
            tiers.append(hm.HexTier(bits, ids.clone(), cp["gate_proj"], cp["up_proj"], cp["down_proj"]).prepare(E))
        out.append(tiers)
    torch.cuda.synchronize()
    return out


def make_inputs(cfg, T, dev):
    import numpy as np
    import torch

    from blackhole_runtime import hex_moe as hm
    E, H, k = cfg["E"], cfg["H"], cfg["k"]
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(dev)
    logits = torch.randn(T, E, generator=torch.Generator().manual_seed(2))
    if cfg.get("zipf"):
        p = 1.0 / np.arange(1, E + 1) ** cfg["zipf"]
        perm = np.random.default_rng(2).permutation(E)
        logits = logits + torch.from_numpy(np.log(p / p.sum())[perm]).float()
    w, ids = hm.route_topk(logits.to(dev), k)
    return x, w, ids, logits


def layer_bytes(cfg, tiers, ids, block, T):
    """(whole-layer algorithmic HBM bytes, gate/up-launch bytes) for the routed experts."""
    import torch
    H, I, k = cfg["H"], cfg["I"], cfg["k"]
    used = set(torch.unique(ids).tolist())
    total, glu = 0, 0
    for t in tiers:
        mine = used.intersection(t._experts_host.tolist())
        gu = 2 * proj_bytes(I, H, t.bits, block)
        total += len(mine) * (gu + proj_bytes(H, I, t.bits, block))
        glu += len(mine) * gu
    total += 2 * T * H + 2 * T * H + 8 * T * k
    glu += 2 * T * H + 2 * T * k * I
    return total, glu, len(used)


def graph_of(fn):
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def warm(g, calls_per_replay: int, min_calls: int) -> int:
    """Replays graph g (untimed) until it has run at least min_calls layer calls and
    WARMUP_FLOOR_S seconds; returns the calls run."""
    import torch
    calls, t0 = 0, time.perf_counter()
    while calls < min_calls or time.perf_counter() - t0 < WARMUP_FLOOR_S:
        g.replay()
        calls += calls_per_replay
        if calls >= min_calls:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return calls


def event_time_ms(g, reps: int) -> float:
    """Average milliseconds per replay of graph g, from HIP events on the current stream."""
    import torch
    warm(g, 1, 1)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        g.replay()
    b.record()
    b.synchronize()
    return a.elapsed_time(b) / reps


def kernel_breakdown(cfg, copies, x, w, ids, reps):
    """Average microseconds per launch of each kernel the layer runs (graphs of one kernel kind over
    the copies), with the launches hex_moe_fused chooses: up to KERNEL_PLAN_MAX slots on the decode
    kernels these sort the slots themselves (no plan launch), otherwise the align plan."""
    import torch

    from blackhole_runtime import _lib
    from blackhole_runtime import hex_moe as hm
    T, k = ids.shape
    S = T * k
    E, H, I = cfg["E"], cfg["H"], cfg["I"]
    if len(copies[0]) == 1 and hm.gemv_prefer(T, k, H, I, copies[0][0]):
        # hex_moe_fused runs the layer as the two matrix-vector launches of one call
        def gemv():
            for tiers in copies:
                hm.hex_moe_gemv(x, w, ids, tiers[0])
        return {"gemv_us": event_time_ms(graph_of(gemv), reps) * 1e3 / len(copies),
                "kernel": "gemv_glu_kernel + gemv_down_kernel (the whole layer)",
                "tiles": {"path": "matrix-vector: bh_hex_moe_gemv (gate/up, then down with the k-slot sum)"}}
    flat = ids.reshape(-1)
    ids_flat, code = hm._ids_arg(flat)
    c1 = hm.default_config(S, I, H, True, E)
    c2 = hm.default_config(S, H, I, False, E)
    bm1 = hm._tile_from(c1)
    bm2 = hm._tile_from(c2)
    own1 = bm1 != 128 and S <= hm.KERNEL_PLAN_MAX          # as hex_moe_fused (align_mode "auto")
    own2 = bm2 != 128 and S <= hm.KERNEL_PLAN_MAX
    n_tiers = len(copies[0])
    lks = [t.lookup if n_tiers > 1 else None for t in copies[0]]     # per-tier plans, as hex_moe_fused
    p1 = [None if own1 else hm.plan(flat, E, bm1, "auto", lk) for lk in lks]
    p2 = [None if own2 else hm.plan(flat, E, bm2, "auto", lk) for lk in lks]
    act = torch.empty(S, I, dtype=x.dtype, device=x.device)
    y = torch.empty(S, H, dtype=x.dtype if bm2 == 128 else torch.float32, device=x.device)   # as hex_moe_fused
    out = torch.empty(T, H, dtype=x.dtype, device=x.device)
    wf = w.reshape(-1).float().contiguous()
    res = {}

    def glu():
        for tiers in copies:
            for i, t in enumerate(tiers):
                if own1:
                    hm._launch_glu_ids(x, act, t, ids_flat, code, S, k, bm1)
                else:
                    hm._launch_glu(x, act, t, *p1[i], S, k, bm1)

    def down():
        for tiers in copies:
            for i, t in enumerate(tiers):
                if own2:
                    hm._launch_down_ids(act, y, t, ids_flat, code, S, wf, bm2)
                else:
                    hm._launch_down(act, y, t, *p2[i], S, wf, bm2)

    def plan():
        for _ in copies:
            for lk in lks:
                hm.plan(flat, E, bm1, "auto", lk)

    def reduce():
        lib = _lib.load()
        for _ in copies:
            _lib.check(lib.bh_hex_moe_reduce(y.data_ptr(), _lib.dtype_code(y.dtype), y.stride(0), ids_flat.data_ptr(),
                                             code, E, T, k, H, out.data_ptr(), _lib.dtype_code(out.dtype),
                                             out.stride(0), _lib.stream_of(x)), "bh_hex_moe_reduce")

    n = len(copies)
    res["glu_us"] = event_time_ms(graph_of(glu), reps) * 1e3 / (n * n_tiers)
    res["down_us"] = event_time_ms(graph_of(down), reps) * 1e3 / (n * n_tiers)
    res["plan_us"] = 0.0 if (own1 and own2) else event_time_ms(graph_of(plan), reps) * 1e3 / n
    res["sum_us"] = event_time_ms(graph_of(reduce), reps) * 1e3 / n
    res["tiles"] = {"glu": c1, "down": c2,
                    "plan": "in-kernel" if (own1 and own2) else ("direct" if S <= hm.DIRECT_MAX else "align")}
    return res


def run_layer(cfg, copies, T, steps, warmup, block, breakdown=True):
    """Time `steps` layer calls (graph replays of len(copies) calls each)."""
    import torch

    from blackhole_runtime import hex_moe as hm
    dev = copies[0][0].lookup.device
    x, w, ids, logits = make_inputs(cfg, T, dev)
    n = len(copies)

    def layers(m):
        def fn():
            for tiers in copies[:m]:
                hm.hex_moe(x, w, ids, tiers, path="fused")
        return fn

    g = graph_of(layers(n))
    rem = steps % n                          # exactly `steps` layer calls: full replays + one partial
    g_rem = graph_of(layers(rem)) if rem else None
    warm_calls = warm(g, n, warmup)
    t0 = time.perf_counter()
    for _ in range(steps // n):
        g.replay()
    if g_rem is not None:
        g_rem.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    calls = steps
    ms = elapsed * 1e3 / calls
    total, glu_b, used = layer_bytes(cfg, copies[0], ids, block, T)
    S = T * cfg["k"]
    flops = 6.0 * S * cfg["H"] * cfg["I"]
    out = {"T": T, "steps": calls, "warmup_calls": warm_calls, "ms_per_step": ms, "tokens_per_s": T / (ms * 1e-3),
           "unique_experts": used,
           "layer_bytes": total, "hbm_gbps": total / (ms * 1e-3) / 1e9,
           "hbm_frac": total / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
           "mfma_frac": flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, "glu_bytes": glu_b}
    if T == 1:
        # the reference's one-token figure (hex_check.py:121,136): top-k routed experts x 3 x H x I
        # at 4.25 bits per weight (3.25 for a 3-bit tier), over the layer time
        bpw = sum(len(t._experts_host) * (t.bits + 0.25) for t in copies[0]) / cfg["E"]
        out["ref_t1_hex_weight_gbps"] = cfg["k"] * 3 * cfg["H"] * cfg["I"] * bpw / 8 / (ms * 1e-3) / 1e9
    if breakdown:
        out["kernels"] = kernel_breakdown(cfg, copies, x, w, ids, max(5, steps // (2 * n)))
    return out, (x, w, ids, logits)


def prefill_roofline(cfg, T, kernels):
    """Roofline entry of the dominant prefill kernel (the gate/up kernel over the whole tier):
    useful matrix flops per launch (4 S H I: gate and up) over its average launch time from HIP
    events, against the bf16 peak; with the counter-measured matrix-core busy fraction of the same
    kernel when its summary is in profiles/."""
    S = T * cfg["k"]
    flops = 4.0 * S * cfg["H"] * cfg["I"]
    us = kernels["glu_us"]
    tf = flops / (us * 1e-6) / 1e12
    busy = json.loads(MFMA_FILE.read_text()) if MFMA_FILE.exists() else None
    return {"bound": "mfma", "achieved": tf, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": tf / BF16_PEAK_TFLOPS, "kernel": f"{PREFILL_GLU_KERNEL} (gate/up + SiLU, 128-slot blocks)",
            "workload": f"config3 T={T}", "flops_per_launch": flops, "avg_launch_us": us,
            "down_us": kernels["down_us"], "plan_us": kernels["plan_us"],
            "mfma_busy_frac": busy["mfma_busy_frac"] if busy else None,
            "mfma_busy_source": str(MFMA_FILE.relative_to(ROOT)) if busy else None}


def cpu_threads() -> int:
    """Host threads this process may use: OMP_NUM_THREADS when set (the GPU box's CPU share),
    else the affinity mask."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    return int(env) if env.isdigit() and int(env) > 0 else len(os.sched_getaffinity(0))


def cpu_baseline(cfg, tiers, x, w, ids, budget_s=12.0):
    """The CPU oracle (numpy float32 restatement of hex_ref.moe_reference: dequant every routed
    expert, per-expert matmuls) on one layer call of the same workload with all host threads the
    process may use; calls repeat until budget_s of CPU work (at least 3), median reported."""
    import numpy as np

    from oracle import hex_oracle as O
    from threadpoolctl import threadpool_limits
    ref = []
    for t in tiers:
        parts = {}
        for proj in ("gate_proj", "up_proj", "down_proj"):
            p = getattr(t, proj)
            parts[proj] = {"idx": p["idx"].cpu().numpy().view(np.uint32), "block_scale": p["block_scale"].cpu().numpy(),
                           "expert_scale": p["expert_scale"].cpu().numpy(), "levels": p["levels"].cpu().numpy()}
        ref.append({"bits": t.bits, "experts": t._experts_host.numpy(), **parts})
    xn, wn, idn = x.float().cpu().numpy(), w.cpu().numpy(), ids.cpu().numpy()
    threads = cpu_threads()
    times = []
    with threadpool_limits(threads):
        t_start = time.perf_counter()
        while len(times) < 3 or (time.perf_counter() - t_start < budget_s and len(times) < 20):
            t0 = time.perf_counter()
            O.moe_reference(xn, wn, idn, ref, "bf16")
            times.append(time.perf_counter() - t0)
            log(f"  cpu baseline call {len(times)}: {times[-1]:.2f} s")
    med = float(np.median(times))
    model = "unknown CPU"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    T = ids.shape[0]
    return {"value": T / med, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{len(times)} calls of the oracle moe_reference (numpy float32, {threads} BLAS threads) on "
                      f"the benchmark layer at T={T} ({sum(times):.1f} s of CPU work), median {med:.3f} s per call, "
                      f"on {model}"}


# ----------------------------------------------------------------------------- rocprofv3 summaries

PROFILES = ROOT / "profiles"
TRAFFIC_FILE = PROFILES / "hex_moe_glu_config2_T16_traffic.json"
MFMA_FILE = PROFILES / "hex_gemm_glu_config3_T4096_mfma.json"
GLU_KERNEL = "hex_moe_kernel<4, 1, true, 1, 4, true>"      # gate/up, 4-bit, bf16, block_m 16, 128-input scales
PREFILL_GLU_KERNEL = "hex_gemm_kernel<3, 1, true, 4>"       # gate/up, 3-bit, bf16, 128-input scales
SIMDS = 1024                                                 # MI355X: 256 CUs x 4 SIMDs
XCDS = 8
COPY_BYTES = 2 * (128 << 20) * 2                             # the calibration kernel: 256 MiB read + 256 MiB written


def _csv_rows(d: str, suffix: str):
    import csv
    import glob
    for f in sorted(glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True)):
        with open(f) as fh:
            yield from csv.DictReader(fh)


def _short(name: str) -> str:
    name = name.replace("void ", "").split("(")[0]
    return name.replace("bh::", "")[:110]


def _kind(name: str) -> str:
    """Role of a dispatch in the decode layer: gate/up, down, sum, plan or other."""
    if "hex_moe_kernel<" in name:
        return "gate/up" if name.split("hex_moe_kernel<", 1)[1].split(",")[2].strip() == "true" else "down"
    if "gemv_glu_kernel" in name:
        return "gate/up"
    if "gemv_down_kernel" in name:
        return "down"
    if "moe_reduce_kernel" in name:
        return "sum"
    if "align" in name or "direct_kernel" in name:
        return "plan"
    return "other"


def layer_sequence(trace: list) -> list[str]:
    """The decode layer's dispatches as the timed graph replays them: every run of consecutive
    dispatches [plan,] gate/up, down[, sum] on one queue (the matrix-vector launches add the
    k-slot sum inside down); median duration of each kernel, the median gap before it, the median
    layer span (first start to last end) and the median period between consecutive layers."""
    import statistics
    rows = sorted(((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), _kind(r["Kernel_Name"]), _short(r["Kernel_Name"]))
                   for r in trace), key=lambda t: t[0])
    layers = []
    i = 0
    while i < len(rows) - 1:
        if rows[i][2] == "gate/up" and rows[i + 1][2] == "down":
            end = i + 3 if i + 2 < len(rows) and rows[i + 2][2] == "sum" else i + 2
            start = i - 1 if i > 0 and rows[i - 1][2] == "plan" else i
            layers.append(rows[start:end])
            i = end
        else:
            i += 1
    if not layers:
        return []
    kinds = " -> ".join(k for _, _, k, _ in layers[len(layers) // 2])
    out = [f"## decode layer as replayed: {len(layers)} runs of {kinds}",
           f"{'kernel':<60} {'role':>8} {'n':>6} {'avg_us':>8} {'med_us':>8} {'gap_before_us':>14}"]
    by = {}
    for seq in layers:
        for j, (st, en, kind, name) in enumerate(seq):
            gap = (st - seq[j - 1][1]) / 1e3 if j else float("nan")
            by.setdefault((kind, name), []).append(((en - st) / 1e3, gap))
    for (kind, name), v in by.items():
        d = [a for a, _ in v]
        g = [b for _, b in v if b == b]
        out.append(f"{name[:60]:<60} {kind:>8} {len(v):>6} {sum(d) / len(d):>8.2f} {statistics.median(d):>8.2f} "
                   f"{(statistics.median(g) if g else float('nan')):>14.2f}")
    spans = [(seq[-1][1] - seq[0][0]) / 1e3 for seq in layers]
    periods = [(b[0][0] - a[0][0]) / 1e3 for a, b in zip(layers, layers[1:])]
    out.append(f"layer span (first start to last end): median {statistics.median(spans):.2f} us, "
               f"mean {sum(spans) / len(spans):.2f} us")
    if periods:
        out.append(f"layer period (start to the next layer's start): median {statistics.median(periods):.2f} us")
    return out


def prefill_timeline(trace: list, last: int = 1) -> list[str]:
    """Every dispatch of the last `last` replayed prefill layers (the dispatches between two
    k-slot sums that include both prefill kernels), with queue, start and end in microseconds from
    the end of the previous layer's sum."""
    def role(n: str) -> str:
        for key, r in (("align_count", "count"), ("align_place", "place"), ("align_scatter", "scatter"),
                       ("align_kernel", "plan"), ("moe_reduce", "sum")):
            if key in n:
                return r
        if PREFILL_GLU_KERNEL.split("<")[0] in n:
            return "gate/up" if n.split("<", 1)[1].split(",")[2].strip() == "true" else "down"
        return ""
    rows = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), role(r["Kernel_Name"]), r.get("Queue_Id", ""))
                  for r in trace)
    rows = [r for r in rows if r[2]]
    sums = [i for i, r in enumerate(rows) if r[2] == "sum"]
    layers = [(a, b) for a, b in zip(sums, sums[1:])
              if {"gate/up", "down"} <= {r[2] for r in rows[a + 1:b]} and b - a < 40]
    out = []
    for a, b in layers[-last:]:
        t0 = rows[a][1]
        out.append(f"## prefill layer timeline ({b - a} dispatches, span {(rows[b][1] - t0) / 1e3:.1f} us after "
                   f"the previous sum)")
        for s0, e0, r, q in rows[a + 1:b + 1]:
            out.append(f"   {r:8s} q={q:>3s} start {(s0 - t0) / 1e3:8.1f} end {(e0 - t0) / 1e3:8.1f} "
                       f"dur {(e0 - s0) / 1e3:7.1f}")
    return out


def rocprof_summary(dirs: list[str]) -> str:
    """Text summary of rocprofv3 CSV output directories: per-kernel dispatch statistics from a
    --kernel-trace --stats run, mean counter values per dispatch from --pmc runs, and, when a
    FETCH_SIZE and a WRITE_SIZE run of the --copy-calibration bench are both given, the gate/up
    kernel's HBM traffic per launch scaled by what the same counters read for the known-size copy
    (written to TRAFFIC_FILE)."""
    out, counters = [], {}
    for d in dirs:
        trace = list(_csv_rows(d, "kernel_trace.csv"))
        out += layer_sequence(trace)
        out += prefill_timeline(trace)
        stats = list(_csv_rows(d, "kernel_stats.csv"))
        if stats:
            out.append(f"## kernel statistics ({d})")
            out.append(f"{'kernel':<112} {'calls':>6} {'avg_us':>9} {'min_us':>9} {'max_us':>9} {'pct':>6}")
            for r in sorted(stats, key=lambda r: -float(r["TotalDurationNs"]))[:16]:
                out.append(f"{_short(r['Name']):<112} {int(r['Calls']):>6} {float(r['AverageNs']) / 1e3:>9.2f} "
                           f"{float(r['MinNs']) / 1e3:>9.2f} {float(r['MaxNs']) / 1e3:>9.2f} "
                           f"{float(r['Percentage']):>6.2f}")
        rows = list(_csv_rows(d, "counter_collection.csv"))
        if rows:
            agg: dict = {}
            for r in rows:
                key = (_short(r["Kernel_Name"]), r["Counter_Name"])
                agg.setdefault(key, []).append(float(r["Counter_Value"]))
            out.append(f"## counters, mean per dispatch ({d})")
            for (k, c), v in sorted(agg.items()):
                if any(s in k for s in ("hex_moe", "hex_gemm", "gemv_", "align_", "moe_reduce", "bitwise_not")):
                    out.append(f"{k:<112} {c:<12} {sum(v) / len(v):>14.1f}  (n={len(v)})")
                counters.setdefault(c, {})[k] = v
    if "SQ_VALU_MFMA_BUSY_CYCLES" in counters and "GRBM_GUI_ACTIVE" in counters:
        # matrix-core busy fraction of the prefill gate/up kernel: busy cycles (summed over the
        # SIMDs) over SIMDs x the kernel's GPU-busy cycles (GRBM_GUI_ACTIVE sums the XCDs)
        busy = {k: v for k, v in counters["SQ_VALU_MFMA_BUSY_CYCLES"].items() if PREFILL_GLU_KERNEL in k}
        grbm = {k: v for k, v in counters["GRBM_GUI_ACTIVE"].items() if PREFILL_GLU_KERNEL in k}
        if busy and grbm:
            k = next(iter(busy))
            b = sum(busy[k]) / len(busy[k])
            gg = sum(grbm[k]) / len(grbm[k])
            res = {"kernel": k, "mfma_busy_cycles": b, "grbm_gui_active": gg, "simds": SIMDS, "xcds": XCDS,
                   "mfma_busy_frac": b / (SIMDS * gg / XCDS), "dispatches": len(busy[k])}
            out.append("## matrix-core busy fraction of the prefill gate/up kernel")
            out.append(json.dumps(res, indent=1))
            PROFILES.mkdir(exist_ok=True)
            MFMA_FILE.write_text(json.dumps(res) + "\n")
    if "FETCH_SIZE" in counters and "WRITE_SIZE" in counters:
        def kernel(c, pred):
            cand = {k: v for k, v in counters[c].items() if pred(k)}
            return max(cand.items(), key=lambda kv: sum(kv[1]) / len(kv[1])) if cand else (None, [])
        ck, cf = kernel("FETCH_SIZE", lambda k: "bitwise_not" in k)
        _, cw = kernel("WRITE_SIZE", lambda k: k == ck)
        gk, gf = kernel("FETCH_SIZE", lambda k: GLU_KERNEL in k)
        _, gw = kernel("WRITE_SIZE", lambda k: GLU_KERNEL in k)
        if ck and gk:
            half = COPY_BYTES // 2                           # bytes the calibration kernel reads, and writes
            f_scale = half / (sum(cf) / len(cf) * 1024)
            w_scale = half / (sum(cw) / len(cw) * 1024)
            fetch = sum(gf) / len(gf) * 1024 * f_scale
            write = sum(gw) / len(gw) * 1024 * w_scale
            res = {"kernel": gk, "fetch_bytes": fetch, "write_bytes": write, "traffic_bytes": fetch + write,
                   "calibration_kernel": ck, "calibration_fetch_kib": sum(cf) / len(cf),
                   "calibration_write_kib": sum(cw) / len(cw), "calibration_bytes_each_way": half,
                   "fetch_scale": f_scale, "write_scale": w_scale, "dispatches": len(gf)}
            out.append("## HBM traffic of the gate/up kernel per launch (counter KiB x 1024 x calibration scale)")
            out.append(json.dumps(res, indent=1))
            PROFILES.mkdir(exist_ok=True)
            TRAFFIC_FILE.write_text(json.dumps(res) + "\n")
    return "\n".join(out) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--config", type=int, default=2, choices=sorted(CONFIGS))
    ap.add_argument("--tokens", type=int, default=0, help="token batch (default: the config's)")
    ap.add_argument("--block", type=int, default=128, help="inputs per fp8 block scale (32 or 128)")
    ap.add_argument("--copies", type=int, default=8, help="resident layer copies the steps cycle through")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run bitwise_not over 128 Mi int16 elements, 3 times (the known-size kernel that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE into bytes)")
    ap.add_argument("--rocprof-summary", nargs="+", metavar="DIR",
                    help="summarise rocprofv3 CSV output directories and exit (no GPU work)")
    a = ap.parse_args(argv)
    if a.rocprof_summary:
        print(rocprof_summary(a.rocprof_summary), end="")
        return 0
    if a.gpus != 1:
        print(f"bench.py runs on one GPU: this build has no multi-GPU path (asked for --gpus {a.gpus})",
              file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    cfg = CONFIGS[a.config]
    T = a.tokens or cfg["T"]
    log(f"bench: {torch.cuda.get_device_name(dev)}; {cfg['name']}, T={T}, block {a.block}, {a.copies} copies")
    t0 = time.perf_counter()
    copies = build_tiers(cfg, a.block, a.copies, dev)
    log(f"  layers quantized and resident in {time.perf_counter() - t0:.1f} s")
    head, (x, w, ids, _) = run_layer(cfg, copies, T, a.steps, a.warmup, a.block)
    log(f"  T={T}: {head['ms_per_step'] * 1e3:.1f} us/layer, {head['tokens_per_s']:.0f} tok/s, "
        f"{head['hbm_gbps']:.0f} GB/s, kernels {head['kernels']}")

    k = head["kernels"]
    traffic, traffic_src = None, None
    if "glu_us" in k:
        glu_gbs = head["glu_bytes"] / (k["glu_us"] * 1e-6) / 1e9
        if a.config == 2 and T == 16 and a.block == 128 and TRAFFIC_FILE.exists():
            traffic = json.loads(TRAFFIC_FILE.read_text())["traffic_bytes"]
            traffic_src = str(TRAFFIC_FILE.relative_to(ROOT))
        roofline = {"bound": "hbm", "achieved": glu_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": glu_gbs / HBM_PEAK_GBS, "traffic": traffic, "traffic_source": traffic_src,
                    "kernel": f"{GLU_KERNEL} (gate/up + SiLU)", "algorithmic_bytes_per_launch": head["glu_bytes"],
                    "avg_launch_us": k["glu_us"]}
    else:   # the matrix-vector launches: the layer's bytes over the two launches' time
        gbs = head["layer_bytes"] / (k["gemv_us"] * 1e-6) / 1e9
        roofline = {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": gbs / HBM_PEAK_GBS, "traffic": None, "traffic_source": None,
                    "kernel": k["kernel"],
                    "algorithmic_bytes_per_launch": head["layer_bytes"], "avg_launch_us": k["gemv_us"]}

    sweep = {}
    roofline_prefill = None
    if not a.no_sweep and a.config == 2:
        for Ts in (1, 4, 64):
            r, _ = run_layer(cfg, copies, Ts, max(80, a.steps // 4), a.warmup, a.block, breakdown=False)
            sweep[f"T{Ts}"] = {kk: r[kk] for kk in ("ms_per_step", "tokens_per_s", "hbm_gbps", "hbm_frac",
                                                     "unique_experts", "ref_t1_hex_weight_gbps") if kk in r}
            log(f"  T={Ts}: {r['ms_per_step'] * 1e3:.1f} us/layer, {r['hbm_gbps']:.0f} GB/s")
        del copies
        torch.cuda.empty_cache()
        keys = ("ms_per_step", "tokens_per_s", "mfma_frac", "hbm_gbps", "hbm_frac", "unique_experts")
        # the other configs: (config, resident copies, token batches, timed calls per batch)
        for c, n_copies, batches, steps in ((3, 2, (4096,), 16), (4, 4, (256,), 100), (5, 8, (1, 16, 256, 2048, 8192), 32)):
            layers = build_tiers(CONFIGS[c], a.block, n_copies, dev)
            for Ts in batches:
                r, _ = run_layer(CONFIGS[c], layers, Ts, steps, a.warmup, a.block, breakdown=c == 3)
                sweep[f"config{c}_T{Ts}"] = {kk: r[kk] for kk in keys + ("ref_t1_hex_weight_gbps",) if kk in r}
                if c == 3:
                    roofline_prefill = prefill_roofline(CONFIGS[c], Ts, r["kernels"])
                log(f"  config{c} T={Ts}: {r['ms_per_step'] * 1e3:.1f} us/layer, {r['hbm_gbps']:.0f} GB/s "
                    f"({r['hbm_frac'] * 100:.1f}% of HBM), MFMA {r['mfma_frac'] * 100:.1f}% of bf16 peak")
            del layers
            torch.cuda.empty_cache()
        copies = None

    if a.copy_calibration:
        src = torch.empty(128 << 20, dtype=torch.int16, device=dev).random_()
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.bitwise_not(src, out=dst)  # a kernel used nowhere else: 256 MiB in, 256 MiB out
        torch.cuda.synchronize()
        log(f"  copy calibration: 3 x ({src.numel() * 2} bytes read + {dst.numel() * 2} written)")
        del src, dst

    cpu = None
    if not a.no_cpu_baseline:
        base = copies[0] if copies is not None else build_tiers(cfg, a.block, 1, dev)[0]
        cpu = cpu_baseline(cfg, base, x, w, ids)

    line = {
        "metric": "HEX MoE layer tokens/s; HBM GB/s @ decode b=16; MFMA util @ 4k prefill",
        "value": head["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": head["steps"],
        "warmup": a.warmup, "warmup_floor_s": WARMUP_FLOOR_S, "warmup_calls": head["warmup_calls"],
        "ms_per_step": head["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: seeded N(0,0.02) weights HEX-quantized on the GPU, bf16 N(0,1) activations, "
                "N(0,1) router logits through the softmax top-k kernel",
        "config": {"workload": f"{cfg['name']}, T={T} tokens, fp8 scale per {a.block} inputs, "
                               f"{a.copies} resident layer copies cycled", "experts": cfg["E"], "hidden": cfg["H"],
                   "moe_intermediate": cfg["I"], "top_k": cfg["k"], "bits": cfg["bits"], "block": a.block,
                   "tokens": T, "unique_experts": head["unique_experts"], "path": "fused"},
        "hbm_gbps_layer": head["hbm_gbps"], "hbm_frac_layer": head["hbm_frac"],
        "kernels_us": {kk: v for kk, v in k.items() if kk.endswith("_us")}, "tiles": k["tiles"],
        "roofline": roofline, "roofline_prefill": roofline_prefill, "cpu_baseline": cpu, "sweep": sweep,
        "gpu": torch.cuda.get_device_name(dev),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.path.insert(0, str(ROOT))
    raise SystemExit(main())
