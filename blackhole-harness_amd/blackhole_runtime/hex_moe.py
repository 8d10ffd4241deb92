"""HEX fused MoE on MI355X: the operator API of runtime/blackhole_runtime/hex_moe.py over HIP
kernels for gfx950 (libbh_hex.so, C ABI in include/bh_hex.h).

Same names, arguments and errors as the reference module, so the `blackhole-hex` vLLM plugin
(vllm_hex.py) and its callers use it unchanged:

    HexTier(bits, experts, gate_proj, up_proj, down_proj).prepare(num_experts)
    hex_moe(x, topk_weights, topk_ids, tiers, config=None, path="auto") -> [T, H] in x.dtype
    hex_moe_fused / hex_moe_dequant / dequant_all / align / direct / plan / default_config

Two ways through a layer, as in the reference (hex_moe.py:7-23):

fused   the HIP kernels: slot plan (direct for a handful of slots, else the align kernel), then
        per tier the gate/up kernel (SiLU fused) and the down kernel (top-k weight fused), then
        the k-slot sum. No host synchronisation, so a hipGraph (torch.cuda.graph) captures it.
dequant every expert decoded once by the dequant kernel into bf16/f16/f32 stacks, then one
        matrix product per routed expert (rocBLAS through torch). It is taken for float32
        activations (the fused kernels run the matrix cores in bf16/f16), for path="dequant", and
        by path="auto" at or above BLACKHOLE_HEX_DEQUANT_MIN slots outside graph capture when
        that variable is set. Unset, path="auto" keeps to the fused kernels at every batch: the
        reference switches at 1024 slots because its fused Triton kernel slows down at large
        batches, while here the prefill kernels take over there, and the dequant path measured
        15 ms per layer against 0.1-0.5 ms fused (config 2 at 128 and 1024 tokens, config 3).

Everything runs on the GPU; CPU tensors are refused (the reference's CPU route is its
Triton interpreter, whose role the tests give to the numpy oracle).
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field

import torch

from blackhole_runtime import _lib

PARTS = ("idx", "block_scale", "expert_scale", "levels")
PROJS = ("gate_proj", "up_proj", "down_proj")
HEX_BLOCK = 32     # inputs per bit stream (blackhole/anatomy/hex.py:44)

DIRECT_MAX = int(os.environ.get("BLACKHOLE_HEX_DIRECT_MAX", "32"))      # slots (hex_moe.py:260)
# slots from which path="auto" takes the dequant path (hex_moe.py:261); never unless set
DEQUANT_MIN = int(os.environ.get("BLACKHOLE_HEX_DEQUANT_MIN", str(1 << 62)))
PREFILL_MIN = 48     # slots per expert above which the fused path takes the 128-slot prefill kernels
PREFILL_MIN_LARGE = 35   # the same for expert matrices of 4M weights or more (config 5's 4096 x 1536)
PREFILL_LARGE = 1 << 22
DECODE16_MAX = 12    # slots per expert up to which the decode kernels take 16-slot blocks
# a single tier's experts run as SPLIT parts on as many streams through the prefill kernels (see
# hex_moe_fused); 1 or less keeps the tier whole. Two parts measured best: 409 / 412 / 413 us for
# 2 / 1 / 3 parts at config 3, 912 / 937 / 931 us at config 5 (T=2048; 16-wave 4-bit kernels).
SPLIT = int(os.environ.get("BLACKHOLE_HEX_SPLIT", "2"))
# slots up to which the decode kernels sort the slots by expert themselves (bh_hex_moe_*_ids), so
# no align launch precedes them (at most 1024; 0 always launches the align kernel)
KERNEL_PLAN_MAX = min(1024, int(os.environ.get("BLACKHOLE_HEX_KERNEL_PLAN_MAX", "1024")))
# A single tier's layer runs as two matrix-vector launches (bh_hex_moe_gemv: no plan, no
# workspace, the k-slot sum inside the down launch) at up to GEMV_MAX slots (0: never) while the
# weight bytes that slots sharing an expert read again stay within GEMV_EXTRA_MB: (slots -
# expected distinct experts) x one expert's bytes, with E (1 - (1 - k/E)^T) distinct experts
# under uniform routing. The matrix-vector launches read each slot's expert once per slot; the
# expert-block kernels read each routed expert once but pay a plan, a workspace exchange and a
# third launch. Measured (layer us, matrix-vector vs expert-block, top-8): 96 experts of 2048 x
# 768: T=6 34.6 vs 52.3, T=8 41.3 vs 57.3 (38 MB read again), T=10 50.9 vs 54.7 (58 MB), T=12 64.7
# vs 55.8 (81 MB); 128 experts of 4096 x 1536: T=4 72.2 vs 89.8 (28 MB), T=5 88.5 vs 92.0 (45 MB),
# T=6 105.7 vs 101.8 (66 MB).
GEMV_MAX = int(os.environ.get("BLACKHOLE_HEX_GEMV_MAX", "256"))
GEMV_EXTRA_MB = float(os.environ.get("BLACKHOLE_HEX_GEMV_EXTRA_MB", "62"))


def _n_in(p: dict, bits: int) -> int:
    return p["idx"].shape[-1] // bits * HEX_BLOCK


def _proj_struct(p: dict, bits: int) -> _lib.HexProj:
    idx, bs = p["idx"], p["block_scale"]
    n_in = _n_in(p, bits)
    nblk = bs.shape[-1]
    if nblk == 0 or n_in % nblk:
        raise ValueError(f"block_scale width {nblk} does not divide the input width {n_in}")
    return _lib.HexProj(idx.data_ptr(), bs.data_ptr(), p["expert_scale"].data_ptr(), p["levels"].data_ptr(),
                        idx.stride(0), idx.stride(1), bs.stride(0), bs.stride(1), n_in // nblk)


@dataclass
class HexTier:
    """One tier of a MoE layer: experts sharing one index width, stacked in the HEX layout
    (hex_moe.py:174-198). Each projection dict holds idx uint32 [n, out, in/32*bits],
    block_scale uint8 [n, out, in/B], expert_scale float32 [n], levels float32 [n, 2**bits]."""
    bits: int
    experts: torch.Tensor
    gate_proj: dict
    up_proj: dict
    down_proj: dict
    lookup: torch.Tensor | None = None
    _structs: dict = field(default_factory=dict, repr=False, compare=False)
    _experts_host: torch.Tensor | None = field(default=None, repr=False, compare=False)
    _expert_set: frozenset = field(default=frozenset(), repr=False, compare=False)
    # the tier's SPLIT parts by expert (views of the same tensors), for hex_moe_fused's streams
    _parts: list | None = field(default=None, repr=False, compare=False)
    _is_part: bool = field(default=False, repr=False, compare=False)
    _expert_bytes: int = field(default=0, repr=False, compare=False)   # one expert's parts, all projections

    def prepare(self, num_experts: int) -> "HexTier":
        """Kernel-ready views (uint32 words as int32, float32 scales and levels, contiguous) and
        the global -> tier-local expert map (-1 for experts of other tiers), as in the reference;
        also the C structs the kernels take."""
        if self.bits not in (3, 4):
            raise ValueError(f"HEX tiers are 3- or 4-bit, got {self.bits}")
        L = 1 << self.bits
        for name in PROJS:
            p = getattr(self, name)
            if p["idx"].dtype == torch.uint32:
                p["idx"] = p["idx"].view(torch.int32)
            p["expert_scale"] = p["expert_scale"].float().reshape(-1).contiguous()
            p["levels"] = p["levels"].float().contiguous()
            for k in ("idx", "block_scale"):
                p[k] = p[k].contiguous()
            if p["levels"].shape[-1] != L:
                raise ValueError(f"{name}: {p['levels'].shape[-1]} levels for a {self.bits}-bit tier")
        dev = self.gate_proj["idx"].device
        self._experts_host = self.experts.detach().to("cpu", torch.int64)
        self._expert_set = frozenset(self._experts_host.tolist())
        if self._experts_host.numel() and (int(self._experts_host.min()) < 0
                                           or int(self._experts_host.max()) >= num_experts):
            raise ValueError(f"tier expert ids must be in 0..{num_experts - 1}")
        lk = torch.full((num_experts,), -1, dtype=torch.int32, device=dev)
        lk[self.experts.to(dev).long()] = torch.arange(len(self.experts), dtype=torch.int32, device=dev)
        self.lookup = lk
        self.experts = self.experts.to(dev).to(torch.int32)
        self._structs = {name: _proj_struct(getattr(self, name), self.bits) for name in PROJS}
        n = len(self.experts)
        self._expert_bytes = sum(int(p["idx"][0].numel()) * 4 + int(p["block_scale"][0].numel()) * 1 + 4
                                 + int(p["levels"][0].numel()) * 4 for p in (getattr(self, q) for q in PROJS)) if n else 0
        if not self._is_part and SPLIT > 1 and n >= SPLIT:
            self._parts = [self._part(n * j // SPLIT, n * (j + 1) // SPLIT, num_experts) for j in range(SPLIT)]
        return self

    def _part(self, lo: int, hi: int, num_experts: int) -> "HexTier":
        """Experts lo..hi-1 of the tier as a tier of their own (views, no copies)."""
        sub = HexTier(self.bits, self.experts[lo:hi],
                      *[{q: v[lo:hi] for q, v in getattr(self, name).items()} for name in PROJS])
        sub._is_part = True
        return sub.prepare(num_experts)

    def struct(self, name: str) -> _lib.HexProj:
        s = self._structs.get(name)
        if s is None:
            raise ValueError("HexTier.prepare(num_experts) has not been called")
        return s


# --------------------------------------------------------------------------- slot plan


def _ids_arg(ids: torch.Tensor) -> tuple[torch.Tensor, int]:
    if ids.dtype not in (torch.int32, torch.int64):
        ids = ids.long()
    ids = ids.reshape(-1).contiguous()
    return ids, _lib.dtype_code(ids.dtype)


def align(ids: torch.Tensor, n: int, block_m: int, lookup: torch.Tensor | None = None, _chunked: bool = True
          ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Group slots by expert, each expert's run padded to block_m, without a host sync
    (hex_moe.py:201-222): sorted slot ids int32 [B * block_m] (S = padding), the expert of every
    block int32 [B] (-1 = unused), the padded length int32 [1]; B = ceil(S/block_m) + min(n, S).
    With a tier's lookup (int32 [n]) only that tier's slots are placed (bh_hex_align_tier).
    Above 4096 slots the slots are counted per 1024-slot chunk into a workspace
    (bh_hex_align_ws); _chunked=False takes the entry points without one."""
    lib = _lib.load()
    _lib.require_gpu(ids)
    ids, code = _ids_arg(ids)
    S = ids.numel()
    nb = lib.bh_hex_align_max_blocks(S, n, block_m)
    if nb < 0:
        raise ValueError(f"bad align sizes S={S} n={n} block_m={block_m}")
    dev = ids.device
    sid = torch.empty(nb * block_m, dtype=torch.int32, device=dev)
    eid = torch.empty(nb, dtype=torch.int32, device=dev)
    npp = torch.empty(1, dtype=torch.int32, device=dev)
    if lookup is not None and (lookup.dtype != torch.int32 or lookup.numel() != n or lookup.device != ids.device):
        raise ValueError(f"lookup must be int32 [{n}] on {ids.device}")
    nws = lib.bh_hex_align_workspace(S, n)
    if _chunked and nws > 0:
        ws = torch.empty(nws, dtype=torch.int32, device=dev)
        lk = None if lookup is None else lookup.contiguous().data_ptr()
        _lib.check(lib.bh_hex_align_ws(ids.data_ptr(), code, S, n, lk, block_m, ws.data_ptr(), nws, sid.data_ptr(),
                                       eid.data_ptr(), npp.data_ptr(), _lib.stream_of(ids)), "bh_hex_align_ws")
    elif lookup is None:
        _lib.check(lib.bh_hex_align(ids.data_ptr(), code, S, n, block_m, sid.data_ptr(), eid.data_ptr(),
                                    npp.data_ptr(), _lib.stream_of(ids)), "bh_hex_align")
    else:
        _lib.check(lib.bh_hex_align_tier(ids.data_ptr(), code, S, n, lookup.contiguous().data_ptr(), block_m,
                                         sid.data_ptr(), eid.data_ptr(), npp.data_ptr(), _lib.stream_of(ids)),
                   "bh_hex_align_tier")
    return sid, eid, npp


def direct(ids: torch.Tensor, block_m: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """One block per slot, no sorting (hex_moe.py:228-237). Same outputs as align()."""
    lib = _lib.load()
    _lib.require_gpu(ids)
    ids, code = _ids_arg(ids)
    S = ids.numel()
    dev = ids.device
    sid = torch.empty(S * block_m, dtype=torch.int32, device=dev)
    eid = torch.empty(S, dtype=torch.int32, device=dev)
    npp = torch.empty(1, dtype=torch.int32, device=dev)
    _lib.check(lib.bh_hex_direct(ids.data_ptr(), code, S, block_m, sid.data_ptr(), eid.data_ptr(), npp.data_ptr(),
                                 _lib.stream_of(ids)), "bh_hex_direct")
    return sid, eid, npp


def plan(ids: torch.Tensor, n: int, block_m: int, mode: str = "auto", lookup: torch.Tensor | None = None):
    """(sorted slot ids, block experts, padded length) for the fused kernels (hex_moe.py:248-257):
    direct for at most DIRECT_MAX slots (or mode="direct"), else the align kernel. The reference's
    "vllm" and "torch" modes name other sorts with the same outputs; both map to the align kernel.
    A tier's lookup restricts an aligned plan to that tier's slots (direct plans ignore it: the
    kernels skip other tiers' blocks)."""
    if mode not in ("auto", "direct", "vllm", "torch"):
        raise ValueError(f"unknown plan mode {mode!r}")
    if mode == "direct" or (mode == "auto" and ids.numel() <= DIRECT_MAX):
        return direct(ids, block_m)
    return align(ids, n, block_m, lookup)


# --------------------------------------------------------------------------- tiles


def _tile_from(cfg: dict) -> int:
    """block_m of a config dict: BLOCK_M (slots per expert block) rounded to 16, 32, 64 or 128
    (128: the prefill kernels). The reference's BLOCK_N, BLOCK_K, num_warps and num_stages have
    no counterpart here (the kernels fix their own output tiles and input steps) and are
    ignored."""
    bm = int(cfg.get("BLOCK_M", 16))
    return 16 if bm <= 16 else (32 if bm <= 32 else (64 if bm <= 64 else 128))


def _fit_tile(bm: int, n_in: int, n_out: int, glu: bool) -> int:
    """The prefill kernels (block_m 128) step through the inputs 128 at a time and write output
    rows (act and y, both in the activation dtype) 16 bytes at a time; other widths take the
    32-slot decode kernels."""
    return 32 if bm == 128 and (n_in % 128 or n_out % 8) else bm


def default_config(slots: int, n_out: int, n_in: int, glu: bool, n_experts: int = 0) -> dict:
    """Tile choice by slot count (hex_moe.py:264-283), or BLACKHOLE_HEX_TILES="BM". BLOCK_M grows
    with the slots each expert gets, so an expert's weights are streamed by few blocks. 64-slot
    blocks are never chosen by default: on MI355X their gate/up kernel spills registers and ran
    over twice as long as 32-slot blocks on config 4's batch. 16-slot blocks up to 12 slots per
    expert on average: at 16 (config 5, T=256) the experts that get more than 16 slots stream
    their weights twice, and 32-slot blocks measured 352 against 434 us; at 10.7 (config 2,
    T=128) the two tie, and at 5.3 (T=64) 16-slot blocks win, 91 against 97 us. The 128-slot
    prefill kernels above PREFILL_MIN (48) slots per expert, or above PREFILL_MIN_LARGE (35) for
    expert matrices of 4M weights or more (n_out x n_in), measured with the current kernels:
    config 5 (4096 x 1536) at 34 slots per expert 569 us on 32-slot blocks against 581 us, at 36
    632 against 584, at 38 651 against 587; config 2 (2048 x 768) at 40 158 against 173 us, at
    42.7 162 against 172, at 53.3 178 against 176, at 64 187 against 180."""
    env = os.environ.get("BLACKHOLE_HEX_TILES")
    if env:
        bm = _tile_from({"BLOCK_M": int(env.split(",")[0])})
    else:
        per_expert = slots / max(1, n_experts or slots)
        pmin = PREFILL_MIN_LARGE if n_out * n_in >= PREFILL_LARGE else PREFILL_MIN
        bm = 16 if per_expert <= DECODE16_MAX else (32 if per_expert <= pmin else 128)
    return {"BLOCK_M": _fit_tile(bm, n_in, n_out, glu), "BLOCK_N": 256}


# --------------------------------------------------------------------------- fused path

# Workspaces of the decode kernels: int32 arrival counters, which must be zero when a call
# starts and which every call leaves zero again, and float32 partial sums (no initial value).
#  * One workspace per (device, stream, kind): calls that may overlap in time (tiers on side
#    streams) never share one, and calls on one stream run in order.
#  * A buffer handed to a kernel is never freed. A hipGraph captured with it replays into it
#    for as long as the graph lives, so a workspace that has to grow takes new buffers and keeps
#    the old ones alive (_RETIRED). Graphs captured on one stream share its workspace and are
#    replayed in order, as a serving engine replays its graphs on one stream.
#  * Counters are slices of a per-device arena zeroed once, outside any capture, so a captured
#    call records no fill: every replay starts from the zeros the previous call left.
_ARENA_INTS = 1 << 22            # int32 counters per arena (16 MiB)
_SLICE_MIN = 1 << 16             # counters per workspace at least (so most never grow)
_ARENAS: dict = {}               # device index -> [zeroed int32 tensor, ints handed out]
_WORKSPACES: dict = {}           # (device index, stream, kind) -> (counters, partials)
_RETIRED: list = []              # replaced buffers, kept alive for the graphs that use them


def _zeroed_counters(device: torch.device, n: int) -> torch.Tensor:
    """n int32 counters that are zero now, from the device's arena. Outside capture an arena
    that is used up is replaced (its slices stay valid) and the host waits for its fill, so
    streams other than the current one see zeros. Inside capture with the arena used up the
    counters come from a captured fill (correct; the graph then replays one fill kernel)."""
    ar = _ARENAS.get(device.index)
    if ar is None or ar[0].numel() - ar[1] < n:
        if torch.cuda.is_current_stream_capturing():
            return torch.zeros(n, dtype=torch.int32, device=device)
        if ar is not None:
            _RETIRED.append(ar[0])
        ar = _ARENAS[device.index] = [torch.zeros(max(n, _ARENA_INTS), dtype=torch.int32, device=device), 0]
        torch.cuda.current_stream(device).synchronize()
    t = ar[0][ar[1]:ar[1] + n]
    ar[1] += -(-n // 64) * 64            # slices start on 256-byte boundaries
    return t


def _kept_workspace(kind: str, device: torch.device, n_counters: int, n_partials: int, min_partials: int):
    """(counters, partials) of the current stream for workspace `kind`, grown (never freed) to at
    least n_counters int32 and n_partials float32."""
    key = (device.index, torch.cuda.current_stream(device).cuda_stream, kind)
    cnt, part = _WORKSPACES.get(key, (None, None))
    if cnt is None or cnt.numel() < n_counters:
        if cnt is not None:
            _RETIRED.append(cnt)
        cnt = _zeroed_counters(device, max(n_counters, _SLICE_MIN))
    if part is None or part.numel() < n_partials:
        if part is not None:
            _RETIRED.append(part)
        part = torch.empty(max(n_partials, min_partials), dtype=torch.float32, device=device)
    _WORKSPACES[key] = (cnt, part)
    return cnt, part


def _workspace(device: torch.device, block_m: int, num_blocks: int, n_out: int, n_in: int, glu: bool):
    """(counters, partials) for one fused launch on the current stream (bh_hex_moe_workspace)."""
    lib = _lib.load()
    nc, npart = _lib.ctypes.c_int64(), _lib.ctypes.c_int64()
    _lib.check(lib.bh_hex_moe_workspace(num_blocks, n_out, n_in, block_m, int(glu), _lib.ctypes.byref(nc),
                                        _lib.ctypes.byref(npart)), "bh_hex_moe_workspace")
    return _kept_workspace("moe", device, nc.value, npart.value, 1 << 16)


_SIDE_STREAMS: dict = {}


def _side_stream(device: torch.device, i: int = 1) -> torch.cuda.Stream:
    """Side stream i of a device (default priority): it runs the launches of a layer's tier (or
    part of a tier) i."""
    s = _SIDE_STREAMS.get((device.index, i))
    if s is None:
        s = _SIDE_STREAMS[(device.index, i)] = torch.cuda.Stream(device)
    return s


def _launch_glu(x, act, t: HexTier, sid, eid, npp, S, a_div, bm):
    lib = _lib.load()
    n_out = t.gate_proj["idx"].shape[1]
    n_in = _n_in(t.gate_proj, t.bits)
    assert x.shape[1] == n_in, f"input width {x.shape[1]} != HEX width {n_in}"
    tile = _lib.HexTile(bm, 256, 1)
    cnt, part = _workspace(x.device, bm, eid.numel(), n_out, n_in, True)
    _lib.check(lib.bh_hex_moe_glu(
        x.data_ptr(), _lib.dtype_code(x.dtype), x.stride(0), act.data_ptr(), act.stride(0),
        t.struct("gate_proj"), t.struct("up_proj"), t.bits, n_out, n_in,
        sid.data_ptr(), eid.data_ptr(), eid.numel(), npp.data_ptr(), t.lookup.data_ptr(), t.lookup.numel(), S, a_div,
        tile, cnt.data_ptr(), cnt.numel(), part.data_ptr(), part.numel(), _lib.stream_of(x)), "bh_hex_moe_glu")


def _launch_glu_ids(x, act, t: HexTier, ids, code, S, a_div, bm):
    """The gate/up launch that sorts the slots itself (no align launch before it)."""
    lib = _lib.load()
    n_out = t.gate_proj["idx"].shape[1]
    n_in = _n_in(t.gate_proj, t.bits)
    assert x.shape[1] == n_in, f"input width {x.shape[1]} != HEX width {n_in}"
    tile = _lib.HexTile(bm, 256, 1)
    E = t.lookup.numel()
    cnt, part = _workspace(x.device, bm, lib.bh_hex_align_max_blocks(S, E, bm), n_out, n_in, True)
    _lib.check(lib.bh_hex_moe_glu_ids(
        x.data_ptr(), _lib.dtype_code(x.dtype), x.stride(0), act.data_ptr(), act.stride(0),
        t.struct("gate_proj"), t.struct("up_proj"), t.bits, n_out, n_in, ids.data_ptr(), code, t.lookup.data_ptr(), E,
        S, a_div, tile, cnt.data_ptr(), cnt.numel(), part.data_ptr(), part.numel(), _lib.stream_of(x)),
        "bh_hex_moe_glu_ids")


def _launch_down(act, y, t: HexTier, sid, eid, npp, S, w, bm):
    lib = _lib.load()
    n_out = t.down_proj["idx"].shape[1]
    n_in = _n_in(t.down_proj, t.bits)
    assert act.shape[1] == n_in, f"input width {act.shape[1]} != HEX width {n_in}"
    tile = _lib.HexTile(bm, 256, 1)
    cnt, part = _workspace(act.device, bm, eid.numel(), n_out, n_in, False)
    _lib.check(lib.bh_hex_moe_down(
        act.data_ptr(), _lib.dtype_code(act.dtype), act.stride(0), y.data_ptr(), _lib.dtype_code(y.dtype), y.stride(0),
        t.struct("down_proj"), t.bits, n_out, n_in,
        sid.data_ptr(), eid.data_ptr(), eid.numel(), npp.data_ptr(), t.lookup.data_ptr(), t.lookup.numel(), S,
        w.data_ptr(), tile, cnt.data_ptr(), cnt.numel(), part.data_ptr(), part.numel(), _lib.stream_of(act)),
        "bh_hex_moe_down")


def _launch_down_ids(act, y, t: HexTier, ids, code, S, w, bm):
    """The down launch that sorts the slots itself."""
    lib = _lib.load()
    n_out = t.down_proj["idx"].shape[1]
    n_in = _n_in(t.down_proj, t.bits)
    assert act.shape[1] == n_in, f"input width {act.shape[1]} != HEX width {n_in}"
    tile = _lib.HexTile(bm, 256, 1)
    E = t.lookup.numel()
    cnt, part = _workspace(act.device, bm, lib.bh_hex_align_max_blocks(S, E, bm), n_out, n_in, False)
    _lib.check(lib.bh_hex_moe_down_ids(
        act.data_ptr(), _lib.dtype_code(act.dtype), act.stride(0), y.data_ptr(), _lib.dtype_code(y.dtype), y.stride(0),
        t.struct("down_proj"), t.bits, n_out, n_in, ids.data_ptr(), code, t.lookup.data_ptr(), E, S, w.data_ptr(),
        tile, cnt.data_ptr(), cnt.numel(), part.data_ptr(), part.numel(), _lib.stream_of(act)), "bh_hex_moe_down_ids")


def gemv_fits(k: int, H: int, I: int) -> bool:
    """Whether bh_hex_moe_gemv takes a layer of these widths (its limits in include/bh_hex.h)."""
    return 0 < k <= 16 and H % HEX_BLOCK == 0 and I % HEX_BLOCK == 0 and H <= 4096 and I <= 2048


def gemv_prefer(T: int, k: int, H: int, I: int, tier: HexTier) -> bool:
    """Whether hex_moe_fused runs a single tier's layer of T tokens as the matrix-vector
    launches (see GEMV_MAX and GEMV_EXTRA_MB)."""
    S = T * k
    if not (0 < S <= GEMV_MAX and gemv_fits(k, H, I)):
        return False
    E = max(1, tier.lookup.numel())
    distinct = E * (1.0 - (1.0 - min(1.0, k / E)) ** T)
    return (S - distinct) * tier._expert_bytes <= GEMV_EXTRA_MB * 1e6


def hex_moe_gemv(x, topk_weights, topk_ids, tier: HexTier) -> torch.Tensor:
    """Routed-expert output [T, H] in x.dtype of one tier for a few tokens, as two matrix-vector
    launches (bh_hex_moe_gemv): gate/up for every slot, then down with the top-k weights and the
    k-slot sum (hex_moe.py:304-325 for such batches). Slots whose expert is not in the tier
    contribute nothing. Reads each routed expert's weights once per slot routed to it."""
    _lib.require_gpu(x, topk_weights, topk_ids)
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise NotImplementedError(f"the matrix-vector launches take bf16 or f16 activations, got {x.dtype}")
    T, k = topk_ids.shape
    H = x.shape[1]
    I = tier.gate_proj["idx"].shape[1]
    assert H == _n_in(tier.gate_proj, tier.bits), f"input width {H} != HEX width {_n_in(tier.gate_proj, tier.bits)}"
    if not gemv_fits(k, H, I):
        raise NotImplementedError(f"bh_hex_moe_gemv takes k <= 16, hidden <= 4096 and inter <= 2048 "
                                  f"(multiples of 32): got k={k}, hidden={H}, inter={I}")
    x = x.contiguous()
    out = torch.empty(T, H, dtype=x.dtype, device=x.device)
    if T == 0:
        return out
    ids, code = _ids_arg(topk_ids)
    w = topk_weights.reshape(-1).float().contiguous()
    act = torch.empty(T * k, I, dtype=x.dtype, device=x.device)
    lib = _lib.load()
    dt = _lib.dtype_code(x.dtype)
    _lib.check(lib.bh_hex_moe_gemv(
        x.data_ptr(), dt, x.stride(0), act.data_ptr(), act.stride(0), out.data_ptr(), dt, out.stride(0),
        tier.struct("gate_proj"), tier.struct("up_proj"), tier.struct("down_proj"), tier.bits, H, I, ids.data_ptr(),
        code, w.data_ptr(), tier.lookup.data_ptr(), tier.lookup.numel(), T, k, _lib.stream_of(x)), "bh_hex_moe_gemv")
    return out


def _covers_all(tiers: list[HexTier]) -> bool:
    """Whether every expert id has a tier (then every slot's y row is written by a kernel)."""
    seen: set = set()
    for t in tiers:
        if t._experts_host is None:
            raise ValueError("HexTier.prepare(num_experts) has not been called")
        seen |= t._expert_set
    return len(seen) == tiers[0].lookup.numel()


def hex_moe_fused(x, topk_weights, topk_ids, tiers: list[HexTier], config: dict | None = None,
                  align_mode: str = "auto") -> torch.Tensor:
    """Routed-expert output [T, H] in x.dtype through the fused HIP kernels (hex_moe.py:304-325).
    x bf16 or f16 [T, H]; topk_weights [T, k]; topk_ids int [T, k]; tiers prepared."""
    if not tiers:
        raise ValueError("no HEX tiers")
    _lib.require_gpu(x, topk_weights, topk_ids)
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise NotImplementedError(f"the fused HEX kernels take bf16 or f16 activations, got {x.dtype} "
                                  "(use path='dequant')")
    T, k = topk_ids.shape
    S = T * k
    H = x.shape[1]
    I = tiers[0].gate_proj["idx"].shape[1]
    E = tiers[0].lookup.numel()
    if len(tiers) == 1 and config is None and align_mode == "auto" and gemv_prefer(T, k, H, I, tiers[0]):
        return hex_moe_gemv(x, topk_weights, topk_ids, tiers[0])
    x = x.contiguous()
    out = torch.empty(T, H, dtype=x.dtype, device=x.device)
    if T == 0:
        return out
    flat = topk_ids.reshape(-1)
    w = topk_weights.reshape(-1).float().contiguous()
    act = torch.empty(S, I, dtype=x.dtype, device=x.device)
    c1 = config or default_config(S, I, H, True, E)
    c2 = config or default_config(S, H, I, False, E)
    bm1 = _fit_tile(_tile_from(c1), H, I, True)
    bm2 = _fit_tile(_tile_from(c2), I, H, False)
    # y per slot: float32 for the decode kernels; in x.dtype for the prefill kernels, as the
    # reference's y (hex_moe.py:316), which halves the y traffic of the down kernel and the sum
    # (16-bit y measured slower in the decode kernels, whose down stores each value separately:
    # config 2 T=16 62.1 -> 63.8 us, T=64 79.0 -> 80.7 us)
    ydt = x.dtype if bm2 == 128 else torch.float32
    y = (torch.empty if _covers_all(tiers) else torch.zeros)(S, H, dtype=ydt, device=x.device)

    # at most KERNEL_PLAN_MAX slots the decode kernels sort the slots themselves (with the tier's
    # lookup, so each tier's launches walk only its blocks) and no align launch precedes them
    ids_flat, ids_code = _ids_arg(flat)
    own1 = align_mode == "auto" and bm1 != 128 and S <= KERNEL_PLAN_MAX
    own2 = align_mode == "auto" and bm2 != 128 and S <= KERNEL_PLAN_MAX

    def run_tier(t: HexTier, lk: torch.Tensor | None) -> None:
        # one plan per tier when there are several, so each tier's launches walk only its blocks
        p1 = None if own1 else plan(flat, E, bm1, align_mode, lk)
        p2 = None if own2 else (p1 if (bm2 == bm1 and p1 is not None) else plan(flat, E, bm2, align_mode, lk))
        if own1:
            _launch_glu_ids(x, act, t, ids_flat, ids_code, S, k, bm1)
        else:
            _launch_glu(x, act, t, *p1, S, k, bm1)
        if own2:
            _launch_down_ids(act, y, t, ids_flat, ids_code, S, w, bm2)
        else:
            _launch_down(act, y, t, *p2, S, w, bm2)

    # Each slot is served by one tier, so the tiers write disjoint rows of act and y: each later
    # tier runs on a side stream of its own beside the first (each stream keeps its own
    # workspace), which overlaps one tier's ramp and tail with the other's streaming (config 4's
    # two tiers: 170 -> 144 us). Through the prefill kernels a single tier runs the same way as
    # its SPLIT parts by expert, so that one part's grid tail overlaps another's tiles (config 3,
    # two parts: 476 -> 465 us); the persistent decode kernels each fill the GPU, and parts of
    # them run one after the other (config 2, T=16: 71 -> 105 us; on 32-slot blocks config 2,
    # T=256: 119 -> 136 us), so a decode tier stays whole.
    # The caller's stream waits for the side streams before the k-slot sum.
    split = SPLIT > 1 and bm1 == 128 and bm2 == 128 and tiers[0]._parts
    chains = tiers if len(tiers) > 1 else (tiers[0]._parts if split else tiers)
    if len(chains) == 1:
        run_tier(chains[0], None)
    else:
        main = torch.cuda.current_stream(x.device)
        sides = [_side_stream(x.device, i) for i in range(1, len(chains))]
        for side, t in zip(sides, chains[1:]):
            side.wait_stream(main)
            with torch.cuda.stream(side):
                run_tier(t, t.lookup)
        run_tier(chains[0], chains[0].lookup)
        for side in sides:
            main.wait_stream(side)
    lib = _lib.load()
    _lib.check(lib.bh_hex_moe_reduce(y.data_ptr(), _lib.dtype_code(y.dtype), y.stride(0), ids_flat.data_ptr(), ids_code, E, T, k,
                                     H, out.data_ptr(), _lib.dtype_code(out.dtype), out.stride(0), _lib.stream_of(x)),
               "bh_hex_moe_reduce")
    return out


# --------------------------------------------------------------------------- dequant path


def hex_dequant(idx, block_scale, expert_scale, levels, bits: int, order: str = "R",
                dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Weights [n, out, in] from stacked HEX parts on the GPU, in the named association order:
    "R" level * (fp8 * es) (blackhole/anatomy/hex.py:180-204), "D" (level * fp8) * es (the
    reference's dequant kernel, hex_moe.py:163-164), "T" bf16(level * fp8) (its fused operand)."""
    lib = _lib.load()
    _lib.require_gpu(idx, block_scale, expert_scale, levels)
    idx = idx.view(torch.int32) if idx.dtype == torch.uint32 else idx
    n, n_out = idx.shape[0], idx.shape[1]
    p = {"idx": idx.contiguous(), "block_scale": block_scale.contiguous(),
         "expert_scale": expert_scale.float().reshape(-1).contiguous(), "levels": levels.float().contiguous()}
    n_in = _n_in(p, bits)
    out = torch.empty(n, n_out, n_in, dtype=dtype, device=idx.device)
    code = {"R": _lib.ORDER_R, "D": _lib.ORDER_D, "T": _lib.ORDER_T}[order]
    _lib.check(lib.bh_hex_dequant(_proj_struct(p, bits), bits, n, n_out, n_in, None, out.data_ptr(),
                                  _lib.dtype_code(dtype), out.stride(0), out.stride(1), 0, code,
                                  _lib.stream_of(idx)), "bh_hex_dequant")
    return out


def dequant_all(tiers: list[HexTier], dtype=torch.bfloat16, order: str = "D") -> tuple[torch.Tensor, torch.Tensor]:
    """All experts as stacks: w13 [E, 2I, H] (gate rows, then up) and w2 [E, H, I]
    (hex_moe.py:328-346), in the reference dequant kernel's order "D" by default."""
    lib = _lib.load()
    t0 = tiers[0]
    E = t0.lookup.numel()
    I = t0.gate_proj["idx"].shape[1]
    H = _n_in(t0.gate_proj, t0.bits)
    dev = t0.gate_proj["idx"].device
    w13 = torch.empty(E, 2 * I, H, dtype=dtype, device=dev)
    w2 = torch.empty(E, H, I, dtype=dtype, device=dev)
    code = {"R": _lib.ORDER_R, "D": _lib.ORDER_D, "T": _lib.ORDER_T}[order]
    st = _lib.stream_of(w13)
    for t in tiers:
        n = len(t.experts)
        for name, out, row_off in (("gate_proj", w13, 0), ("up_proj", w13, I), ("down_proj", w2, 0)):
            p = getattr(t, name)
            N, K = p["idx"].shape[1], _n_in(p, t.bits)
            _lib.check(lib.bh_hex_dequant(t.struct(name), t.bits, n, N, K, t.experts.data_ptr(), out.data_ptr(),
                                          _lib.dtype_code(dtype), out.stride(0), out.stride(1), row_off, code, st),
                       "bh_hex_dequant")
    return w13, w2


def hex_moe_dequant(x, topk_weights, topk_ids, tiers: list[HexTier]) -> torch.Tensor:
    """Routed-expert output [T, H]: every expert decoded once (dequant kernel), then per routed
    expert gate/up and down products in the weights' dtype (hex_moe.py:357-371; vLLM's bf16
    fused MoE is not part of this build, so the products go through torch's GEMM per expert).
    The activation is handed to the down product in x.dtype, as the reference's kernels do."""
    _lib.require_gpu(x, topk_weights, topk_ids)
    wdt = x.dtype if x.dtype in (torch.bfloat16, torch.float16) else torch.float32
    w13, w2 = dequant_all(tiers, wdt)
    T, k = topk_ids.shape
    I = w2.shape[-1]
    out = torch.zeros(T, x.shape[1], dtype=torch.float32, device=x.device)
    xw = x.to(wdt)
    ids = topk_ids.long()
    for e in torch.unique(ids).tolist():
        tok, slot = (ids == e).nonzero(as_tuple=True)
        h = torch.nn.functional.linear(xw[tok], w13[e]).float()
        a = (torch.nn.functional.silu(h[:, :I]) * h[:, I:]).to(x.dtype).to(wdt)
        out.index_add_(0, tok, torch.nn.functional.linear(a, w2[e]).float() * topk_weights[tok, slot, None].float())
    return out.to(x.dtype)


def hex_moe(x: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor, tiers: list[HexTier],
            config: dict | None = None, path: str = "auto") -> torch.Tensor:
    """Routed-expert output [T, H] of a SwiGLU MoE layer whose experts are HEX tiers (prepared)
    (hex_moe.py:374-382). path: "auto" (fused below DEQUANT_MIN slots, which is unbounded unless
    BLACKHOLE_HEX_DEQUANT_MIN is set, else dequant, never
    dequant while capturing a graph; float32 activations always dequant), "fused" or "dequant"."""
    if path not in ("auto", "fused", "dequant"):
        raise ValueError(f"unknown path {path!r}")
    capturing = x.is_cuda and torch.cuda.is_current_stream_capturing()
    if capturing and (path == "dequant" or (path == "auto" and x.dtype == torch.float32)):
        # the dequant path synchronises with the host (the routed experts are read back), which a
        # capture cannot record; the fused kernels, the ones a graph can hold, take bf16/f16 only
        raise NotImplementedError("the HEX dequant path cannot be captured in a graph: it reads the routed "
                                  f"experts back to the host (activations {x.dtype}; capture bf16 or f16 "
                                  "activations, which take the fused kernels)")
    if path == "dequant" or (path == "auto" and x.dtype == torch.float32) or (
            path == "auto" and config is None and not capturing and topk_ids.numel() >= DEQUANT_MIN):
        return hex_moe_dequant(x, topk_weights, topk_ids, tiers)
    return hex_moe_fused(x, topk_weights, topk_ids, tiers, config)


# --------------------------------------------------------------------------- routing


def _routing(scoring: str, renormalize: bool, n_group: int, topk_group: int, correction_bias, scale: float, E: int,
             device) -> tuple:
    """The bh_hex_routing struct of the options (and the bias tensor it points to)."""
    if scoring not in ("softmax", "sigmoid"):
        raise ValueError(f"scoring must be 'softmax' or 'sigmoid', got {scoring!r}")
    bias = None
    if correction_bias is not None:
        if correction_bias.device != device and torch.cuda.is_current_stream_capturing():
            raise ValueError("correction_bias must be on the GPU when the routing is captured in a graph "
                             "(a host tensor would be copied during capture)")
        bias = correction_bias.to(device=device, dtype=torch.float32).reshape(-1).contiguous()
        if bias.numel() != E:
            raise ValueError(f"correction_bias has {bias.numel()} values for {E} experts")
    r = _lib.Routing(_lib.SCORE_SIGMOID if scoring == "sigmoid" else _lib.SCORE_SOFTMAX, int(renormalize), int(n_group),
                     int(topk_group), float(scale), None if bias is None else bias.data_ptr())
    return r, bias


def route_select(logits: torch.Tensor, k: int, scoring: str = "softmax", renormalize: bool = True, n_group: int = 1,
                 topk_group: int = 0, correction_bias: torch.Tensor | None = None,
                 routed_scaling_factor: float = 1.0, ids_dtype: torch.dtype = torch.int64
                 ) -> tuple[torch.Tensor, torch.Tensor]:
    """Expert choice from router logits [T, E] on the GPU (reaper/reaper_pipeline/moe.py:141-168,
    route_from_logits): softmax top-k, or sigmoid scores plus correction_bias for the choice,
    group-limited by n_group / topk_group, unbiased weights; renormalised, then scaled.
    (weights float32 [T, k] in descending order of choice, ids [T, k])."""
    lib = _lib.load()
    _lib.require_gpu(logits)
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    T, E = logits.shape
    r, bias = _routing(scoring, renormalize, n_group, topk_group, correction_bias, routed_scaling_factor, E,
                       logits.device)
    w = torch.empty(T, k, dtype=torch.float32, device=logits.device)
    ids = torch.empty(T, k, dtype=ids_dtype, device=logits.device)
    _lib.check(lib.bh_hex_route_select(logits.data_ptr(), _lib.dtype_code(logits.dtype), logits.stride(0), T, E, k,
                                       r, w.data_ptr(), ids.data_ptr(), _lib.dtype_code(ids_dtype),
                                       _lib.stream_of(logits)), "bh_hex_route_select")
    return w, ids


def route(x: torch.Tensor, router_weight: torch.Tensor, k: int, scoring: str = "softmax", renormalize: bool = True,
          n_group: int = 1, topk_group: int = 0, correction_bias: torch.Tensor | None = None,
          routed_scaling_factor: float = 1.0, ids_dtype: torch.dtype = torch.int64
          ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Router logits x [T, H] @ router_weight [E, H]^T (the MoE block's gate linear, bf16/f16,
    rounded to x.dtype) and the expert choice of route_select, in one launch (bh_hex_route_gemm).
    Returns (weights float32 [T, k], ids [T, k], logits float32 [T, E])."""
    lib = _lib.load()
    _lib.require_gpu(x, router_weight)
    if x.dtype not in (torch.bfloat16, torch.float16) or router_weight.dtype != x.dtype:
        raise NotImplementedError("route takes bf16 or f16 activations and a router weight of the same dtype")
    x = x if x.stride(-1) == 1 and x.stride(0) % 8 == 0 else x.contiguous()
    wr = router_weight if router_weight.stride(-1) == 1 and router_weight.stride(0) % 8 == 0 else router_weight.contiguous()
    T, H = x.shape
    E = wr.shape[0]
    if wr.shape[1] != H:
        raise ValueError(f"router weight {tuple(wr.shape)} does not match hidden size {H}")
    r, bias = _routing(scoring, renormalize, n_group, topk_group, correction_bias, routed_scaling_factor, E, x.device)
    w = torch.empty(T, k, dtype=torch.float32, device=x.device)
    ids = torch.empty(T, k, dtype=ids_dtype, device=x.device)
    logits = torch.empty(T, E, dtype=torch.float32, device=x.device)
    cnt, _ = _kept_workspace("route", x.device, max(1, lib.bh_hex_route_gemm_workspace(T)), 0, 0)
    _lib.check(lib.bh_hex_route_gemm(x.data_ptr(), _lib.dtype_code(x.dtype), x.stride(0), wr.data_ptr(), wr.stride(0),
                                     T, H, E, k, r, logits.data_ptr(), logits.stride(0), w.data_ptr(), ids.data_ptr(),
                                     _lib.dtype_code(ids_dtype), cnt.data_ptr(), cnt.numel(), _lib.stream_of(x)),
               "bh_hex_route_gemm")
    return w, ids, logits


def moe_layer(x: torch.Tensor, router_weight: torch.Tensor, tiers: list[HexTier], k: int, **routing) -> torch.Tensor:
    """A routed-expert MoE layer from its router weight: route (router logits and expert choice,
    one launch), then hex_moe on the chosen experts. routing: route()'s options (scoring,
    renormalize, n_group, topk_group, correction_bias, routed_scaling_factor). The shared experts
    are not applied (as in the reference's plugin path, vllm_hex.py:145-146)."""
    w, ids, _ = route(x, router_weight, k, **routing)
    return hex_moe(x, w, ids, tiers)


def route_topk(logits: torch.Tensor, k: int, renormalize: bool = True,
               ids_dtype: torch.dtype = torch.int64) -> tuple[torch.Tensor, torch.Tensor]:
    """Softmax routing on the GPU (reaper/reaper_pipeline/moe.py:161-166, softmax branch):
    (weights float32 [T, k] in descending order, ids [T, k])."""
    lib = _lib.load()
    _lib.require_gpu(logits)
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    T, E = logits.shape
    w = torch.empty(T, k, dtype=torch.float32, device=logits.device)
    ids = torch.empty(T, k, dtype=ids_dtype, device=logits.device)
    _lib.check(lib.bh_hex_route_topk(logits.data_ptr(), _lib.dtype_code(logits.dtype), logits.stride(0), T, E, k,
                                     int(renormalize), w.data_ptr(), ids.data_ptr(), _lib.dtype_code(ids_dtype),
                                     _lib.stream_of(logits)), "bh_hex_route_topk")
    return w, ids
