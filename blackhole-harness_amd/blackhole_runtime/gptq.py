"""HEX producer with GPTQ rounding onto each expert's level table (torch; GPU or CPU tensors).

The parts the pipeline's hexvllm stage writes for a stack of expert matrices
(harness/blackhole_pipeline/stages/hexvllm.py:75-96, hex_parts), from the weights W [n, out, in]
and each expert's input Hessian H [n, in, in] (the sum of x x^T over the tokens routed to it):

  header     expert scale es = max|W| / 448; per 32-input block an fp8 e4m3 scale of the block's
             max|w| / es, rounded to nearest even (reaper/gpu_perf/headers.py:43-55)
  levels     L sorted levels per expert: Lloyd k-means on the block-normalised weights, started
             at quantiles, each value weighted by its input channel's Hessian diagonal times its
             block scale squared (error in weight units), 20 rounds, a seeded sample of 2^17
             values when there are more (headers.py:66-83, 96-103)
  rounding   GPTQ (Frantar et al. 2022) onto the table: columns in order, each rounded to the
             nearest level of its scaled table, its error spread over the later columns through
             the upper Cholesky factor of H^-1, with lazy updates per 128 columns; dead columns
             (zero weights or no activation) stay zero; the damping grows until both Cholesky
             factorisations succeed (reaper/gpu_perf/gptq.py:36-83, 134-141)
  packing    table indices, fp8 block codes and the HEX bit stream
             (harness/blackhole_pipeline/pack.py:53-86, 104-110)

The arithmetic (float32 sweeps, float64 factorisations, the order of every reduction on the
CPU) follows those files so that, on CPU tensors, the parts equal the reference's bit for bit.
On device tensors the block header (bh_hex_block_header), the k-means (bh_hex_fit_levels, each
level's sums in sample order as the CPU's scatter_add) and the column sweep with the table indices
(bh_hex_gptq_sweep, one lane per weight row) run in this library's HIP kernels, which repeat the
CPU's arithmetic operation for operation (IEEE divides, the same products and sums in the same
order, the CPU matrix product's fused multiply-add chain): on the same inputs they equal the
reference's outputs bit for bit. The damped Hessian factorisations stay torch float64 on the
device; their float32 cast equals the CPU's except where a value sits within float64 rounding of a
float32 midpoint. The GPU's batched float64 Cholesky has returned wrong factors with a success code
here, so every device factorisation is checked by its residual and the failing problems are
factorised again on the CPU.
"""

from __future__ import annotations

import torch

from . import _lib
from .quant import FP8_MAX, HEX_BLOCK, pack


def block_headers(W: torch.Tensor, block: int = HEX_BLOCK):
    """(block-normalised values [n, out, in/block, block] in [-1, 1], dequant block scales
    [n, out, in/block, 1], expert scales [n]) of W [n, out, in] (in a multiple of block)."""
    n, out, inp = W.shape
    if inp % block:
        raise ValueError(f"input width {inp} is not a multiple of the block {block}")
    x = W.float().view(n, out, inp // block, block)
    amax = x.abs().amax(-1, keepdim=True)
    es = (amax.amax(dim=(1, 2, 3), keepdim=True) / FP8_MAX).clamp(min=1e-30)
    blk = (amax / es).clamp(max=FP8_MAX).to(torch.float8_e4m3fn).float() * es
    blk = torch.where(blk > 0, blk, torch.ones_like(blk))
    return (x / blk).clamp(-1, 1), blk, es.reshape(n)


def fit_levels(xn: torch.Tensor, wt: torch.Tensor | None, L: int, iters: int = 20, sample: int = 1 << 17,
               seed: int = 0) -> torch.Tensor:
    """Sorted levels [n, L]: weighted 1-D Lloyd k-means per row of xn [n, N] (weights wt [n, N]),
    started at the L inner quantiles; a seeded sample of `sample` columns when N is larger (the
    draw comes from a CPU generator, so it is the same on every device)."""
    n, N = xn.shape
    if N > sample:
        g = torch.Generator(device="cpu").manual_seed(seed)
        pick = torch.randint(0, N, (sample,), generator=g).to(xn.device)
        xn = xn[:, pick]
        wt = wt[:, pick] if wt is not None else None
    w = wt if wt is not None else torch.ones_like(xn)
    q = torch.linspace(0, 1, L + 2, device=xn.device)[1:-1]
    lev = torch.quantile(xn.float(), q, dim=1).T.contiguous()
    for _ in range(iters):
        mids = (lev[:, 1:] + lev[:, :-1]) / 2
        a = torch.searchsorted(mids.contiguous(), xn.contiguous())
        num = torch.zeros(n, L, device=xn.device).scatter_add_(1, a, xn * w)
        den = torch.zeros(n, L, device=xn.device).scatter_add_(1, a, w)
        lev = torch.where(den > 0, num / den.clamp(min=1e-30), lev)
        lev = lev.sort(1).values
    return lev


def nearest_index(x: torch.Tensor, levels: torch.Tensor) -> torch.Tensor:
    """Index of the nearest of each row's sorted levels [n, L] for x [n, ...] (midpoint search)."""
    n = x.shape[0]
    mids = (levels[:, 1:] + levels[:, :-1]) / 2
    return torch.searchsorted(mids.contiguous(), x.reshape(n, -1).contiguous()).view(x.shape)


def _checked(A: torch.Tensor, F: torch.Tensor, info: torch.Tensor, residual, redo):
    """On a GPU, replace the factors of problems whose residual(F) against A exceeds 1e-9 of
    max|A| by redo(A on the CPU): the device's batched float64 Cholesky has returned wrong factors
    with a zero info code on this platform."""
    if A.device.type == "cpu":
        return F, info
    bad = (info == 0) & (residual(F) > 1e-9 * A.abs().amax(dim=(-2, -1)))
    if bad.any():
        Fc, ic = redo(A[bad].cpu())
        F[bad] = Fc.to(F.device)
        info[bad] = ic.to(info.device)
    return F, info


def _cholesky(A: torch.Tensor, upper: bool = False):
    """Batched float64 Cholesky factor (lower, or upper) with per-problem info, checked by
    max|F F^T - A| (or F^T F) on a GPU."""
    F, info = torch.linalg.cholesky_ex(A, upper=upper)
    mt = lambda x: x.transpose(-1, -2)                                            # noqa: E731
    res = (lambda F_: (mt(F_) @ F_ - A).abs().amax(dim=(-2, -1))) if upper else \
        (lambda F_: (F_ @ mt(F_) - A).abs().amax(dim=(-2, -1)))
    return _checked(A, F, info, res, lambda a: torch.linalg.cholesky_ex(a, upper=upper))


def _inverse_from_factor(L: torch.Tensor, A: torch.Tensor) -> torch.Tensor:
    """A^-1 from its lower factor L, checked by max|A^-1 A - I| on a GPU."""
    Ci = torch.cholesky_inverse(L)
    eye = torch.eye(A.shape[-1], dtype=A.dtype, device=A.device)
    Ci, _ = _checked(A, Ci, torch.zeros(A.shape[0], dtype=torch.int32, device=A.device),
                     lambda C: (C @ A - eye).abs().amax(dim=(-2, -1)) * A.abs().amax(dim=(-2, -1)),
                     lambda a: (torch.cholesky_inverse(torch.linalg.cholesky_ex(a)[0]),
                                torch.zeros(a.shape[0], dtype=torch.int32)))
    return Ci


def hessian_factor(W: torch.Tensor, H: torch.Tensor, damp: float = 0.01):
    """(W with dead columns zeroed, float32 upper Cholesky factor of the damped H^-1 [n, in, in],
    dead columns [n, in]). An expert with an all-zero Hessian is rounded plainly (H = I); a column
    is dead when its weights are all zero or its channel is never active. The damping, a
    fraction of the mean live diagonal, triples for a problem until both factorisations succeed."""
    W = W.float().clone()
    H = H.double().clone()
    n, _, m = W.shape
    eye = torch.eye(m, dtype=H.dtype, device=H.device)
    H[(H.diagonal(dim1=1, dim2=2) == 0).all(1)] = eye
    dead = (H.diagonal(dim1=1, dim2=2) == 0) | (W.abs().amax(1) == 0)
    live = (~dead).to(H.dtype)
    H = H * live[:, :, None] * live[:, None, :] + eye * dead.to(H.dtype)[:, :, None]
    W = W * (~dead)[:, None, :]
    diag = H.diagonal(dim1=1, dim2=2)
    base = (diag * live).sum(1) / live.sum(1).clamp(min=1)
    base = torch.where(base > 0, base, torch.ones_like(base))
    d = torch.full((n,), damp, dtype=H.dtype, device=H.device)
    for _ in range(6):
        Hd = H + (d * base)[:, None, None] * eye
        Lc, info = _cholesky(Hd)
        U, info2 = _cholesky(_inverse_from_factor(Lc, Hd), upper=True)
        bad = (info != 0) | (info2 != 0) | ~torch.isfinite(U).all(-1).all(-1)
        if not bad.any():
            return W, U.float(), dead
        d = torch.where(bad, d * 3, d)
    raise RuntimeError("GPTQ: Hessian not positive definite even with heavy damping")


def gptq_sweep(W: torch.Tensor, U: torch.Tensor, round_col, block: int = 128) -> torch.Tensor:
    """The GPTQ column sweep over W [n, out, in] with the factor U [n, in, in]: column c is rounded
    by round_col(values [n, out, 1], c), its error divided by U[c, c] is pushed onto the rest of its
    128-column block at once and onto the later blocks when the block ends. Returns Q."""
    m = W.shape[-1]
    Q = torch.zeros_like(W)
    for b0 in range(0, m, block):
        b1 = min(b0 + block, m)
        Wb = W[..., b0:b1].clone()
        Eb = torch.zeros_like(Wb)
        Ub = U[:, b0:b1, b0:b1]
        for j in range(b1 - b0):
            q = round_col(Wb[..., j:j + 1], b0 + j)
            Q[..., b0 + j:b0 + j + 1] = q
            e = (Wb[..., j:j + 1] - q) / Ub[:, j, j][:, None, None]
            Wb[..., j:] -= e @ Ub[:, j:j + 1, j:]
            Eb[..., j:j + 1] = e
        W[..., b1:] -= Eb @ U[:, b0:b1, b1:]
    return Q


def _ptr(t: torch.Tensor | None):
    return t.data_ptr() if t is not None else None


@torch.no_grad()
def block_headers_device(W: torch.Tensor, block: int = HEX_BLOCK, col_weight: torch.Tensor | None = None):
    """The block header on the GPU (bh_hex_block_header): (xn [n, out, in] in [-1, 1], dequant
    scales [n, out, in / block], fp8 block codes uint8 [n, out, in / block], expert scales [n],
    k-means weights [n, out, in] = col_weight[col] * scale^2 or None). Equal to block_headers and
    the reference's expert_scale / block_codes on the CPU bit for bit."""
    _lib.require_gpu(W, col_weight)
    n, out, inp = W.shape
    if inp % block:
        raise ValueError(f"input width {inp} is not a multiple of the block {block}")
    w = W.float().contiguous()
    cw = col_weight.float().contiguous() if col_weight is not None else None
    if cw is not None and cw.shape != (n, inp):
        raise ValueError(f"col_weight must be [n, in] = {(n, inp)}, got {tuple(cw.shape)}")
    xn = torch.empty_like(w)
    scale = torch.empty(n, out, inp // block, dtype=torch.float32, device=w.device)
    codes = torch.empty(n, out, inp // block, dtype=torch.uint8, device=w.device)
    es = torch.empty(n, dtype=torch.float32, device=w.device)
    wt = torch.empty_like(w) if cw is not None else None
    lib = _lib.load()
    _lib.check(lib.bh_hex_block_header(w.data_ptr(), n, out, inp, block, _ptr(cw), xn.data_ptr(), scale.data_ptr(),
                                       codes.data_ptr(), _ptr(wt), es.data_ptr(), _lib.stream_of(w)),
               "bh_hex_block_header")
    return xn, scale, codes, es, wt


@torch.no_grad()
def fit_levels_device(xn: torch.Tensor, wt: torch.Tensor | None, L: int, iters: int = 20, sample: int = 1 << 17,
                      seed: int = 0) -> torch.Tensor:
    """fit_levels on the GPU (bh_hex_fit_levels): the same seeded sample (drawn from a CPU
    generator), the quantile start from the sorted sample (sorting is exact) with the ranks formed
    on the CPU as the reference's CPU run forms them, and the Lloyd rounds in the kernel. Equal to
    fit_levels on the CPU bit for bit."""
    _lib.require_gpu(xn, wt)
    n, N = xn.shape
    dev = xn.device
    g = torch.Generator(device="cpu").manual_seed(seed)
    if N > sample:
        pick = torch.randint(0, N, (sample,), generator=g).to(dev)
        xs = xn[:, pick]
        ws = wt[:, pick] if wt is not None else None
    else:
        xs, ws = xn, wt
    xs = xs.float().contiguous()
    ws = ws.float().contiguous() if ws is not None else torch.ones_like(xs)
    S = xs.shape[1]
    q = torch.linspace(0, 1, L + 2)[1:-1]                 # float32 on the CPU
    ranks = q * (S - 1)
    lo, hi = ranks.long(), ranks.ceil().long()
    frac = (ranks - lo).float().contiguous().to(dev)
    srt = xs.sort(1).values
    q_lo = srt[:, lo.to(dev)].contiguous()
    q_hi = srt[:, hi.to(dev)].contiguous()
    levels = torch.empty(n, L, dtype=torch.float32, device=dev)
    lib = _lib.load()
    _lib.check(lib.bh_hex_fit_levels(xs.data_ptr(), ws.data_ptr(), n, S, L, q_lo.data_ptr(), q_hi.data_ptr(),
                                     frac.data_ptr(), iters, levels.data_ptr(), _lib.stream_of(xs)), "bh_hex_fit_levels")
    return levels


@torch.no_grad()
def sweep_device(W: torch.Tensor, U: torch.Tensor, levels: torch.Tensor, block_scale: torch.Tensor,
                 scale_block: int = HEX_BLOCK, dead: torch.Tensor | None = None, block: int = 128):
    """The GPTQ sweep and the table indices on the GPU (bh_hex_gptq_sweep): W [n, out, in] with
    dead columns zeroed, U [n, in, in] the upper factor, levels [n, L] sorted, block_scale
    [n, out, in / scale_block] the dequant scales, dead [n, in] bool or None. Returns (Q float32
    [n, out, in] with dead columns zeroed, codes uint8 [n, out, in]), equal to gptq_sweep +
    nearest_index on the CPU bit for bit."""
    _lib.require_gpu(W, U, levels, block_scale, dead)
    n, out, inp = W.shape
    L = levels.shape[-1]
    w = W.float().contiguous().clone()
    u = U.float().contiguous()
    lev = levels.float().contiguous()
    sc = block_scale.float().contiguous()
    if sc.shape != (n, out, inp // scale_block) or u.shape != (n, inp, inp) or lev.shape != (n, L):
        raise ValueError(f"shapes: W {tuple(W.shape)}, U {tuple(u.shape)}, levels {tuple(lev.shape)}, "
                         f"block_scale {tuple(sc.shape)} (scale block {scale_block})")
    d = dead.to(torch.uint8).contiguous() if dead is not None else None
    q = torch.empty_like(w)
    codes = torch.empty(w.shape, dtype=torch.uint8, device=w.device)
    lib = _lib.load()
    _lib.check(lib.bh_hex_gptq_sweep(w.data_ptr(), u.data_ptr(), lev.data_ptr(), L, sc.data_ptr(), scale_block,
                                     d.data_ptr() if d is not None else None, n, out, inp, block, q.data_ptr(),
                                     codes.data_ptr(), _lib.stream_of(w)), "bh_hex_gptq_sweep")
    return q, codes


@torch.no_grad()
def quantize_experts_gptq(W: torch.Tensor, H: torch.Tensor, L: int = 16, block: int = HEX_BLOCK,
                          damp: float = 0.01, sweep_block: int = 128) -> dict:
    """HEX parts of W [n, out, in] with GPTQ rounding under the Hessians H [n, in, in]:
    {"idx" int32 [n, out, in/32*bits], "block_scale" uint8 [n, out, in/block], "expert_scale"
    float32 [n], "levels" float32 [n, L], "q" float32 [n, out, in] (the rounded weights)}."""
    if W.dim() != 3 or H.dim() != 3 or H.shape != (W.shape[0], W.shape[2], W.shape[2]):
        raise ValueError(f"W [n, out, in] and H [n, in, in] expected, got {tuple(W.shape)} and {tuple(H.shape)}")
    bits = int(L).bit_length() - 1
    if L != 1 << bits or bits not in (3, 4):
        raise ValueError("HEX tables have 8 or 16 levels")
    if block % HEX_BLOCK:
        raise ValueError(f"the scale block must be a multiple of {HEX_BLOCK}")
    n, out, inp = W.shape
    if W.is_cuda:
        # header, k-means and sweep in this library's kernels; the factorisations in torch
        cw = H.diagonal(dim1=-2, dim2=-1).float().contiguous()
        xn, bscale, bcodes, es_w, wt = block_headers_device(W, block, cw)
        levels = fit_levels_device(xn.reshape(n, -1), wt.reshape(n, -1), L)
        Wd, U, dead = hessian_factor(W, H, damp)
        Q, codes = sweep_device(Wd, U, levels, bscale, block, dead, sweep_block)
        return {"idx": pack(codes, bits), "block_scale": bcodes, "expert_scale": es_w, "levels": levels, "q": Q}
    xn, blk, es = block_headers(W, block)
    cw = H.diagonal(dim1=-2, dim2=-1).float().view(n, 1, inp // block, block)
    wt = (cw.expand(n, out, -1, -1) * blk.pow(2)).reshape(n, -1)
    levels = fit_levels(xn.reshape(n, -1), wt, L).contiguous().float()
    scale = blk.expand(-1, -1, -1, block).reshape(n, out, inp)        # per-element dequant scale

    def round_col(x: torch.Tensor, c: int) -> torch.Tensor:
        s = scale[..., c:c + 1]
        return torch.gather(levels, 1, nearest_index((x / s).clamp(-1, 1), levels).reshape(n, -1)).view(x.shape) * s

    Wd, U, dead = hessian_factor(W, H, damp)
    Q = gptq_sweep(Wd, U, round_col, sweep_block) * (~dead)[:, None, :]
    codes = nearest_index((Q / scale).clamp(-1, 1), levels)
    es_w = (W.float().abs().amax(dim=(1, 2)) / FP8_MAX).clamp(min=1e-30)
    bs = (blk[..., 0] / es_w[:, None, None]).clamp(max=FP8_MAX).to(torch.float8_e4m3fn).view(torch.uint8)
    return {"idx": pack(codes, bits), "block_scale": bs.contiguous(), "expert_scale": es_w.float().contiguous(),
            "levels": levels, "q": Q}
