"""The HEX producer with GPTQ rounding on the GPU (marked gpu).

The block header (bh_hex_block_header), the weighted k-means (bh_hex_fit_levels) and the column
sweep with the table indices (bh_hex_gptq_sweep) run in HIP kernels; the damped Hessian
factorisations are torch float64 on the device. Each kernel equals its CPU statement bit for bit:
the header on every fp8 rounding region (subnormal scales, ties, zero blocks) and both block
sizes, the k-means with and without the seeded sample, the sweep on multi-block shapes (lazy
updates of later blocks, tail chunks, partial waves, 8 and 16 levels, other scale and sweep
blocks, dead columns) and, given the reference's own header, levels and factor, on the golden
vectors the reference wrote. The whole producer on the device equals those golden vectors bit for
bit (scales, codes, levels, indices and Q). On a config-2-width stack (4 experts, 768 x 2048)
GPTQ's layer error is below plain rounding's, and the parts run through the fused kernels."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from blackhole_runtime import gptq
from oracle import hex_oracle as O

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import make_golden_gptq as G  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLD = np.load(Path(__file__).resolve().parent / "golden" / "gptq.npz")


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def layer_err(W, Q, H):
    d = (W - Q).double()
    return torch.einsum("eoi,eij,eoj->e", d, H.double(), d)


@pytest.mark.parametrize("case", G.CASES, ids=[c[0] for c in G.CASES])
def test_gptq_on_gpu_matches_reference(case):
    name, n, o, i, L, tokens, seed = case
    say(f"gptq on the GPU, case {name}")
    W, H = G.make_case(name, n, o, i, tokens, seed)
    got = gptq.quantize_experts_gptq(torch.from_numpy(W).to(DEV), torch.from_numpy(H).to(DEV), L)
    # header, k-means, sweep and indices in the HIP kernels: every part equals the reference's
    assert np.array_equal(got["expert_scale"].cpu().numpy(), GOLD[f"{name}__expert_scale"])
    assert np.array_equal(got["block_scale"].cpu().numpy(), GOLD[f"{name}__block_scale"])
    assert np.array_equal(got["levels"].cpu().numpy(), GOLD[f"{name}__levels"])
    assert np.array_equal(got["idx"].cpu().numpy(), GOLD[f"{name}__idx"])
    assert np.array_equal(got["q"].cpu().numpy().view(np.uint32), GOLD[f"{name}__q"].view(np.uint32))


@pytest.mark.parametrize("block", [32, 128])
def test_header_kernel_bit_exact(block):
    """Expert scale, block scales, fp8 codes, normalised values and k-means weights against the CPU
    statement (block_headers and the reference's block_codes): weights spanning the fp8 range, a
    zero block, a block of fp8-subnormal scale and values on fp8 rounding ties."""
    say(f"block header kernel, block {block}")
    g = torch.Generator().manual_seed(block)
    n, o, i = 3, 40, 512
    W = torch.randn(n, o, i, generator=g) * torch.logspace(-6, 0, i)[None, None, :] * 0.05
    W[0, 3, :block] = 0.0                                  # a zero block
    W[1, 5, :block] *= 1e-4                                # an fp8-subnormal block scale
    es = W.abs().amax(dim=(1, 2)) / 448.0
    ties = torch.tensor([0.0029296875, 1.0625, 2.125, 17.0, 0.009765625]) * 1.0  # fp8 midpoints
    W[2, 7, :5] = ties * es[2]
    cw = torch.rand(n, i, generator=g) * 10
    xn, blk, es_c = gptq.block_headers(W, block)
    wt_c = (cw.view(n, 1, i // block, block).expand(n, o, -1, -1) * blk.pow(2)).reshape(n, o, i)
    codes_c = (blk[..., 0] / es_c[:, None, None]).clamp(max=448).to(torch.float8_e4m3fn).view(torch.uint8)
    xn_d, sc_d, co_d, es_d, wt_d = gptq.block_headers_device(W.to(DEV), block, cw.to(DEV))
    assert torch.equal(es_d.cpu(), es_c)
    assert torch.equal(sc_d.cpu(), blk[..., 0])
    assert torch.equal(co_d.cpu(), codes_c)
    assert torch.equal(xn_d.cpu(), xn.reshape(n, o, i))
    assert torch.equal(wt_d.cpu(), wt_c)


@pytest.mark.parametrize("L,N", [(16, 5000), (8, 3000), (16, 200_000)])
def test_fit_levels_kernel_bit_exact(L, N):
    """The weighted k-means against fit_levels on the CPU: with all values, and above 2^17 values
    through the seeded sample."""
    say(f"k-means kernel L={L} N={N}")
    g = torch.Generator().manual_seed(L + N)
    n = 3
    xn = (torch.randn(n, N, generator=g) * 0.4).clamp(-1, 1)
    wt = torch.rand(n, N, generator=g) * 3
    wt[1, : N // 3] = 0.0
    want = gptq.fit_levels(xn, wt, L)
    got = gptq.fit_levels_device(xn.to(DEV), wt.to(DEV), L)
    assert torch.equal(got.cpu(), want)
    assert torch.equal(gptq.fit_levels_device(xn.to(DEV), None, L).cpu(), gptq.fit_levels(xn, None, L))


def _cpu_inputs(W, H, L, block=32):
    """The sweep's inputs as the reference forms them, on the CPU: (W with dead columns zeroed,
    upper factor U, dead mask, block scales [n, out, in / block], levels)."""
    xn, blk, _ = gptq.block_headers(W, block)
    n, out, inp = W.shape
    cw = H.diagonal(dim1=-2, dim2=-1).float().view(n, 1, inp // block, block)
    wt = (cw.expand(n, out, -1, -1) * blk.pow(2)).reshape(n, -1)
    levels = gptq.fit_levels(xn.reshape(n, -1), wt, L).contiguous().float()
    Wd, U, dead = gptq.hessian_factor(W, H)
    return Wd, U, dead, blk[..., 0].contiguous(), levels


@pytest.mark.parametrize("case", G.CASES, ids=[c[0] for c in G.CASES])
def test_sweep_kernel_bit_exact_on_golden(case):
    name, n, o, i, L, tokens, seed = case
    say(f"gptq sweep kernel, golden case {name}")
    W, H = G.make_case(name, n, o, i, tokens, seed)
    Wd, U, dead, bs, levels = _cpu_inputs(torch.from_numpy(W), torch.from_numpy(H), L)
    assert torch.equal(levels, torch.from_numpy(GOLD[f"{name}__levels"]))
    q, codes = gptq.sweep_device(Wd.to(DEV), U.to(DEV), levels.to(DEV), bs.to(DEV), 32, dead.to(DEV))
    assert np.array_equal(q.cpu().numpy().view(np.uint32), GOLD[f"{name}__q"].view(np.uint32))
    bits = L.bit_length() - 1
    from blackhole_runtime.quant import pack
    assert np.array_equal(pack(codes.cpu(), bits).numpy(), GOLD[f"{name}__idx"])


@pytest.mark.parametrize("n,o,i,L,sblock,block", [(2, 70, 352, 16, 32, 128), (3, 64, 256, 8, 32, 128),
                                                  (1, 130, 192, 16, 64, 64), (2, 5, 160, 8, 32, 100)])
def test_sweep_kernel_equals_cpu_sweep(n, o, i, L, sblock, block):
    say(f"gptq sweep kernel vs the CPU sweep n={n} out={o} in={i} L={L} sblock={sblock} block={block}")
    g = torch.Generator().manual_seed(o + i)
    W = torch.randn(n, o, i, generator=g) * 0.02
    X = torch.randn(n, 3 * i, i, generator=g)
    X[:, :, 3] *= 8.0
    H = X.transpose(1, 2).contiguous() @ X
    W[0, :, 9] = 0.0                                       # a dead column
    Wd, U, dead, bs, levels = _cpu_inputs(W, H, L, sblock)
    scale = bs[..., None].expand(-1, -1, -1, sblock).reshape(n, o, i)

    def round_col(x, c):
        s = scale[..., c:c + 1]
        return torch.gather(levels, 1, gptq.nearest_index((x / s).clamp(-1, 1), levels).reshape(n, -1)).view(x.shape) * s
    Q = gptq.gptq_sweep(Wd.clone(), U, round_col, block) * (~dead)[:, None, :]
    codes = gptq.nearest_index((Q / scale).clamp(-1, 1), levels)
    q_d, c_d = gptq.sweep_device(Wd.to(DEV), U.to(DEV), levels.to(DEV), bs.to(DEV), sblock, dead.to(DEV), block)
    assert np.array_equal(q_d.cpu().numpy().view(np.uint32), Q.numpy().view(np.uint32))
    assert torch.equal(c_d.cpu().long(), codes)


def test_sweep_kernel_argument_checks():
    say("gptq sweep kernel argument checks")
    z = torch.zeros(1, 4, 64, device=DEV)
    with pytest.raises(ValueError, match="shapes"):
        gptq.sweep_device(z, torch.zeros(1, 64, 64, device=DEV), torch.zeros(1, 16, device=DEV),
                          torch.ones(1, 4, 3, device=DEV))
    with pytest.raises(NotImplementedError, match="8 or 16 levels"):
        gptq.sweep_device(z, torch.zeros(1, 64, 64, device=DEV), torch.zeros(1, 4, device=DEV),
                          torch.ones(1, 4, 2, device=DEV))
    with pytest.raises(ValueError, match="on the GPU"):
        gptq.sweep_device(z.cpu(), torch.zeros(1, 64, 64), torch.zeros(1, 16), torch.ones(1, 4, 2))
    with pytest.raises(NotImplementedError, match="at least 32 inputs"):
        gptq.sweep_device(z, torch.zeros(1, 64, 64, device=DEV), torch.zeros(1, 16, device=DEV),
                          torch.ones(1, 4, 4, device=DEV), 16)


def test_gptq_config2_width_and_fused_kernels():
    say("gptq at config-2 width")
    from blackhole_runtime import hex_moe as hm
    g = torch.Generator().manual_seed(7)
    n, o, i = 4, 768, 2048
    W = (torch.randn(n, o, i, generator=g) * 0.02).to(DEV)
    X = torch.randn(n, 1024, i, generator=g).to(DEV)
    H = X.transpose(1, 2).contiguous() @ X
    got = gptq.quantize_experts_gptq(W, H, 16)
    scale = gptq.block_headers(W)[1].expand(-1, -1, -1, 32).reshape(W.shape)
    rtn = torch.gather(got["levels"], 1, gptq.nearest_index((W / scale).clamp(-1, 1), got["levels"]).reshape(n, -1)
                       ).view(W.shape) * scale
    e_g, e_r = layer_err(W, got["q"], H), layer_err(W, rtn, H)
    say(f"  layer error GPTQ / plain rounding: {(e_g / e_r).tolist()}")
    assert torch.all(e_g < e_r)
    # the parts are HEX parts: the dequant kernel gives back Q
    deq = hm.hex_dequant(got["idx"], got["block_scale"], got["expert_scale"], got["levels"], 4, "R")
    torch.testing.assert_close(deq, got["q"], rtol=2e-6, atol=0)


def test_gptq_tiers_through_the_folder_checker(tmp_path):
    """Producer to consumer: a two-layer model's experts GPTQ-quantized on the GPU into a 16-level
    and an 8-level tier, written as a blackhole-hex folder, pass the folder checker's kernel check
    (the fused kernels against the float32 reference MoE on those tiers)."""
    say("gptq tiers through the folder checker")
    import json

    from safetensors.torch import save_file

    from blackhole_runtime import check_folder as cf
    E, H, I, hot = 6, 256, 128, 3
    g = torch.Generator().manual_seed(11)
    t = {}
    for li in range(2):
        pre = f"model.layers.{li}.mlp.experts"
        for L, ids in ((16, list(range(hot))), (8, list(range(hot, E)))):
            t[f"{pre}.tier{L}.experts"] = torch.tensor(ids, dtype=torch.int32)
            for proj, (o, i) in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
                W = (torch.randn(len(ids), o, i, generator=g) * 0.02).to(DEV)
                X = torch.randn(len(ids), 512, i, generator=g).to(DEV)
                parts = gptq.quantize_experts_gptq(W, X.transpose(1, 2).contiguous() @ X, L)
                for part in ("idx", "block_scale", "expert_scale", "levels"):
                    t[f"{pre}.tier{L}.{proj}.{part}"] = parts[part].cpu().contiguous()
    save_file(t, str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps({
        "text_config": {"num_experts": E, "num_experts_per_tok": 2, "hidden_size": H, "moe_intermediate_size": I},
        "quantization_config": {"quant_method": "blackhole-hex"}}))
    r = cf.check(tmp_path, DEV, tokens=9)
    say(f"  {r}")
    assert r["ok"] and r["checked"] == 2 and r["kernel_rel"] < 1e-2, r


def test_wrong_device_factor_is_recomputed():
    """A factor that does not reproduce its matrix (as the device routine has returned with a zero
    info code) is replaced by the CPU's; correct ones are kept."""
    say("gptq: checked Cholesky")
    g = torch.Generator().manual_seed(3)
    X = torch.randn(3, 300, 64, generator=g, dtype=torch.float64)
    A = (X.transpose(1, 2).contiguous() @ X).to(DEV)
    L, info = torch.linalg.cholesky_ex(A)
    L = L.clone()
    L[1] += 0.5                                              # a wrong factor with info 0
    mt = lambda x: x.transpose(-1, -2)                       # noqa: E731
    F, info = gptq._checked(A, L, info, lambda F_: (F_ @ mt(F_) - A).abs().amax(dim=(-2, -1)),
                            lambda a: torch.linalg.cholesky_ex(a))
    want = torch.linalg.cholesky(A.cpu())
    torch.testing.assert_close(F.cpu(), want, rtol=1e-10, atol=1e-10)
    assert info.tolist() == [0, 0, 0]
