"""The blackhole-hex plugin's MoE method on device tensors (the vLLM module tree is faked, as on
the CPU side: vLLM is not installed here): register(), load a HEX layer's tier tensors by their
folder names, then HexMoEMethod.apply(layer, x, topk_weights, topk_ids, None, None) as vLLM's
FusedMoE calls it (runtime/blackhole_runtime/vllm_hex.py:121-146), against the CPU oracle, eager
and captured in a hipGraph; and the hex_check command on a small shape."""

from __future__ import annotations

import sys
import types

import numpy as np
import pytest
import torch

from blackhole_runtime import hex_check, vllm_hex
from fake_vllm import fake_vllm
from oracle import hex_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL_16 = 1e-2


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _layer_tensors(E, H, I, hot, seed):
    """Folder tensors of one MoE layer with a 16-level (4-bit) and an 8-level (3-bit) tier:
    [(name, CPU tensor)] under the reference's names, and the oracle's tier dicts."""
    perm = np.random.default_rng(seed).permutation(E)
    weights, ref = [], []
    for j, (ids, bits) in enumerate(((perm[:hot], 4), (perm[hot:], 3))):
        L = 1 << bits
        parts = {proj: O.random_parts(len(ids), o, i, bits, seed=seed + 10 * j + q, block=32)
                 for q, (proj, (o, i)) in enumerate((("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))))}
        ref.append({"bits": bits, "experts": ids, **parts})
        weights.append((f"model.layers.3.mlp.experts.tier{L}.experts", torch.from_numpy(ids.astype(np.int32))))
        for proj, p in parts.items():
            for q in ("idx", "block_scale", "expert_scale", "levels"):
                v = np.ascontiguousarray(p[q])
                if q == "idx":
                    v = v.view(np.int32)
                weights.append((f"model.layers.3.mlp.experts.tier{L}.{proj}.{q}",
                                torch.from_numpy(v.astype(np.float32) if q in ("expert_scale", "levels") else v)))
    return weights, ref


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_plugin_apply_on_device(monkeypatch, dt):
    say(f"plugin apply on device dt={dt}")
    E, H, I, k = 16, 512, 256, 4
    registry, RoutedExperts, _, _ = fake_vllm(monkeypatch)
    vllm_hex.register()
    cfg = registry[vllm_hex.NAME].from_config({"quant_method": "blackhole-hex"})

    class Layer(RoutedExperts, torch.nn.Module):
        def __init__(self):
            torch.nn.Module.__init__(self)
            self.moe_config = types.SimpleNamespace(tp_size=1, ep_size=1)
            self.layer_name = "model.layers.3.mlp.experts"

    layer = Layer()
    method = cfg.get_quant_method(layer, "model.layers.3.mlp.experts")
    method.create_weights(layer, E, H, I, dt)
    weights, ref = _layer_tensors(E, H, I, hot=6, seed=70)
    loaded = list(layer.load_weights(iter((n.split("experts.", 1)[1], t) for n, t in weights)))
    assert len(loaded) == len(weights)
    assert all(p.is_cuda for p in layer.parameters())
    method.process_weights_after_loading(layer)
    assert [t.bits for t in layer.hex_tiers] == [4, 3]
    act_round = {torch.bfloat16: "bf16", torch.float16: "f16"}[dt]
    for T in (1, 7, 64):
        rng = np.random.default_rng(T)
        w, ids = O.route_topk(rng.standard_normal((T, E)).astype(np.float32), k)
        x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(dt)
        xd, wd = x.to(DEV), torch.from_numpy(w).to(DEV)
        idd = torch.from_numpy(ids.astype(np.int32)).to(DEV)           # vLLM's topk_ids are int32
        out = method.apply(layer, xd, wd, idd, None, None)
        assert out.dtype == dt and out.shape == (T, H) and out.is_cuda
        want = O.moe_reference(x.float().numpy(), w, ids, ref, act_round)
        err = O.rel_err(out.float().cpu().numpy(), want)
        assert err < TOL_16, (T, err)
        # as vLLM's decode graphs capture it
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            method.apply(layer, xd, wd, idd, None, None)
        torch.cuda.current_stream().wait_stream(s)
        with torch.cuda.graph(g):
            cap = method.apply(layer, xd, wd, idd, None, None)
        for i in range(2):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(cap, out), (T, i)
            method.apply(layer, xd * 2, wd, idd, None, None)            # unrelated eager work between replays
            torch.cuda.synchronize()


def test_hex_check_command(capsys):
    """python -m blackhole_runtime.hex_check on a small shape: every numbers check passes and the
    timing table prints (the reference's hex_check.py:94-154)."""
    say("hex_check small shape")
    rc = hex_check.main(["--experts", "24", "--hidden", "512", "--inter", "256", "--topk", "4", "--hot", "0.25",
                         "--tokens", "1,8,300", "--iters", "5", "--sweep"])
    out = capsys.readouterr().out
    assert rc == 0, out
    assert "HEX HIP kernels OK" in out and "max rel error" in out and "HEX weight traffic" in out
