"""Host logic without a GPU: tile choice, HexTier.prepare, the GPU-only guard, and the
"blackhole-hex" vLLM plugin against fake vLLM modules (as runtime/tests/test_folder.py:60-93
tests the reference's plugin)."""

from __future__ import annotations

import sys
import types

import numpy as np
import pytest
import torch

from blackhole_runtime import hex_moe as hm
from blackhole_runtime import vllm_hex
from fake_vllm import fake_vllm
from oracle import hex_oracle as O


def _parts(n, out, inp, bits, seed):
    p = O.random_parts(n, out, inp, bits, seed=seed)
    return {"idx": torch.from_numpy(p["idx"].view(np.int32)).view(torch.uint32) if hasattr(torch, "uint32")
            else torch.from_numpy(p["idx"].view(np.int32)),
            "block_scale": torch.from_numpy(p["block_scale"]), "expert_scale": torch.from_numpy(p["expert_scale"]),
            "levels": torch.from_numpy(p["levels"])}


def _tier(ids, bits, H=64, I=32, seed=0):
    n = len(ids)
    return hm.HexTier(bits, torch.tensor(ids), _parts(n, I, H, bits, seed + 1), _parts(n, I, H, bits, seed + 2),
                      _parts(n, H, I, bits, seed + 3))


def test_prepare_views_lookup_and_structs():
    t = _tier([3, 0, 5], 4).prepare(6)
    assert t.gate_proj["idx"].dtype == torch.int32 and t.experts.dtype == torch.int32
    assert t.lookup.tolist() == [1, -1, -1, 0, -1, 2]
    s = t.struct("down_proj")
    assert s.block == 32 and s.s_in == t.down_proj["idx"].stride(1)
    with pytest.raises(ValueError, match="expert ids"):
        _tier([0, 7], 4).prepare(6)
    with pytest.raises(ValueError, match="levels"):
        _tier([0], 3).__class__(4, torch.tensor([0]), *[_parts(1, 8, 64, 3, 1)] * 3).prepare(2)


def test_prepare_splits_experts_into_parts():
    """prepare() also builds the tier's SPLIT parts by expert for the prefill streams: views of
    the tier's own tensors (no copies), each with the lookup of its own experts."""
    t = _tier([3, 0, 5, 1, 4], 4).prepare(6)
    assert hm.SPLIT == 2 and len(t._parts) == 2
    a, b = t._parts
    assert a.experts.tolist() == [3, 0] and b.experts.tolist() == [5, 1, 4]
    assert a.lookup.tolist() == [1, -1, -1, 0, -1, -1] and b.lookup.tolist() == [-1, 1, -1, -1, 2, 0]
    for name in hm.PROJS:
        whole, pa, pb = getattr(t, name), getattr(a, name), getattr(b, name)
        for q in ("idx", "block_scale", "expert_scale", "levels"):
            assert pa[q].data_ptr() == whole[q].data_ptr()
            assert pb[q].data_ptr() == whole[q][2:].data_ptr() and torch.equal(pb[q], whole[q][2:])
    assert a._parts is None and b._parts is None             # parts are not split again
    assert _tier([2], 4).prepare(6)._parts is None           # one expert: nothing to split


def test_block_from_shapes_128():
    t = _tier([0], 4, H=256, I=128)
    for name in ("gate_proj", "up_proj", "down_proj"):
        p = getattr(t, name)
        p["block_scale"] = p["block_scale"][..., ::4].contiguous()
    t.prepare(1)
    assert t.struct("gate_proj").block == 128 and t.struct("down_proj").block == 128


def test_default_config_and_env(monkeypatch):
    assert hm.default_config(8, 768, 2048, True, 96) == {"BLOCK_M": 16, "BLOCK_N": 256}    # T=1 decode
    assert hm.default_config(128, 768, 2048, True, 96)["BLOCK_M"] == 16                    # T=16
    assert hm.default_config(96 * 12, 768, 2048, True, 96)["BLOCK_M"] == 16                # 12 per expert
    assert hm.default_config(2048, 1536, 4096, True, 128)["BLOCK_M"] == 32                 # 16 per expert
    assert hm.default_config(32768, 2048, 768, False, 96)["BLOCK_M"] == 128                # prefill
    assert hm.default_config(32768, 2048, 96, False, 96)["BLOCK_M"] == 32                  # inputs % 128 != 0
    assert hm.default_config(3000, 768, 2048, True, 96)["BLOCK_M"] == 32                   # 31 per expert
    assert hm.default_config(96 * 48, 768, 2048, True, 96)["BLOCK_M"] == 32                # 48 per expert
    assert hm.default_config(96 * 49, 768, 2048, True, 96)["BLOCK_M"] == 128               # (64 never by default)
    # experts of 4M weights or more (config 5) take the prefill kernels above 35 slots per expert
    assert hm.default_config(128 * 35, 1536, 4096, True, 128)["BLOCK_M"] == 32
    assert hm.default_config(128 * 36, 1536, 4096, True, 128)["BLOCK_M"] == 128
    assert hm.default_config(128 * 36, 4096, 1536, False, 128)["BLOCK_M"] == 128
    monkeypatch.setenv("BLACKHOLE_HEX_TILES", "64")
    assert hm.default_config(8, 768, 2048, True, 96) == {"BLOCK_M": 64, "BLOCK_N": 256}
    # the reference's own config keys map onto the tile
    assert hm._tile_from({"BLOCK_M": 16, "BLOCK_N": 32, "BLOCK_K": 32, "num_warps": 4, "num_stages": 1}) == 16
    assert hm._tile_from({"BLOCK_M": 64, "BLOCK_N": 128}) == 64
    assert hm._tile_from({"BLOCK_M": 128, "BLOCK_N": 128}) == 128
    assert hm._tile_from({"BLOCK_M": 24}) == 32
    assert hm._fit_tile(128, 768, 2048, False) == 128 and hm._fit_tile(128, 160, 2048, False) == 32
    assert hm._fit_tile(128, 2048, 100, True) == 32 and hm._fit_tile(128, 2048, 100, False) == 32
    assert hm._fit_tile(128, 2048, 104, False) == 128 and hm._fit_tile(64, 2048, 100, False) == 64
    assert hm._fit_tile(32, 160, 99, True) == 32


def _zero_tier(n_local, E, H, I, bits=4, block=128):
    def proj(o, i):
        return {"idx": torch.zeros(n_local, o, i // 32 * bits, dtype=torch.int32),
                "block_scale": torch.zeros(n_local, o, i // block, dtype=torch.uint8),
                "expert_scale": torch.ones(n_local), "levels": torch.zeros(n_local, 1 << bits)}
    return hm.HexTier(bits, torch.arange(n_local, dtype=torch.int32), proj(I, H), proj(I, H), proj(H, I)).prepare(E)


def test_gemv_prefer_follows_the_measured_crossovers(monkeypatch):
    """The matrix-vector launches are taken while the bytes that slots sharing an expert read again
    stay within GEMV_EXTRA_MB: at 96 experts of 2048 x 768 (top-8) up to 10 tokens (measured
    faster at 8 and 10, slower at 12), at 128 experts of 4096 x 1536 up to 5 (faster at 4 and 5,
    slower at 6); never past GEMV_MAX slots or the launches' width limits."""
    t2 = _zero_tier(2, 96, 2048, 768)
    assert t2._expert_bytes == 3 * 768 * 2048 // 2 + 2 * 768 * 16 + 2048 * 6 + 3 * (4 + 16 * 4)
    assert [T for T in range(1, 17) if hm.gemv_prefer(T, 8, 2048, 768, t2)] == list(range(1, 11))
    t5 = _zero_tier(2, 128, 4096, 1536)
    assert [T for T in range(1, 17) if hm.gemv_prefer(T, 8, 4096, 1536, t5)] == list(range(1, 6))
    assert not hm.gemv_prefer(0, 8, 2048, 768, t2) and not hm.gemv_prefer(1, 17, 2048, 768, t2)
    monkeypatch.setattr(hm, "GEMV_MAX", 0)
    assert not hm.gemv_prefer(1, 8, 2048, 768, t2)


def test_kernels_refuse_cpu_tensors():
    x = torch.zeros(2, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        hm.align(torch.zeros(4, dtype=torch.long), 4, 16)
    t = _tier([0, 1], 4).prepare(2)
    with pytest.raises(ValueError, match="GPU"):
        hm.hex_moe_fused(x, torch.ones(2, 1), torch.zeros(2, 1, dtype=torch.long), [t])
    with pytest.raises(ValueError, match="unknown path"):
        hm.hex_moe(x, torch.ones(2, 1), torch.zeros(2, 1, dtype=torch.long), [t], path="triton")


def test_dequant_path_refused_while_capturing(monkeypatch):
    """Under graph capture, float32 activations (path "auto") and path "dequant" raise a clear
    NotImplementedError instead of reaching the host synchronisation of the dequant path; bf16
    activations go on to the fused path (which then refuses the CPU tensor here)."""
    class FakeX:                     # a device tensor as far as hex_moe's dispatch looks
        is_cuda = True
        dtype = torch.float32
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    t = _tier([0, 1], 4).prepare(2)
    ids = torch.zeros(2, 1, dtype=torch.long)
    with pytest.raises(NotImplementedError, match="cannot be captured"):
        hm.hex_moe(FakeX(), torch.ones(2, 1), ids, [t])
    FakeX.dtype = torch.bfloat16
    with pytest.raises(NotImplementedError, match="cannot be captured"):
        hm.hex_moe(FakeX(), torch.ones(2, 1), ids, [t], path="dequant")
    with pytest.raises(ValueError, match="GPU"):
        hm.hex_moe(torch.zeros(2, 64, dtype=torch.bfloat16), torch.ones(2, 1), ids, [t])


# --------------------------------------------------------------------------- the vLLM plugin


def test_tier_param_names():
    assert vllm_hex.tier_param_name("model.layers.0.mlp.experts.tier16.experts") == "hex_t16_experts"
    assert vllm_hex.tier_param_name("tier8.down_proj.levels") == "hex_t8_down_proj_levels"
    with pytest.raises(ValueError, match="unexpected expert tensor"):
        vllm_hex.tier_param_name("experts.0.gate_proj.weight", "layer")


def _params(tiers):
    out = {}
    for L, t in tiers:
        out[f"hex_t{L}_experts"] = t.experts
        for proj in ("gate_proj", "up_proj", "down_proj"):
            for q in ("idx", "block_scale", "expert_scale", "levels"):
                out[f"hex_t{L}_{proj}_{q}"] = getattr(t, proj)[q]
    return out


def test_assemble_tiers_checks():
    good = [(16, _tier([0, 2], 4)), (8, _tier([1, 3], 3, seed=5))]
    tiers = vllm_hex.assemble_tiers(_params(good), (4, 64, 32), "l0")
    assert [t.bits for t in tiers] == [4, 3]
    with pytest.raises(ValueError, match=r"no weights for experts \[3\]"):
        vllm_hex.assemble_tiers(_params([(16, _tier([0, 2], 4)), (8, _tier([1], 3))]), (4, 64, 32), "l0")
    with pytest.raises(ValueError, match="shapes do not match"):
        vllm_hex.assemble_tiers(_params(good), (4, 64, 48), "l0")
    with pytest.raises(ValueError, match="no HEX experts"):
        vllm_hex.assemble_tiers({}, (4, 64, 32), "l0")


def test_register_with_fake_vllm(monkeypatch):
    registry, RoutedExperts, ParallelLMHead, LinearBase = fake_vllm(monkeypatch)
    vllm_hex.register()
    vllm_hex.register()                                       # idempotent
    cfg = registry[vllm_hex.NAME].from_config({"quant_method": "blackhole-hex", "head_ids": [1, 3]})
    assert cfg.get_name() == "blackhole-hex" and cfg.get_min_capability() == 80
    assert cfg.get_supported_act_dtypes() == [torch.bfloat16, torch.float16]

    class Layer(RoutedExperts, torch.nn.Module):
        def __init__(self):
            torch.nn.Module.__init__(self)
            self.moe_config = types.SimpleNamespace(tp_size=1, ep_size=1)
            self.layer_name = "model.layers.0.mlp.experts"

    layer = Layer()
    method = cfg.get_quant_method(layer, "p")
    assert type(method).__name__ == "HexMoEMethod"
    method.create_weights(layer, 4, 64, 32, torch.bfloat16)
    src = [(16, _tier([0, 2], 4)), (8, _tier([1, 3], 3, seed=5))]
    weights = []
    for L, t in src:
        weights.append((f"tier{L}.experts", t.experts))
        for proj in ("gate_proj", "up_proj", "down_proj"):
            for part in ("idx", "block_scale", "expert_scale", "levels"):
                weights.append((f"tier{L}.{proj}.{part}", getattr(t, proj)[part]))
    loaded = list(layer.load_weights(iter(weights)))
    assert "hex_t16_gate_proj_idx" in loaded and len(loaded) == len(weights)
    method.process_weights_after_loading(layer)
    assert [t.bits for t in layer.hex_tiers] == [4, 3]
    with pytest.raises(ValueError, match="unexpected expert tensor"):
        list(layer.load_weights(iter([("experts.0.w1", torch.zeros(1))])))
    bad = Layer()
    bad.moe_config = types.SimpleNamespace(tp_size=2, ep_size=1)
    with pytest.raises(ValueError, match="one GPU"):
        cfg.get_quant_method(bad, "p").create_weights(bad, 4, 64, 32, torch.bfloat16)

    class Head(ParallelLMHead, torch.nn.Module):
        def __init__(self):
            torch.nn.Module.__init__(self)
            self.weight = torch.nn.Parameter(torch.ones(5, 3), requires_grad=False)

    head = Head()
    hm_ = cfg.get_quant_method(head, "lm_head")
    hm_.process_weights_after_loading(head)
    logits = hm_.apply(head, torch.ones(2, 3))
    assert logits[0].tolist() == [vllm_hex.HEAD_FILL + 3, 3.0, vllm_hex.HEAD_FILL + 3, 3.0, vllm_hex.HEAD_FILL + 3]

    class Lin(LinearBase):
        pass

    assert type(cfg.get_quant_method(Lin(), "q")).__name__ == "UnquantizedLinearMethod"
    assert cfg.get_quant_method(object(), "x") is None


def test_qwen4_exp_ple_embedding_patch(monkeypatch):
    """The counterpart of runtime/tests/test_folder.py:60-93."""
    calls = []

    class Method:
        @staticmethod
        def from_quant_config(quant_config, prefix, embedding_dtype=None):
            calls.append(quant_config)
            if quant_config is not None and quant_config.get_name() != "fp8":
                raise NotImplementedError("unsupported")
            return "plain" if quant_config is None else "fp8"

    ng = types.ModuleType("vllm.models.qwen4_exp.common.ngram_embedding")
    ng.Qwen4ExpPLEEmbeddingMethod = Method
    for name in ("vllm", "vllm.models", "vllm.models.qwen4_exp", "vllm.models.qwen4_exp.common"):
        monkeypatch.setitem(sys.modules, name, types.ModuleType(name))
    sys.modules["vllm.models.qwen4_exp.common"].ngram_embedding = ng
    monkeypatch.setitem(sys.modules, ng.__name__, ng)

    class Q:
        def __init__(self, n):
            self.n = n

        def get_name(self):
            return self.n

    assert vllm_hex.plain_ple_embedding() and vllm_hex.plain_ple_embedding()
    assert Method.from_quant_config(Q(vllm_hex.NAME), "model.layers.1.ple") == "plain"
    assert Method.from_quant_config(Q("online"), "model.layers.1.ple") == "plain"
    assert Method.from_quant_config(Q("fp8"), "x") == "fp8"
    with pytest.raises(NotImplementedError):
        Method.from_quant_config(Q("awq"), "x")


def test_plain_ple_embedding_without_vllm(monkeypatch):
    monkeypatch.setitem(sys.modules, "vllm", None)
    assert vllm_hex.plain_ple_embedding() is False
