"""The blackhole-hex folder checker's structural checks, on the CPU (no kernels run here): a good
folder passes, and each kind of broken folder names its problem. Mirrors
runtime/tests/test_folder.py:38-47 (ok folder; a dropped expert), plus the shape, method and
CLI cases this checker adds. The kernel check itself is a GPU test (test_gpu_folder.py)."""

from __future__ import annotations

import json

import torch

from blackhole_runtime import check_folder as cf
from blackhole_runtime.quant import random_parts


def write_folder(d, E=6, H=64, I=32, hot=3, drop=None, block=32, layers=2, method="blackhole-hex", cfg_extra=None,
                 mangle=None):
    """Two layers, each a 16-level tier (experts 0..hot-1) and an 8-level tier (the rest)."""
    from safetensors.torch import save_file
    t = {}
    for li in range(layers):
        pre = f"model.language_model.layers.{li}.mlp.experts"
        for L, ids in ((16, list(range(hot))), (8, list(range(hot, E)))):
            if drop is not None and drop in ids:
                ids = [i for i in ids if i != drop]
            bits = L.bit_length() - 1
            t[f"{pre}.tier{L}.experts"] = torch.tensor(ids, dtype=torch.int32)
            for proj, (o, i) in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
                for part, v in random_parts(len(ids), o, i, bits, device="cpu", seed=li * 10 + L, block=block).items():
                    t[f"{pre}.tier{L}.{proj}.{part}"] = v.contiguous()
    t["model.language_model.layers.0.self_attn.q_proj.weight"] = torch.zeros(4, 4)    # not a HEX tensor
    if mangle:
        mangle(t)
    save_file(t, str(d / "model.safetensors"))
    tc = {"num_experts": E, "num_experts_per_tok": 2, **(cfg_extra or {})}
    (d / "config.json").write_text(json.dumps({"model_type": "qwen3_moe", "text_config": tc,
                                               "quantization_config": {"quant_method": method}}))


def test_tiers_by_layer_finds_every_tier(tmp_path):
    write_folder(tmp_path)
    layers = cf.tiers_by_layer(tmp_path)
    assert sorted(layers) == [f"model.language_model.layers.{i}.mlp.experts" for i in range(2)]
    for tiers in layers.values():
        assert sorted(tiers) == [8, 16]
        assert tiers[16]["experts"].tolist() == [0, 1, 2]
        assert tiers[8]["gate_proj"]["idx"].shape == (3, 32, 64 // 32 * 3)
        assert tiers[16]["down_proj"]["levels"].shape == (3, 16)


def test_good_folder_passes_structure_on_cpu(tmp_path):
    write_folder(tmp_path, cfg_extra={"hidden_size": 64, "moe_intermediate_size": 32})
    r = cf.check(tmp_path, "cpu")
    assert r["ok"] and r["layers"] == 2 and r["checked"] == 0 and r["kernel_rel"] is None, r


def test_missing_expert_is_a_problem(tmp_path):
    write_folder(tmp_path, drop=4)
    r = cf.check(tmp_path, "cpu")
    assert not r["ok"] and "expected each of 0..5 once" in r["problems"][0], r


def test_wrong_method_no_tiers_and_shape_problems(tmp_path):
    a = tmp_path / "a"
    a.mkdir()
    write_folder(a, method="gptq")
    r = cf.check(a, "cpu")
    assert not r["ok"] and "not 'blackhole-hex'" in r["problems"][0]

    b = tmp_path / "b"
    b.mkdir()
    write_folder(b, layers=0)
    r = cf.check(b, "cpu")
    assert not r["ok"] and "no HEX tiers" in r["problems"][0]

    c = tmp_path / "c"
    c.mkdir()
    write_folder(c, cfg_extra={"hidden_size": 128})
    r = cf.check(c, "cpu")
    assert not r["ok"] and any("config.json says 128" in p for p in r["problems"]), r

    d = tmp_path / "d"
    d.mkdir()

    def cut_down(t):          # layer 1's 8-level down_proj loses an output row
        k = "model.language_model.layers.1.mlp.experts.tier8.down_proj.idx"
        t[k] = t[k][:, :-1].contiguous()
    write_folder(d, mangle=cut_down)
    r = cf.check(d, "cpu")
    assert not r["ok"] and r["layers"] == 2, r
    assert any("layers.1.mlp.experts.tier8.down_proj.block_scale" in p for p in r["problems"]), r
    assert not any("layers.0" in p for p in r["problems"]), r

    e = tmp_path / "e"
    e.mkdir()

    def drop_levels(t):
        del t["model.language_model.layers.0.mlp.experts.tier16.up_proj.levels"]
    write_folder(e, mangle=drop_levels)
    r = cf.check(e, "cpu")
    assert not r["ok"] and "missing up_proj.levels" in r["problems"][0], r


def test_cli_prints_one_json_line_and_exit_code(tmp_path, capsys):
    write_folder(tmp_path)
    assert cf.main([str(tmp_path), "--device", "cpu"]) == 0
    out = capsys.readouterr().out.strip().splitlines()
    assert len(out) == 1 and json.loads(out[0])["ok"] is True
    bad = tmp_path / "bad"
    bad.mkdir()
    write_folder(bad, drop=0)
    assert cf.main([str(bad), "--device", "cpu"]) == 1
    assert json.loads(capsys.readouterr().out.strip())["ok"] is False
