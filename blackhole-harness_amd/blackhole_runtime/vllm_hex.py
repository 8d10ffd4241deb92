"""The "blackhole-hex" vLLM quantization method over the MI355X HEX kernels.

The drop-in counterpart of runtime/blackhole_runtime/vllm_hex.py: the same plugin entry point
(vllm.general_plugins -> register), quantization name, tensor names, weight loading, checks
and errors, with the routed experts served by blackhole_runtime.hex_moe (HIP kernels for gfx950).

A HEX folder stores each MoE layer's routed experts as tiers `<mlp>.experts.tier<L>` (experts
sharing one table size L) with `.experts` (int32 global ids) and per projection
`.<gate_proj|up_proj|down_proj>.<idx|block_scale|expert_scale|levels>`; everything else is
plain bf16. config.json carries quantization_config = {"quant_method": "blackhole-hex", ...,
optional "head_ids": [...]} (an output-trimmed LM head: other tokens get HEAD_FILL).
One GPU: tensor and expert parallel sizes must be 1 (vllm_hex.py:195-196).
"""

from __future__ import annotations

import re

import torch

NAME = "blackhole-hex"
KEEP_PLE = {NAME, "online"}    # quantization methods under which Qwen4Exp's n-gram table stays as stored
HEAD_FILL = -1.0e4             # logit of a token an output-trimmed LM head cannot write
_TIER = re.compile(r"^(?:.*\.)?tier(\d+)\.(?:(experts)|(gate_proj|up_proj|down_proj)\."
                   r"(idx|block_scale|expert_scale|levels))$")
_PARTS = ("idx", "block_scale", "expert_scale", "levels")


def _device() -> torch.device:
    return torch.device("cuda", torch.cuda.current_device()) if torch.cuda.is_available() else torch.device("cpu")


def plain_ple_embedding() -> bool:
    """Let vLLM's Qwen4Exp n-gram embedding (PLE) load under this method (and under vLLM's
    "online" methods): it is a lookup table kept as stored, so it is built as if the model were
    unquantized (vllm_hex.py:41-64). Idempotent; returns whether that model is in this vLLM."""
    try:
        from vllm.models.qwen4_exp.common import ngram_embedding as ng
    except Exception:  # noqa: BLE001  (no vLLM, or a vLLM without this model)
        return False
    cls = getattr(ng, "Qwen4ExpPLEEmbeddingMethod", None)
    if cls is None:
        return False
    if getattr(cls, "_blackhole_hex", False):
        return True
    original = cls.from_quant_config

    def from_quant_config(quant_config, prefix, embedding_dtype=None):
        name = getattr(quant_config, "get_name", lambda: None)() if quant_config is not None else None
        return original(None if name in KEEP_PLE else quant_config, prefix, embedding_dtype)

    cls.from_quant_config = staticmethod(from_quant_config)
    cls._blackhole_hex = True
    return True


def assemble_tiers(params: dict, shape: tuple[int, int, int], layer_name: str = "") -> list:
    """HexTiers of one layer from its loaded parameters {"hex_t{L}_experts": ids,
    "hex_t{L}_{proj}_{part}": tensor}, largest table first, checked against the model shape
    (E, H, I) and for full expert coverage (vllm_hex.py:215-234)."""
    from blackhole_runtime.hex_moe import HexTier
    E, H, I = shape
    levels = sorted({int(k.split("_")[1][1:]) for k in params if k.startswith("hex_t")}, reverse=True)
    if not levels:
        raise ValueError(f"blackhole-hex: no HEX experts were loaded for {layer_name}")
    seen = torch.zeros(E, dtype=torch.bool)
    tiers = []
    for L in levels:
        def proj(p, L=L):
            return {q: params[f"hex_t{L}_{p}_{q}"] for q in _PARTS}
        ids = params[f"hex_t{L}_experts"]
        tier = HexTier(L.bit_length() - 1, ids, proj("gate_proj"), proj("up_proj"), proj("down_proj")).prepare(E)
        if tier.gate_proj["idx"].shape[1] != I or tier.down_proj["idx"].shape[1] != H:
            raise ValueError(f"blackhole-hex: {layer_name} tier{L} shapes do not match the model")
        seen[ids.long().cpu()] = True
        tiers.append(tier)
    if not bool(seen.all()):
        missing = (~seen).nonzero().flatten().tolist()
        raise ValueError(f"blackhole-hex: {layer_name} has no weights for experts {missing[:8]}")
    return tiers


def tier_param_name(name: str, layer_name: str = "") -> str:
    """Parameter name of a checkpoint tensor of a HEX tier (vllm_hex.py:203-213)."""
    m = _TIER.match(name)
    if not m:
        raise ValueError(f"blackhole-hex: unexpected expert tensor {layer_name}.{name} "
                         "(expected <experts>.tier<L>.<proj>.<part> and .tier<L>.experts)")
    L = m.group(1)
    return f"hex_t{L}_experts" if m.group(2) else f"hex_t{L}_{m.group(3)}_{m.group(4)}"


def register() -> None:
    """vLLM general-plugin entry point; safe to call more than once (vllm_hex.py:67-180)."""
    plain_ple_embedding()
    from vllm.model_executor.layers.fused_moe import FusedMoEMethodBase, RoutedExperts
    from vllm.model_executor.layers.linear import LinearBase, UnquantizedLinearMethod
    from vllm.model_executor.layers.quantization import register_quantization_config
    from vllm.model_executor.layers.quantization.base_config import QuantizationConfig
    from vllm.model_executor.layers.vocab_parallel_embedding import ParallelLMHead, UnquantizedEmbeddingMethod

    from blackhole_runtime.hex_moe import hex_moe

    class HexHeadMethod(UnquantizedEmbeddingMethod):
        """bf16 LM head whose logits outside the kept output tokens are HEAD_FILL."""

        def __init__(self, ids):
            super().__init__()
            self.ids = ids

        def process_weights_after_loading(self, layer) -> None:
            super().process_weights_after_loading(layer)
            w = layer.weight
            mask = torch.full((w.shape[0],), HEAD_FILL, dtype=w.dtype, device=w.device)
            mask[torch.as_tensor(self.ids, dtype=torch.long, device=w.device)] = 0
            layer.register_buffer("hex_head_mask", mask, persistent=False)

        def apply(self, layer, x, bias=None):
            return super().apply(layer, x, bias) + layer.hex_head_mask

    class HexMoEMethod(FusedMoEMethodBase):
        def create_weights(self, layer, num_experts, hidden_size, intermediate_size_per_partition, params_dtype,
                           **extra_weight_attrs):
            if getattr(self.moe, "tp_size", 1) != 1 or getattr(self.moe, "ep_size", 1) != 1:
                raise ValueError("blackhole-hex runs on one GPU: use --tensor-parallel-size 1 and no expert parallel")
            layer.hex_shape = (num_experts, hidden_size, intermediate_size_per_partition)
            layer.hex_tiers = []
            # tier shapes come from the checkpoint, so parameters are registered as they load
            layer.load_weights = lambda weights: self._load(layer, weights)

        def _load(self, layer, weights):
            dev = _device()
            for name, t in weights:
                key = tier_param_name(name, getattr(layer, "layer_name", ""))
                layer.register_parameter(key, torch.nn.Parameter(t.to(dev), requires_grad=False))
                yield key

        def process_weights_after_loading(self, layer) -> None:
            params = {n: p.data for n, p in layer.named_parameters(recurse=False) if n.startswith("hex_t")}
            layer.hex_tiers = assemble_tiers(params, layer.hex_shape, getattr(layer, "layer_name", ""))

        def get_fused_moe_quant_config(self, layer):
            return None

        def apply(self, layer, x, topk_weights, topk_ids, shared_experts, shared_experts_input):
            return hex_moe(x, topk_weights, topk_ids.long(), layer.hex_tiers)

    @register_quantization_config(NAME)
    class HexConfig(QuantizationConfig):
        def __init__(self, cfg: dict):
            super().__init__()
            self.cfg = cfg
            self.head_ids = cfg.get("head_ids")

        def get_name(self):
            return NAME

        def get_supported_act_dtypes(self):
            return [torch.bfloat16, torch.float16]

        @classmethod
        def get_min_capability(cls) -> int:
            return 80

        @staticmethod
        def get_config_filenames():
            return []

        @classmethod
        def from_config(cls, config: dict):
            return cls(config)

        def get_quant_method(self, layer, prefix: str):
            if isinstance(layer, RoutedExperts):
                return HexMoEMethod(layer.moe_config)
            if isinstance(layer, ParallelLMHead) and self.head_ids:
                return HexHeadMethod(self.head_ids)
            if isinstance(layer, LinearBase):
                return UnquantizedLinearMethod()
            return None
