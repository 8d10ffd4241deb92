"""A stand-in for the parts of vLLM's module tree that the blackhole-hex plugin imports
(vllm is not installed on this image or on the GPU boxes): the base classes and the quantization
registry, installed into sys.modules through pytest's monkeypatch."""

from __future__ import annotations

import sys
import types


def fake_vllm(monkeypatch):
    """Installs the fake modules; returns (registry, RoutedExperts, ParallelLMHead, LinearBase)."""
    registry = {}

    def mod(name):
        m = types.ModuleType(name)
        monkeypatch.setitem(sys.modules, name, m)
        return m

    for name in ("vllm", "vllm.model_executor", "vllm.model_executor.layers"):
        mod(name)
    fm = mod("vllm.model_executor.layers.fused_moe")

    class FusedMoEMethodBase:
        def __init__(self, moe):
            self.moe = moe

    class RoutedExperts:
        pass

    fm.FusedMoEMethodBase, fm.RoutedExperts = FusedMoEMethodBase, RoutedExperts
    lin = mod("vllm.model_executor.layers.linear")

    class LinearBase:
        pass

    class UnquantizedLinearMethod:
        pass

    lin.LinearBase, lin.UnquantizedLinearMethod = LinearBase, UnquantizedLinearMethod
    q = mod("vllm.model_executor.layers.quantization")

    def register_quantization_config(name):
        def deco(cls):
            registry[name] = cls
            return cls
        return deco

    q.register_quantization_config = register_quantization_config
    bc = mod("vllm.model_executor.layers.quantization.base_config")

    class QuantizationConfig:
        pass

    bc.QuantizationConfig = QuantizationConfig
    ve = mod("vllm.model_executor.layers.vocab_parallel_embedding")

    class UnquantizedEmbeddingMethod:
        def process_weights_after_loading(self, layer):
            pass

        def apply(self, layer, x, bias=None):
            return x @ layer.weight.T

    class ParallelLMHead:
        pass

    ve.ParallelLMHead, ve.UnquantizedEmbeddingMethod = ParallelLMHead, UnquantizedEmbeddingMethod
    return registry, RoutedExperts, ParallelLMHead, LinearBase
