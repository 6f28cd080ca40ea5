"""Stand-in vLLM modules for the quantization plugin (vLLM is not installed here).

They carry the names plugin.define_vllm_classes() imports: LinearBase and
UnquantizedLinearMethod, ParallelLMHead and UnquantizedEmbeddingMethod, QuantizationConfig,
and register_quantization_config, which records what it registers. The base classes are
plain Python classes; the hooks the plugin overrides (process_weights_after_loading, apply)
are what vLLM calls on them.
"""
import sys
import types

MODULES = ("vllm", "vllm.model_executor", "vllm.model_executor.layers", "vllm.model_executor.layers.linear",
           "vllm.model_executor.layers.quantization", "vllm.model_executor.layers.quantization.base_config",
           "vllm.model_executor.layers.vocab_parallel_embedding")


class LinearBase:
    pass


class ParallelLMHead:
    pass


class VocabParallelEmbedding:
    pass


class UnquantizedLinearMethod:
    def process_weights_after_loading(self, layer):
        pass


class UnquantizedEmbeddingMethod:
    def process_weights_after_loading(self, layer):
        pass


class QuantizationConfig:
    def __init__(self):
        self.packed_modules_mapping = {}


def install(monkeypatch):
    """Register the stand-in modules in sys.modules (undone by monkeypatch); returns the dict
    that register_quantization_config fills, name -> registered class."""
    registry = {}

    def register_quantization_config(name):
        def deco(cls):
            if name in registry:
                raise ValueError(f"quantization config {name!r} is already registered")
            registry[name] = cls
            return cls
        return deco

    mods = {name: types.ModuleType(name) for name in MODULES}
    mods["vllm.model_executor.layers.linear"].LinearBase = LinearBase
    mods["vllm.model_executor.layers.linear"].UnquantizedLinearMethod = UnquantizedLinearMethod
    mods["vllm.model_executor.layers.quantization"].register_quantization_config = register_quantization_config
    mods["vllm.model_executor.layers.quantization.base_config"].QuantizationConfig = QuantizationConfig
    emb = mods["vllm.model_executor.layers.vocab_parallel_embedding"]
    emb.ParallelLMHead, emb.UnquantizedEmbeddingMethod = ParallelLMHead, UnquantizedEmbeddingMethod
    emb.VocabParallelEmbedding = VocabParallelEmbedding
    for name, mod in mods.items():
        monkeypatch.setitem(sys.modules, name, mod)
    return registry
