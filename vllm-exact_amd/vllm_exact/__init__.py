"""vllm-exact for MI355X: batch-invariant exact linear layers and decode attention.

Usage (enable() must be called before importing vllm), as in the reference (__init__.py):

    import vllm_exact
    kw = vllm_exact.enable(max_model_len=16784)
    from vllm import LLM
    llm = LLM(model=..., dtype="bfloat16", max_model_len=16784, **kw)

enable() turns on vLLM's batch-invariant mode with the engine core in-process, bypasses
vLLM's GDN batch-invariance check, registers quantization="exact_int8" (every linear layer,
lm_head by default, through the gfx950 exact matmul), returns the LLM keyword arguments
(no chunked prompts, Triton GDN prefill, the FLASH_ATTN backend unless another is named, no
prefix caching), and patches that backend's decode attention onto the fixed-order paged
kernel.
"""
import os
import sys
from pathlib import Path

__version__ = "0.1.0"
_ENABLED = False
# Tuning tables ship for MI355X only; the reference's H200/B300 tables describe other GPUs.
TABLES = {"mi355x": Path(__file__).with_name("cfg_table_mi355x_F14.json")}
# Tuned at F = 15 (offset digits, 4 dots): enable(f=15) takes it for the same key.
TABLES_F15 = {"mi355x": Path(__file__).with_name("cfg_table_mi355x_F15.json")}


def _attention_backends():
    from . import paged_attn
    return paged_attn.BACKENDS


def enable(max_model_len, f=14, lm_head=True, attention=True, cfg_table="mi355x", max_num_batched_tokens=131072,
           attention_backend="FLASH_ATTN", release_weights=False):
    """Return keyword arguments for vllm.LLM(...) (reference __init__.py:32-68).

    max_model_len: the value passed to LLM (fixes the attention kernel's segment count).
    f: 14 (truncated, 3 INT8 dots; default) or 15 (offset digits, 4 dots).
    cfg_table: "mi355x", a path to a table, or None (built-in configs). Tables change speed
      only, never results. "mi355x" means the table tuned at F = 15 when f = 15.
    max_num_batched_tokens: must exceed every prompt length (prompts are never chunked).
    attention_backend: the vLLM backend whose decode path is replaced (paged_attn.BACKENDS;
      the reference always uses FLASH_ATTN). vLLM is asked for the same backend.
    release_weights: free each linear layer's bf16 weight once its digits are packed (the
      lm_head's is kept). The reference keeps both copies; this halves the weight memory but
      breaks code that reads a linear layer's .weight after loading.
    """
    global _ENABLED
    if _ENABLED:
        raise RuntimeError("vllm_exact.enable() can only be called once")
    if "vllm" in sys.modules:
        raise RuntimeError("vllm_exact.enable() must be called before importing vllm")
    if attention and attention_backend not in _attention_backends():
        raise ValueError(f"attention_backend must be one of {sorted(_attention_backends())}")
    if cfg_table in ("h200", "b300"):
        raise ValueError(f"the {cfg_table} table describes another GPU; use 'mi355x', a path, or None")
    os.environ["VLLM_BATCH_INVARIANT"] = "1"
    os.environ["VLLM_ENABLE_V1_MULTIPROCESSING"] = "0"

    from . import plugin
    if not plugin.HAVE_VLLM:
        raise ImportError("vllm_exact.enable() needs vLLM (the host engine) to be importable")
    plugin.F = f
    plugin.TRUNC = f == 14
    plugin.LMHEAD = lm_head
    plugin.RELEASE_WEIGHTS = bool(release_weights)
    tables = TABLES_F15 if f == 15 else TABLES
    plugin.load_table(tables.get(cfg_table, cfg_table) if cfg_table else None)

    from vllm.v1.attention.backends.gdn_attn import GDNAttentionBackend
    GDNAttentionBackend.supports_batch_invariance = classmethod(lambda cls: True)

    kw = dict(quantization="exact_int8", max_num_batched_tokens=max_num_batched_tokens, enable_prefix_caching=False,
              additional_config={"gdn_prefill_backend": "triton"})
    if attention:
        from . import paged_attn
        paged_attn.MAX_LEN = max_model_len
        paged_attn.install(attention_backend)
        kw["attention_config"] = {"backend": attention_backend}
    _ENABLED = True
    return kw
