"""GPU check of the decode-step emulation (the ~9B hybrid's exact linears, paged decode
attention and exact lm_head, as bench.py times it): the logits of every request are bitwise
the same whether it runs alone, inside the full batch, or in a batch of another order and
size.

* A reduced model (4 layers, one attention layer, a 2048-row lm_head) with ragged context
  lengths, every request checked alone.
* The full model (32 layers of QKV 4096->6144, O 4096->4096, gate_up 4096->24576 and down
  12288->4096, attention on 8 of them, the 151936-row lm_head) at batch / context 256 / 1K,
  64 / 8K and 16 / 16K, with context lengths drawn from [L/2, L]: the first, a middle and the
  last request alone, and a reordered sub-batch, against the full batch.
"""
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import bench  # noqa: E402
from vllm_exact import paged_attn as P  # noqa: E402
from vllm_exact import plugin  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_decode_step_logits_are_batch_invariant(monkeypatch):
    monkeypatch.setattr(plugin, "F", 14)
    monkeypatch.setattr(plugin, "TRUNC", True)
    monkeypatch.setattr(P, "MAX_LEN", 4096)
    gen = torch.Generator(device=DEV).manual_seed(7)
    model = bench.DecodeStep(torch, plugin, P, torch.device(DEV), gen, layers=4, vocab=2048, keep_bf16=False)
    B, L = 6, 1000
    caches, bt, _ = model.kv(B, L, gen)
    sl = torch.tensor([1000, 517, 64, 999, 1, 730], device=DEV, dtype=torch.int32)
    h0 = torch.randn(B, bench.HIDDEN, device=DEV, generator=gen).to(torch.bfloat16)
    full = model.step(h0, caches, bt, sl)
    assert full.shape == (B, 2048) and torch.isfinite(full.float()).all()
    for i in range(B):
        alone = model.step(h0[i:i + 1], caches, bt[i:i + 1], sl[i:i + 1])
        assert torch.equal(alone, full[i:i + 1]), i
    sel = torch.tensor([4, 1, 5, 0], device=DEV)
    sub = model.step(h0[sel], caches, bt[sel].contiguous(), sl[sel].contiguous())
    assert torch.equal(sub, full[sel])


@pytest.fixture(scope="module")
def full_model():
    """The full-size decode-step model with the shipped F = 14 table (enable()'s default)."""
    import vllm_exact

    saved = plugin.F, plugin.TRUNC, P.MAX_LEN
    plugin.F, plugin.TRUNC, P.MAX_LEN = 14, True, 16384
    plugin.load_table(vllm_exact.TABLES["mi355x"])
    gen = torch.Generator(device=DEV).manual_seed(11)
    try:
        yield bench.DecodeStep(torch, plugin, P, torch.device(DEV), gen, keep_bf16=False), gen
    finally:
        plugin.F, plugin.TRUNC, P.MAX_LEN = saved
        plugin.load_table(None)
        torch.cuda.empty_cache()


@pytest.mark.parametrize("B,L", bench.DECODE_CASES)
def test_full_decode_step_logits_are_batch_invariant(full_model, B, L):
    model, gen = full_model
    assert len(model.layers) == bench.LAYERS
    print(f"full decode step B={B} L={L}", flush=True)
    caches, bt, _ = model.kv(B, L, gen)
    sl = torch.randint(L // 2, L + 1, (B,), device=DEV, generator=gen, dtype=torch.int32)
    h0 = torch.randn(B, bench.HIDDEN, device=DEV, generator=gen).to(torch.bfloat16)
    full = model.step(h0, caches, bt, sl)
    assert full.shape == (B, bench.VOCAB) and torch.isfinite(full.float()).all()
    for i in (0, B // 2, B - 1):
        assert torch.equal(model.step(h0[i:i + 1], caches, bt[i:i + 1], sl[i:i + 1]), full[i:i + 1]), i
    sel = torch.tensor([B - 1, B // 3, 0], device=DEV)
    assert torch.equal(model.step(h0[sel], caches, bt[sel].contiguous(), sl[sel].contiguous()), full[sel])
    del caches, bt, sl, full
    torch.cuda.empty_cache()
