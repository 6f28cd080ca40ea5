"""GPU check of the decode-step emulation (the ~9B hybrid's exact linears, paged decode
attention and exact lm_head, as bench.py times it): the logits of every request are bitwise
the same whether it runs alone, inside the full batch, or in a batch of another order and
size. Reduced to 4 layers (one attention layer) and a 2048-row lm_head, with ragged
context lengths, so it runs in seconds.
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


def test_decode_step_logits_are_batch_invariant():
    plugin.F, plugin.TRUNC = 14, True
    P.MAX_LEN = 4096
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
