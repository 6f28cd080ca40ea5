"""HIP-graph capture of the decode path: the exactmm::linear op (one launch at 1 row, digitize
+ split-K GEMM + finalize at 64 rows, with the shipped table's cfgs), the multi-segment paged
decode, and the prefix launch whose count install() computes on the GPU. The graph is
replayed several times with new inputs copied in eagerly between replays (and a changed
decode count), and every replay must equal the eager result bit for bit."""
import numpy as np
import pytest
import torch

import vllm_exact
from helpers import kv_views, make_paged
from vllm_exact import paged_attn as P
from vllm_exact import plugin

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_graph_replays_equal_eager():
    N, Kd = 4096, 12288
    plugin.load_table(vllm_exact.TABLES["mi355x"])
    try:
        assert plugin._one_launch(1, N, Kd) and not plugin._one_launch(64, N, Kd)
        assert plugin._cfg(64, N, Kd)[6] > 1  # split-K: partials, then the finalize kernel
        g = torch.Generator().manual_seed(17)
        w = (torch.randn(N, Kd, generator=g) * 0.02).to(torch.bfloat16)
        wbuf = plugin.pack_weight(w.to(DEV))
        xs = {m: torch.empty(m, Kd, device=DEV, dtype=torch.bfloat16) for m in (1, 64)}
        B, H, KV, D = 6, 8, 2, 128
        q0, kv, bt, sl = make_paged(B, 5000, 16, H, KV, D, seed=3)
        q = q0.to(DEV)
        kv, bt, sl = kv.to(DEV), bt.to(DEV), sl.to(DEV)
        kc, vc = kv_views(kv, D)
        qsl = torch.zeros(B + 1, dtype=torch.int32, device=DEV)
        scale = D ** -0.5
        max_len = int(sl.max())  # host value read before capture (paged_decode ignores it)

        def step():
            ys = [torch.ops.exactmm.linear(xs[m], *wbuf) for m in (1, 64)]
            full = torch.empty(B, H, D, device=DEV)
            P.paged_decode(q, kc, vc, bt, sl, scale, full, B, max_len)
            part = torch.full((B, H, D), float("nan"), device=DEV)
            P.paged_decode(q, kc, vc, bt, sl, scale, part, B, max_len, n_live=P.leading_decodes(qsl))
            return ys + [full, part]

        def refill(trial):
            for m, x in xs.items():
                x.copy_((torch.randn(m, Kd, generator=g) * (1 + trial)).to(torch.bfloat16))
            q.copy_(torch.randn(B, H, D, generator=g).to(torch.bfloat16))
            lens = [1] * (trial + 1) + [5] * (B - trial - 1)  # trial + 1 leading decodes
            qsl.copy_(torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32))

        refill(0)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            captured = step()
        for trial in range(3):
            refill(trial)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            eager = step()
            torch.cuda.synchronize()
            for i, (a, b) in enumerate(zip(captured[:3], eager[:3])):
                assert torch.equal(a.view(torch.int16 if a.dtype == torch.bfloat16 else torch.int32),
                                   b.view(torch.int16 if b.dtype == torch.bfloat16 else torch.int32)), (trial, i)
            live = trial + 1
            assert torch.equal(captured[3][:live].view(torch.int32), eager[2][:live].view(torch.int32)), trial
            assert torch.isnan(captured[3][live:]).all(), trial
        del graph
    finally:
        plugin.load_table(None)
