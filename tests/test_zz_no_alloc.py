"""vxa_exact_linear_op_noalloc, the exactmm::linear op with no allocation (digits and split-K
partials in the library's fixed per-GPU scratch), called through the C ABI: its output equals
that of vxa_digitize_packed + vxa_exact_linear_packed with caller-allocated buffers, bit for
bit, on two calls in a row (the second smaller, so it runs on what the first left in the
scratch), at F = 14 and F = 15, and both equal the oracle."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from vllm_exact import _native as nx
from vllm_exact import kernels as K
from vllm_exact import plugin

pytestmark = pytest.mark.gpu
DEV = "cuda"


def noalloc(x, wp, K_, F, trunc, out, cfg):
    pw, cw, sw = wp
    arr, n = nx.cfg_array(cfg)
    M, N = x.shape[0], sw.numel()
    nx.check(nx.lib().vxa_exact_linear_op_noalloc(
        x.data_ptr(), nx.dtype_enum(x.dtype), x.stride(0), pw.data_ptr(), cw.data_ptr(), sw.data_ptr(),
        out.data_ptr(), nx.dtype_enum(out.dtype), out.stride(0), M, N, K_, int(F), int(bool(trunc)), arr, n,
        nx.stream_handle(x.device)), "exact_linear_op_noalloc")
    return out


@pytest.mark.parametrize("F,trunc", [(14, True), (15, False)])
def test_noalloc_op_matches_the_allocating_entry_points(F, trunc):
    g = torch.Generator().manual_seed(40 + F)
    # (M, N, K, cfg): a split-K plan over 64 rows of the down shape, then a smaller call
    cases = [(64, 4096, 12288, (64, 64, 128, 4, 1, 8, 4)), (16, 1000, 4096, (16, 64, 128, 8, 1, 8, 2)),
             (3, 200, 1000, (16, 64, 128, 4, 1, 8, 1))]
    for M, N, Kd, cfg in cases:
        print(f"noalloc F={F} M={M} N={N} K={Kd} cfg={cfg}", flush=True)
        x = (torch.randn(M, Kd, generator=g) * 3).to(torch.bfloat16)
        w = (torch.randn(N, Kd, generator=g) * 0.02).to(torch.bfloat16)
        wp = K.digitize_packed(w.to(DEV), F)
        xg = x.to(DEV)
        _, _, ws_bytes = nx.exact_plan(M, N, ((Kd + 63) // 64) * 64, cfg)
        assert (ws_bytes > 0) == (cfg[6] > 1)
        want = K.exact_linear_packed(K.digitize_packed(xg, F), wp, Kd, F, trunc,
                                     out=torch.empty(M, N, device=DEV, dtype=torch.bfloat16), cfg=cfg)
        got = noalloc(xg, wp, Kd, F, trunc, torch.full((M, N), float("nan"), device=DEV, dtype=torch.bfloat16), cfg)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (M, N, Kd, cfg)
        rows = np.array([0, M // 2, M - 1])
        ref = oracle.exact_linear_c(oracle.digitize_c(x.float().numpy()[rows], F),
                                    oracle.digitize_c(w.float().numpy(), F), F, trunc)
        bits = got.cpu().view(torch.int16).numpy().view(np.uint16)[rows]
        assert np.array_equal(bits, oracle.bf16_rne_c(ref).reshape(len(rows), N)), (M, N, Kd)


def test_noalloc_op_fp32_output_and_fp32_input():
    """fp32 activations and an fp32 output through the same scratch, against the op's bits."""
    g = torch.Generator().manual_seed(7)
    M, N, Kd, cfg = 40, 640, 2048, (64, 64, 128, 4, 1, 8, 2)
    x = torch.randn(M, Kd, generator=g).to(DEV)
    w = (torch.randn(N, Kd, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wp = K.digitize_packed(w, plugin.F)
    want = K.exact_linear_packed(K.digitize_packed(x, plugin.F), wp, Kd, plugin.F, plugin.TRUNC, cfg=cfg)
    got = noalloc(x, wp, Kd, plugin.F, plugin.TRUNC, torch.empty(M, N, device=DEV), cfg)
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_noalloc_op_under_graph_capture():
    """The entry point captured in a HIP graph: one warm call outside capture, then the call
    captured; each replay (after new activations are copied in, with eager work and a
    synchronisation between replays) equals exact_linear_packed on the same input, and the
    captured call allocates nothing (torch's allocated bytes grow by no more than an empty
    capture makes them grow)."""
    g = torch.Generator().manual_seed(11)
    M, N, Kd, F, trunc, cfg = 24, 768, 4096, 14, True, (16, 64, 128, 4, 1, 8, 2)
    w = (torch.randn(N, Kd, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wp = K.digitize_packed(w, F)
    x = torch.empty(M, Kd, device=DEV, dtype=torch.bfloat16)
    out = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
    x.copy_(torch.randn(M, Kd, generator=g).to(torch.bfloat16))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        noalloc(x, wp, Kd, F, trunc, out, cfg)  # warm call: looks up the scratch address
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    # Capturing a graph costs torch a few bytes of its own (the RNG state it keeps per graph):
    # measured on an empty capture, after a first capture has paid any one-time cost.
    empties = [torch.cuda.CUDAGraph() for _ in range(2)]
    with torch.cuda.graph(empties[0]):
        pass
    before = torch.cuda.memory_allocated()
    with torch.cuda.graph(empties[1]):
        pass
    capture_cost = torch.cuda.memory_allocated() - before
    graph = torch.cuda.CUDAGraph()
    before = torch.cuda.memory_allocated()
    with torch.cuda.graph(graph):
        noalloc(x, wp, Kd, F, trunc, out, cfg)
    assert torch.cuda.memory_allocated() - before == capture_cost
    for rep in range(3):
        print(f"noalloc graph replay {rep}", flush=True)
        x.copy_((torch.randn(M, Kd, generator=g) * (rep + 1)).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        want = K.exact_linear_packed(K.digitize_packed(x, F), wp, Kd, F, trunc,
                                     out=torch.empty(M, N, device=DEV, dtype=torch.bfloat16), cfg=cfg)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), rep
    del graph, empties
