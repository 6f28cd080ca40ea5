"""GPU parity of the paths a vLLM user runs, at the workload's full sizes.

* the exact lm_head (4096 -> 151936) through the exactmm::linear op on load-time packed
  weights, with the shipped F = 14 table (3 dots) and F = 15 table (offset digits, 4 dots),
  at 16 and 256 rows with per-row activation scales 10^U(-2, 2): every column of sampled rows
  against the oracle;
* the F = 15 table through the op at the four decode-sweep shapes and 1-256 rows, and both
  tables at seeded random batch sizes of 1-512 rows;
* autotune_exact, the reference's path when no cfg is given (kernels.py:267, 292-316);
* the vLLM plugin hooks process_weights_after_loading and apply (plugin.py:87-102), run on
  stand-in vLLM base classes, with a bias and with the lm_head.
"""
import numpy as np
import pytest
import torch

import oracle
import vllm_exact
import vllm_standin
from helpers import f32_bits, np_digits, xw
from vllm_exact import kernels as K
from vllm_exact import plugin

pytestmark = pytest.mark.gpu
DEV = "cuda"
VOCAB, HIDDEN = 151936, 4096
SWEEP = [(6144, 4096), (4096, 4096), (24576, 4096), (4096, 12288)]  # qkv, o, gate_up, down


def bf16_bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def use(monkeypatch, F):
    """Digit format and table of enable(f=F): F = 14 truncated with the F14 table, F = 15 with
    4 dots and the F15 table."""
    monkeypatch.setattr(plugin, "F", F)
    monkeypatch.setattr(plugin, "TRUNC", F == 14)
    tables = vllm_exact.TABLES_F15 if F == 15 else vllm_exact.TABLES
    plugin.load_table(tables["mi355x"])


@pytest.fixture(autouse=True)
def _no_table():
    yield
    plugin.load_table(None)


@pytest.fixture(scope="module")
def lm_weight():
    g = torch.Generator(device=DEV).manual_seed(21)
    w = (torch.randn(VOCAB, HIDDEN, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    return w, w.float().cpu().numpy()


@pytest.mark.parametrize("F", [14, 15])
def test_lm_head_full_width_through_the_op(monkeypatch, lm_weight, F):
    w, w_np = lm_weight
    use(monkeypatch, F)
    wbuf = plugin.pack_weight(w)
    wd_np = oracle.digitize_c(w_np, F)
    g = torch.Generator().manual_seed(F)
    for M in (16, 256):
        scale = 10.0 ** (torch.rand(M, 1, generator=g) * 4 - 2)
        x = (torch.randn(M, HIDDEN, generator=g) * scale).to(torch.bfloat16)
        y = torch.ops.exactmm.linear(x.to(DEV), *wbuf)
        assert y.shape == (M, VOCAB) and y.dtype == torch.bfloat16
        rows = np.array([0, 1, M // 2, M - 1])
        xd_np = oracle.digitize_c(x.float().numpy()[rows], F)
        want = oracle.bf16_rne_c(oracle.exact_linear_c(xd_np, wd_np, F, F == 14)).reshape(len(rows), VOCAB)
        got = bf16_bits(y)[rows]
        assert np.array_equal(got, want), (F, M, plugin._cfg(M, VOCAB, HIDDEN), int((got != want).sum()))


def test_lm_head_column_split_gives_the_one_launch_bits(monkeypatch, lm_weight):
    """The F = 14 table splits the lm_head's columns at 193-256 rows (the whole rounds of
    workgroups, then the rest with a grid of its own): the op's output equals, bit for bit over
    the whole width, one GEMM launch over all columns with the row's cfg."""
    w, _ = lm_weight
    F = 14
    use(monkeypatch, F)
    wbuf = plugin.pack_weight(w)
    g = torch.Generator().manual_seed(30 + F)
    for M in (256, 200):
        split = plugin._n_split(M, VOCAB, HIDDEN)
        assert split is not None and 0 < split[0] < VOCAB, (F, M)
        x = torch.randn(M, HIDDEN, generator=g).to(torch.bfloat16).to(DEV)
        y = torch.ops.exactmm.linear(x, *wbuf)
        whole = torch.empty(M, VOCAB, device=DEV, dtype=torch.bfloat16)
        K.exact_linear_packed(K.digitize_packed(x, F), (wbuf[0], wbuf[2], wbuf[3]), HIDDEN, F, F == 14, out=whole,
                              cfg=plugin._cfg(M, VOCAB, HIDDEN))
        assert torch.equal(y.view(torch.int16), whole.view(torch.int16)), (F, M, split)
    assert all(plugin._n_split(m, VOCAB, HIDDEN) is None for m in (16, 192, 512))


@pytest.mark.parametrize("N,Kd", SWEEP)
def test_f15_table_through_the_op_at_sweep_shapes(monkeypatch, N, Kd):
    use(monkeypatch, 15)
    g = torch.Generator().manual_seed(N + Kd)
    w = (torch.randn(N, Kd, generator=g) * 0.02).to(torch.bfloat16)
    wbuf = plugin.pack_weight(w.to(DEV))
    wd_np = oracle.digitize_c(w.float().numpy(), 15)
    for M in (1, 16, 64, 256):
        x = torch.randn(M, Kd, generator=g).to(torch.bfloat16)
        y = torch.ops.exactmm.linear(x.to(DEV), *wbuf)
        rows = np.arange(M) if M <= 16 else np.array([0, 17, M // 2, M - 1])
        xd_np = oracle.digitize_c(x.float().numpy()[rows], 15)
        want = oracle.bf16_rne_c(oracle.exact_linear_c(xd_np, wd_np, 15, False)).reshape(len(rows), N)
        assert np.array_equal(bf16_bits(y)[rows], want), (M, N, Kd, plugin._cfg(M, N, Kd),
                                                          plugin._one_launch(M, N, Kd))


@pytest.mark.parametrize("F", [14, 15])
def test_both_tables_through_the_op_at_random_batch_sizes(monkeypatch, F):
    """The shipped F = 14 and F = 15 tables through the op at the four decode-sweep shapes, at
    seeded random batch sizes of 1-512 rows (most between the table's buckets, so the lookup
    picks a neighbouring bucket's cfg and, below 17 rows, the one- or two-launch path): the
    first, two random and the last row equal the oracle's bf16 bits."""
    import random

    use(monkeypatch, F)
    rng = random.Random(F)
    g = torch.Generator().manual_seed(F)
    for N, Kd in SWEEP:
        w = (torch.randn(N, Kd, generator=g) * 0.02).to(torch.bfloat16)
        wbuf = plugin.pack_weight(w.to(DEV))
        wd_np = oracle.digitize_c(w.float().numpy(), F)
        for M in sorted(rng.sample(range(1, 513), 4)):
            x = torch.randn(M, Kd, generator=g) * (10.0 ** torch.empty(M, 1).uniform_(-2, 2, generator=g))
            x = x.to(torch.bfloat16)
            y = torch.ops.exactmm.linear(x.to(DEV), *wbuf)
            rows = np.unique(np.array([0, rng.randrange(M), rng.randrange(M), M - 1]))
            xd_np = oracle.digitize_c(x.float().numpy()[rows], F)
            want = oracle.bf16_rne_c(oracle.exact_linear_c(xd_np, wd_np, F, F == 14)).reshape(len(rows), N)
            assert np.array_equal(bf16_bits(y)[rows], want), (F, M, N, Kd, plugin._cfg(M, N, Kd),
                                                              plugin._one_launch(M, N, Kd))


@pytest.mark.parametrize("M,N,Kd", [(16, 512, 1024), (37, 200, 1000)])
def test_autotune_exact_without_cfg(monkeypatch, M, N, Kd):
    """exact_linear with no cfg times the candidate cfgs (kernels.py:292-316), caches the
    fastest for the shape, and gives the oracle's bits; the next call takes the cache."""
    F, tr = 14, True
    x, w = xw(M, N, Kd, seed=M)
    xd, wd = K.digitize(x.to(DEV), F), K.digitize(w.to(DEV), F)
    want = f32_bits(oracle.exact_linear_c(np_digits(xd), np_digits(wd), F, tr))
    key = (M, N, Kd, F, tr)
    K._CFG_CACHE.pop(key, None)
    y = K.exact_linear(xd, wd, F, tr)
    assert np.array_equal(f32_bits(y.cpu().numpy()), want)
    cfg = K._CFG_CACHE[key]
    assert tuple(cfg[:6]) in {tuple(c) for c in K.EXACT_CFGS} and cfg[6] in K.AUTOTUNE_SPLITS
    assert cfg[0] <= max(16, 1 << (M - 1).bit_length())  # the reference's BM filter (kernels.py:298)

    def no_tuning(*a):
        raise AssertionError("the cached cfg should be used")

    monkeypatch.setattr(K, "autotune_exact", no_tuning)
    y2 = K.exact_linear(xd, wd, F, tr)
    assert torch.equal(y2, y)


def test_plugin_methods_process_weights_and_apply(monkeypatch):
    """vLLM's hooks on the plugin's methods: process_weights_after_loading packs a linear
    layer's weight (and frees the bf16 copy when RELEASE_WEIGHTS), apply adds the bias after
    the exact product; the lm_head method keeps its weight. Bits: the oracle's exact product
    rounded to bf16, plus the bias in bf16 as torch adds it."""
    vllm_standin.install(monkeypatch)
    lin_m, head_m, _ = plugin.define_vllm_classes()
    g = torch.Generator().manual_seed(31)
    N, Kd, M = 320, 1024, 5
    w = (torch.randn(N, Kd, generator=g) * 0.02).to(torch.bfloat16)
    b = torch.randn(N, generator=g).to(torch.bfloat16)
    x = torch.randn(M, Kd, generator=g).to(torch.bfloat16)
    exact = oracle.bf16_rne_c(oracle.exact_linear_c(oracle.digitize_c(x.float().numpy(), plugin.F),
                                                    oracle.digitize_c(w.float().numpy(), plugin.F), plugin.F,
                                                    plugin.TRUNC)).reshape(M, N)
    exact_t = torch.from_numpy(exact.view(np.int16)).view(torch.bfloat16)
    for release in (False, True):
        monkeypatch.setattr(plugin, "RELEASE_WEIGHTS", release)
        layer = torch.nn.Linear(Kd, N, bias=True, device=DEV, dtype=torch.bfloat16)
        layer.weight.data.copy_(w)
        layer.bias.data.copy_(b)
        meth = lin_m()
        meth.process_weights_after_loading(layer)
        assert layer.weight.numel() == (0 if release else N * Kd)
        y = meth.apply(layer, x.to(DEV), layer.bias)
        assert np.array_equal(bf16_bits(y), bf16_bits(exact_t + b)), release
        assert np.array_equal(bf16_bits(meth.apply(layer, x.to(DEV))), exact)
    head = torch.nn.Module()
    head.weight = torch.nn.Parameter(w.to(DEV), requires_grad=False)
    hm = head_m()
    hm.process_weights_after_loading(head)
    assert head.weight.numel() == N * Kd  # kept: a tied lm_head shares it with the embedding
    assert np.array_equal(bf16_bits(hm.apply(head, x.to(DEV))), exact)
