"""GPU parity of the exact GEMM path against the CPU oracle (bitwise).

Restates the reference's tests/test_gpu.py:13-43 (every tiling and split-K partition equals
the CPU integer reference; bf16 output equals the fp32 output cast to bf16; bf16 input
digitizes like its fp32 upcast) and extends them to the decode shapes of a ~9B model:
* M=16, K=N=4096, 4 dots, no split-K (CPU-runnable configuration): full output;
* decode-shaped QKV/O/gate_up/down at M in {1, 16, 64, 256}, 3 and 4 dots, every split-K
  factor in {1, 2, 4, 8} and every tile config: all bits equal each other and the oracle
  (full outputs for M <= 64, sampled rows at M = 256: rows are independent);
* exact lm_head N=151936 with per-row scales 10^U(-2, 2): digits in full, output rows sampled.
"""
import itertools

import numpy as np
import pytest
import torch

import oracle
from helpers import f32_bits, np_digits, stress_xw, xw
from vllm_exact import kernels as K

pytestmark = pytest.mark.gpu
DEV = "cuda"

REF_CFGS = ((16, 64, 128, 4, 3, 8), (64, 128, 128, 4, 4, 8), (16, 128, 256, 8, 3, 8))  # tests/test_gpu.py:27
OWN_CFGS = ((16, 64, 128, 8, 1, 8), (16, 256, 128, 4, 1, 8), (32, 128, 128, 8, 1, 8), (64, 64, 128, 4, 1, 8),
            (16, 16, 128, 16, 4, 8), (32, 32, 128, 8, 2, 8), (64, 32, 128, 8, 1, 8), (128, 128, 128, 4, 4, 8),
            (64, 64, 128, 4, 8, 8), (128, 64, 128, 4, 6, 8))


def _bf16_of(ref_f32):
    return oracle.bf16_rne_c(ref_f32).reshape(ref_f32.shape)


def _gpu_bf16_bits(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


# ------------------------------------------------------------------ digitize
@pytest.mark.parametrize("F", [14, 15])
def test_digitize_bf16_input(F):
    """tests/test_gpu.py:35-43: bf16 in == fp32 upcast in == the oracle."""
    g = torch.Generator().manual_seed(1)
    xb = (torch.randn(300, 4096, generator=g) * 3).to(torch.bfloat16)
    got_b = np_digits(K.digitize(xb.to(DEV), F))
    got_f = np_digits(K.digitize(xb.float().to(DEV).contiguous(), F))
    want = oracle.digitize_c(xb.float().numpy(), F)
    for a, b, c in zip(got_b, got_f, want):
        assert np.array_equal(a, b) and np.array_equal(a, c)


@pytest.mark.parametrize("F", [14, 15])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("R,Kd", [(16, 4096), (7, 1000), (1, 12288), (33, 24), (5, 1001), (3, 40000), (2, 40001)])
def test_digitize_matches_oracle(F, dtype, R, Kd):
    x, _ = xw(R, 1, Kd, seed=R + Kd)
    x[0] = 0.0  # zero row
    if R > 2:
        x[1] = 0.0
        x[1, Kd // 2] = -0.25  # power-of-two absmax, negative
        x[2, -1] = 1e4  # single large outlier
    if dtype == torch.float16:
        x = x.clamp(-6e4, 6e4)
    xt = x.to(dtype)
    got = np_digits(K.digitize(xt.to(DEV), F))
    want = oracle.digitize_c(xt.float().numpy(), F)
    for a, b in zip(got, want):
        assert np.array_equal(a, b)


def test_digitize_strided_rows():
    x, _ = xw(9, 1, 2048, seed=11)
    big = torch.zeros(9, 2304)
    big[:, :2048] = x
    view = big.to(DEV)[:, :2048]  # row stride 2304 elements
    got = np_digits(K.digitize(view, 14))
    want = oracle.digitize_c(x.numpy(), 14)
    for a, b in zip(got, want):
        assert np.array_equal(a, b)


# ------------------------------------------------------------------ exact GEMM
@pytest.mark.parametrize("F,tr", [(14, True), (15, False), (14, False), (15, True)])
@pytest.mark.parametrize("M,N,Kd", [(24, 384, 4096), (5, 200, 12288), (1, 64, 4096), (300, 256, 12288),
                                    (7, 201, 4096)])
def test_exact_linear_split_k_bitwise(F, tr, M, N, Kd):
    """tests/test_gpu.py:13-32: every cfg x SK x mma equals the CPU integer reference. An odd N
    takes the split-K finalize's one-column loads."""
    x, w = stress_xw(M, N, Kd)
    xd, wd = K.digitize(x.to(DEV), F), K.digitize(w.to(DEV), F)
    ref = oracle.exact_linear_c(np_digits(xd), np_digits(wd), F, tr)
    ref_bits, ref_bf16 = f32_bits(ref), _bf16_of(ref)
    for sk, mma in itertools.product((1, 2, 4, 8), (0, 1)):
        for base in REF_CFGS + OWN_CFGS:
            cfg = base + (sk, mma)
            y = K.exact_linear(xd, wd, F, tr, cfg=cfg)
            assert np.array_equal(f32_bits(y.cpu().numpy()), ref_bits), cfg
            yb = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
            K.exact_linear(xd, wd, F, tr, out=yb, cfg=cfg)
            assert np.array_equal(_gpu_bf16_bits(yb), ref_bf16), cfg


def test_exact_linear_fp16_and_strided_output():
    x, w = stress_xw(9, 300, 4096, seed=2)
    xd, wd = K.digitize(x.to(DEV), 15), K.digitize(w.to(DEV), 15)
    ref = oracle.exact_linear_c(np_digits(xd), np_digits(wd), 15, False)
    yh = torch.empty(9, 300, device=DEV, dtype=torch.float16)
    K.exact_linear(xd, wd, 15, False, out=yh, cfg=(16, 64, 128, 4, 1, 8, 2))
    assert torch.equal(yh.cpu(), torch.from_numpy(ref).to(torch.float16))
    wide = torch.zeros(9, 512, device=DEV)
    K.exact_linear(xd, wd, 15, False, out=wide[:, 100:400], cfg=(32, 128, 128, 8, 1, 8, 1))
    assert np.array_equal(f32_bits(wide[:, 100:400].cpu().numpy()), f32_bits(ref))
    assert not wide[:, :100].any() and not wide[:, 400:].any()


def test_exact_linear_ragged_k_scalar_path():
    """K not a multiple of 64 takes the scalar kernel: same bits."""
    x, w = stress_xw(6, 90, 1000, seed=4)
    for F, tr in ((14, True), (15, False)):
        xd, wd = K.digitize(x.to(DEV), F), K.digitize(w.to(DEV), F)
        ref = f32_bits(oracle.exact_linear_c(np_digits(xd), np_digits(wd), F, tr))
        for cfg in ((16, 64, 128, 4, 1, 8, 1), (16, 64, 128, 4, 1, 8, 3)):
            assert np.array_equal(f32_bits(K.exact_linear(xd, wd, F, tr, cfg=cfg).cpu().numpy()), ref)


def test_exact_linear_rows_past_grid_y_limit_split_k():
    """66000 rows with split-K 2: the finalize grid covers at most 65535 rows per y and strides
    over the rest; every row equals the oracle."""
    x, w = stress_xw(66000, 18, 256, seed=5)
    F, tr = 14, True
    xd, wd = K.digitize(x.to(DEV), F), K.digitize(w.to(DEV), F)
    ref = f32_bits(oracle.exact_linear_c(np_digits(xd), np_digits(wd), F, tr))
    for cfg in ((16, 16, 128, 4, 1, 8, 2), (64, 64, 128, 4, 4, 8, 2)):
        assert np.array_equal(f32_bits(K.exact_linear(xd, wd, F, tr, cfg=cfg).cpu().numpy()), ref), cfg


def test_config1_single_linear_bitwise():
    """M=16, K=N=4096, bf16 x ~ N(0,1), w ~ N(0,0.02), seed 0, F=14 4 dots, no split-K."""
    x, w = xw(16, 4096, 4096, seed=0, outlier=False)
    xb, wb = x.to(torch.bfloat16), w.to(torch.bfloat16)
    xd, wd = K.digitize(xb.to(DEV), 14), K.digitize(wb.to(DEV), 14)
    for a, b in zip(np_digits(xd), oracle.digitize_c(xb.float().numpy(), 14)):
        assert np.array_equal(a, b)
    for a, b in zip(np_digits(wd), oracle.digitize_c(wb.float().numpy(), 14)):
        assert np.array_equal(a, b)
    ref = oracle.exact_linear_c(np_digits(xd), np_digits(wd), 14, False)
    y = K.exact_linear(xd, wd, 14, False, cfg=(16, 64, 128, 8, 1, 8, 1))
    assert np.array_equal(f32_bits(y.cpu().numpy()), f32_bits(ref))
    yb = torch.empty(16, 4096, device=DEV, dtype=torch.bfloat16)
    K.exact_linear(xd, wd, 14, False, out=yb, cfg=(16, 64, 128, 8, 1, 8, 1))
    assert np.array_equal(_gpu_bf16_bits(yb), _bf16_of(ref))


DECODE_SHAPES = {"qkv": (6144, 4096), "o": (4096, 4096), "gate_up": (24576, 4096), "down": (4096, 12288)}
SWEEP_CFGS = ((16, 64, 128, 4, 1, 8), (16, 16, 128, 16, 4, 8), (16, 32, 128, 8, 2, 8), (16, 256, 128, 8, 1, 8),
              (32, 128, 128, 8, 1, 8), (64, 64, 128, 4, 1, 8), (64, 64, 128, 4, 4, 8), (128, 128, 128, 4, 4, 8),
              (64, 128, 128, 4, 6, 8))


@pytest.mark.parametrize("shape", list(DECODE_SHAPES))
def test_decode_sweep_all_partitions_bitwise(shape):
    N, Kd = DECODE_SHAPES[shape]
    g = torch.Generator().manual_seed(0)
    w = (torch.randn(N, Kd, generator=g) * 0.02).to(torch.bfloat16)
    xs = {M: torch.randn(M, Kd, generator=g).to(torch.bfloat16) for M in (1, 16, 64, 256)}
    for F in (14, 15):
        wd = K.digitize(w.to(DEV), F)
        wd_np = np_digits(wd)
        for a, b in zip(wd_np, oracle.digitize_c(w.float().numpy(), F)):
            assert np.array_equal(a, b)
        for M, x in xs.items():
            xd = K.digitize(x.to(DEV), F)
            xd_np = np_digits(xd)
            for tr in ((True, False) if F == 14 else (False,)):
                outs = []
                for base, sk in itertools.product(SWEEP_CFGS, (1, 2, 4, 8)):
                    outs.append(K.exact_linear(xd, wd, F, tr, cfg=base + (sk,)))
                first = outs[0]
                for o in outs[1:]:
                    assert torch.equal(o.view(torch.int32), first.view(torch.int32))
                got = f32_bits(first.cpu().numpy())
                if M <= 64:
                    ref = oracle.exact_linear_c(xd_np, wd_np, F, tr)
                    assert np.array_equal(got, f32_bits(ref)), (shape, F, tr, M)
                else:
                    rows = np.array([0, 77, 200, 255])
                    sub = tuple(t[rows] for t in xd_np)
                    ref = oracle.exact_linear_c(sub, wd_np, F, tr)
                    assert np.array_equal(got[rows], f32_bits(ref)), (shape, F, tr, M)


@pytest.mark.parametrize("M", [16, 256])
def test_lm_head_wide_n_bitwise(M):
    """Exact lm_head: K=4096, N=151936, bf16 w ~ N(0, 0.02), x rows scaled by 10^U(-2, 2)."""
    N, Kd = 151936, 4096
    g = torch.Generator().manual_seed(0)
    x = torch.randn(M, Kd, generator=g)
    x = x * torch.pow(10.0, torch.rand(M, 1, generator=g) * 4 - 2)
    w = (torch.randn(N, Kd, generator=g) * 0.02).to(torch.bfloat16)
    xb = x.to(torch.bfloat16)
    F = 14
    xd, wd = K.digitize(xb.to(DEV), F), K.digitize(w.to(DEV), F)
    wd_np = np_digits(wd)
    for a, b in zip(wd_np, oracle.digitize_c(w.float().numpy(), F)):
        assert np.array_equal(a, b)
    xd_np = np_digits(xd)
    for tr in (True, False):
        y = K.exact_linear(xd, wd, F, tr, cfg=(16, 64, 128, 8, 1, 8, 1))
        for cfg in ((16, 256, 128, 8, 1, 8, 2), (64, 64, 128, 4, 1, 8, 4), (128, 128, 128, 4, 4, 8, 1),
                    (16, 32, 128, 16, 2, 8, 1)):
            assert torch.equal(K.exact_linear(xd, wd, F, tr, cfg=cfg).view(torch.int32), y.view(torch.int32))
        rows = np.arange(M) if M <= 16 else np.array([0, 1, 128, 255])
        ref = oracle.exact_linear_c(tuple(t[rows] for t in xd_np), wd_np, F, tr)
        got = y.cpu().numpy()[rows]
        assert np.array_equal(f32_bits(got), f32_bits(ref)), tr
        yb = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
        K.exact_linear(xd, wd, F, tr, out=yb, cfg=(16, 64, 128, 8, 1, 8, 1))
        assert np.array_equal(_gpu_bf16_bits(yb)[rows], _bf16_of(ref))


def test_custom_op_bf16_matches_oracle():
    from vllm_exact import plugin

    x, w = xw(37, 512, 4096, seed=9, outlier=False)
    xb, wb = x.to(torch.bfloat16), w.to(torch.bfloat16)
    wd = plugin.digitize_weight_rows(wb.to(DEV))
    y = torch.ops.exactmm.linear(xb.to(DEV).view(37, 1, 4096), *wd)
    assert y.shape == (37, 1, 512) and y.dtype == torch.bfloat16
    ref = oracle.exact_linear_c(oracle.digitize_c(xb.float().numpy(), plugin.F),
                                oracle.digitize_c(wb.float().numpy(), plugin.F), plugin.F, plugin.TRUNC)
    assert np.array_equal(_gpu_bf16_bits(y.view(37, 512)), _bf16_of(ref))
