"""Pins the CPU oracle (oracle/) before anything is checked against it.

The reference ships no golden vectors (its tests are property tests with seeded RNG), so
every oracle function is pinned here by checks a plausible mistake would fail:
* digitize: hand-computed known answers (scale, truncation toward zero, balanced and offset
  digit split, carries at +-128, zero rows, power-of-two maxima), Python's math.frexp,
  the reference's reconstruction property (tests/test_reference_cpu.py:16-23), digit ranges;
* exact matmul: exact-integer brute force on the reconstructed fixed-point values (a
  different formula from the digit-sum one the oracle uses), a hand-made round-to-even tie,
  the reference's float-error, row-independence and K-split properties
  (tests/test_reference_cpu.py:26-60);
* bf16 rounding: known ties and torch's own float -> bf16 conversion;
* attention: one key, zero query, two keys in closed form, scipy's softmax, page
  permutation.
"""
import math
from fractions import Fraction

import numpy as np
import pytest
import scipy.special
import torch

import oracle
from helpers import make_paged, xw

DIGITIZERS = [oracle.digitize_np, oracle.digitize_c]


# ------------------------------------------------------------------ digitize known answers
@pytest.mark.parametrize("dig", DIGITIZERS)
def test_digitize_known_answers_f14(dig):
    x = np.array([[1.0, -0.75, 0.5, 3.0e-5, -1.0],
                  [100.0, 1.0, -0.3, 0.0, 0.0],
                  [0.0, 0.0, 0.0, 0.0, 0.0],
                  [0.25, -0.125, 0.0, 0.0, 0.0],
                  [np.float32(0.99999994), 0.0, 0.0, 0.0, 0.0],
                  [1.0, -1.5 / 8192, 0.0, 0.0, 0.0]], np.float32)
    h, l, cs, sh = dig(x, 14)
    # row 0: absmax 1 = 0.5 * 2^1 -> e = 1, sh = 13, q = trunc(x * 8192)
    assert sh[0] == 13
    assert h[0].tolist() == [32, -24, 16, 0, -32] and l[0].tolist() == [0, 0, 0, 0, 0]
    # row 1: absmax 100 -> e = 7, sh = 7, q = [12800, 128, -38]: 128 = 256*1 - 128 (carry)
    assert sh[1] == 7
    assert h[1, :3].tolist() == [50, 1, 0] and l[1, :3].tolist() == [0, -128, -38]
    # zero row: e = 0, sh = F, all digits 0
    assert sh[2] == 14 and not h[2].any() and not l[2].any()
    # power-of-two absmax 2^-2 -> e = -1, sh = 15, q = 8192 = 2^(F-1)
    assert sh[3] == 15 and h[3, 0] == 32 and l[3, 0] == 0 and h[3, 1] == -16
    # largest float below 1: q = 2^14 - 1 = 16383 = 256*64 - 1 (h reaches its bound 64)
    assert sh[4] == 14 and h[4, 0] == 64 and l[4, 0] == -1
    # truncation toward zero: -1.5 -> -1 (not -2)
    assert h[5, 1] == 0 and l[5, 1] == -1
    assert not cs.any()


@pytest.mark.parametrize("dig", DIGITIZERS)
def test_digitize_known_answers_f15(dig):
    x = np.array([[100.0, 1.0, -0.3], [0.0, 0.0, 0.0]], np.float32)
    h, l, cs, sh = dig(x, 15)
    # absmax 100 -> e = 7, sh = 8, q = [25600, 256, -76]; offset digits q = 256h + l + 128
    assert sh[0] == 8
    assert h[0].tolist() == [100, 1, -1] and l[0].tolist() == [-128, -128, 52]
    assert cs[0] == 25396  # = sum(q) - 128 K
    # zero row: q = 0 -> l = -128, h = 0, cs = -128 K
    assert h[1].tolist() == [0, 0, 0] and l[1].tolist() == [-128, -128, -128] and cs[1] == -384


@pytest.mark.parametrize("F", [14, 15])
@pytest.mark.parametrize("dig", DIGITIZERS)
def test_digitize_properties(dig, F):
    x, _ = xw(7, 33, 512)
    x = x.numpy()
    h, l, cs, sh = dig(x, F)
    off = 128 if F == 15 else 0
    q = 256 * h.astype(np.int64) + l.astype(np.int64) + off
    # shift from Python's frexp of the row absmax
    for r in range(x.shape[0]):
        assert sh[r] == F - math.frexp(float(np.abs(x[r]).max()))[1]
    # q == trunc(x * 2^sh) exactly, checked with exact rationals on a sample of entries
    for r in range(x.shape[0]):
        for k in range(0, x.shape[1], 37):
            v = Fraction(float(x[r, k])) * Fraction(2) ** int(sh[r])
            assert q[r, k] == math.trunc(v)
    # the reference's reconstruction bound
    err = np.abs(q * np.exp2(-sh.astype(np.float64))[:, None] - x).max(1) / np.abs(x).max(1)
    assert err.max() < 2.0 ** -(F - 1)
    # digit ranges and |q| < 2^F
    assert np.abs(q).max() < 2 ** F
    if F == 15:
        assert h.min() >= -128 and h.max() <= 127
        assert (cs == (q - 128).sum(1)).all()
    else:
        assert h.min() >= -64 and h.max() <= 64
        assert not cs.any()
    assert l.min() >= -128 and l.max() <= 127


def test_digitize_restatements_agree():
    from vllm_exact import kernels as K

    for seed in range(3):
        x, w = xw(9, 70, 1000, seed=seed)
        for F in (14, 15):
            for t in (x, w, x.to(torch.bfloat16).float(), x * 1e-30, x * 1e30):
                a = oracle.digitize_np(t.numpy(), F)
                b = oracle.digitize_c(t.numpy(), F)
                c = [u.numpy() for u in K.digitize_torch(t, F)]
                for u, v, s in zip(a, b, c):
                    assert np.array_equal(u, v) and np.array_equal(u, s)


# ------------------------------------------------------------------ exact matmul
def _rand_digits(rng, R, K, F):
    hmax = 64 if F == 14 else 127
    hmin = -64 if F == 14 else -128
    h = rng.integers(hmin, hmax + 1, size=(R, K)).astype(np.int8)
    l = rng.integers(-128, 128, size=(R, K)).astype(np.int8)
    sh = rng.integers(-20, 40, size=R).astype(np.int32)
    if F == 15:
        cs = (256 * h.astype(np.int64) + l).sum(1).astype(np.int32)
    else:
        cs = np.zeros(R, np.int32)
    return h, l, cs, sh


@pytest.mark.parametrize("F,trunc", [(14, False), (14, True), (15, False), (15, True)])
def test_exact_linear_brute_force(F, trunc):
    """y = fp32( sum_k qx*qw [- sum_k lx*lw when truncated] * 2^-(sx+sw) ) with q rebuilt from the
    digits and the sum taken over Python integers: a different formula from the oracle's
    digit-plane sums, so a wrong shift, dropped cross term or offset term fails here."""
    rng = np.random.default_rng(F * 10 + trunc)
    M, N, K = 5, 7, 96
    xd = _rand_digits(rng, M, K, F)
    wd = _rand_digits(rng, N, K, F)
    off = 128 if F == 15 else 0
    qx = 256 * xd[0].astype(object) + xd[1].astype(object) + off
    qw = 256 * wd[0].astype(object) + wd[1].astype(object) + off
    for impl in (oracle.exact_linear_np, oracle.exact_linear_c):
        y = impl(xd, wd, F, trunc)
        for i in range(M):
            for j in range(N):
                tot = sum(int(a) * int(b) for a, b in zip(qx[i], qw[j]))
                if trunc:
                    tot -= sum(int(a) * int(b) for a, b in zip(xd[1][i], wd[1][j]))
                val = Fraction(tot) * Fraction(2) ** int(-(xd[3][i] + wd[3][j]))
                assert y[i, j] == np.float32(float(val)), (impl.__name__, i, j)


def test_exact_linear_round_to_even_tie():
    # tot = 16384*1024 + 1 = 2^24 + 1 sits exactly between two fp32 values: RNE gives 2^24.
    xd = (np.array([[64, 0]], np.int8), np.array([[0, 1]], np.int8), np.zeros(1, np.int32), np.zeros(1, np.int32))
    wd = (np.array([[4, 0]], np.int8), np.array([[0, 1]], np.int8), np.zeros(1, np.int32), np.zeros(1, np.int32))
    for impl in (oracle.exact_linear_np, oracle.exact_linear_c):
        assert impl(xd, wd, 14, False)[0, 0] == np.float32(2 ** 24)
        assert impl(xd, wd, 14, True)[0, 0] == np.float32(2 ** 24)  # ll = 1 dropped
    # tot = 2^24 + 3 rounds up to 2^24 + 4
    xd2 = (xd[0], np.array([[0, 3]], np.int8), xd[2], xd[3])
    assert oracle.exact_linear_c(xd2, wd, 14, False)[0, 0] == np.float32(2 ** 24 + 4)


def test_exact_linear_close_to_float():
    """tests/test_reference_cpu.py:26-34: relative error below 1e-3 without outliers."""
    x, w = xw(7, 33, 512, outlier=False)
    ref = x.double().numpy() @ w.double().numpy().T
    for F, tr in ((15, False), (14, True), (14, False)):
        y = oracle.exact_linear_c(oracle.digitize_c(x.numpy(), F), oracle.digitize_c(w.numpy(), F), F, tr)
        rel = np.abs(y - ref).max() / np.abs(ref).max()
        assert rel < 1e-3, (F, tr, rel)


def test_rows_independent():
    """tests/test_reference_cpu.py:37-46: a row alone gives the bits it gets inside the batch."""
    x, w = xw(9, 33, 512)
    for F, tr in ((15, False), (14, True)):
        wd = oracle.digitize_c(w.numpy(), F)
        full = oracle.exact_linear_c(oracle.digitize_c(x.numpy(), F), wd, F, tr)
        for i in (0, 4, 8):
            one = oracle.exact_linear_c(oracle.digitize_c(x[i:i + 1].numpy(), F), wd, F, tr)
            assert np.array_equal(one[0].view(np.uint32), full[i].view(np.uint32))


def test_k_split_is_exact():
    """tests/test_reference_cpu.py:49-60: integer partial sums over K slices add up exactly."""
    x, w = xw(7, 33, 1024)
    xd, wd = oracle.digitize_np(x.numpy(), 14), oracle.digitize_np(w.numpy(), 14)
    whole = oracle.exact_tot_np(xd, wd, 14, True)
    parts = 0
    for s in (slice(0, 300), slice(300, 777), slice(777, 1024)):
        parts = parts + oracle.exact_tot_np(tuple(t[:, s] for t in xd[:2]) + xd[2:],
                                            tuple(t[:, s] for t in wd[:2]) + wd[2:], 14, True)
    assert np.array_equal(whole, parts)


def test_exact_entries_match_full():
    x, w = xw(6, 50, 640, seed=3)
    for F, tr in ((14, True), (15, False)):
        xd, wd = oracle.digitize_c(x.numpy(), F), oracle.digitize_c(w.numpy(), F)
        full = oracle.exact_linear_c(xd, wd, F, tr)
        rows = np.array([0, 5, 3, 2]), np.array([49, 0, 17, 33])
        assert np.array_equal(oracle.exact_entries_c(xd, wd, F, tr, *rows), full[rows])


# ------------------------------------------------------------------ bf16 rounding
def test_bf16_known_ties():
    vals = np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8 + 2 ** -20), 0.0, -0.0, np.inf, -np.inf],
                    np.float32)
    want = [0x3F80, 0x3F82, 0xBF81, 0x0000, 0x8000, 0x7F80, 0xFF80]
    for impl in (oracle.bf16_rne_np, oracle.bf16_rne_c):
        assert impl(vals).tolist() == want
    assert oracle.bf16_rne_c(np.array([np.nan], np.float32)).tolist() == [0x7FC0]


def test_bf16_matches_torch():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    vals = vals[~np.isnan(vals)]
    vals = np.concatenate([vals, rng.standard_normal(1 << 16).astype(np.float32),
                           np.array([3.3895314e38, 1e-40, -1e-45], np.float32)])
    want = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.bf16_rne_np(vals), want)
    assert np.array_equal(oracle.bf16_rne_c(vals), want)


# ------------------------------------------------------------------ attention
def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _case(B=3, L=70, BS=16, H=8, KV=2, D=32, seed=0):
    q, kv, bt, sl = make_paged(B, L, BS, H, KV, D, seed=seed)
    kc, vc = kv.transpose(1, 2).split(D, dim=-1)
    return _bits(q), _bits(kc), _bits(vc), bt.numpy(), sl.numpy()


@pytest.mark.parametrize("impl", [oracle.paged_decode_np, oracle.paged_decode_c])
def test_attention_special_cases(impl):
    q, kc, vc, bt, sl = _case()
    vf = oracle.bf16_bits_to_f32(vc).astype(np.float64)
    # one key: softmax of a single logit is 1, the output is that key's value row
    sl1 = np.ones_like(sl)
    out = impl(q, kc, vc, bt, sl1, 0.125, 3)
    for b in range(3):
        page = bt[b, 0]
        for h in range(8):
            assert np.array_equal(out[b, h], vf[page, 0, h // 4])
    # zero query: uniform weights, the output is the mean value row
    qz = np.zeros_like(q)
    out = impl(qz, kc, vc, bt, sl, 0.125, 3)
    for b in range(3):
        L = sl[b]
        pos = np.arange(L)
        rows = vf[bt[b, pos // 16], pos % 16]
        for h in range(8):
            np.testing.assert_allclose(out[b, h], rows[:, h // 4].mean(0), rtol=1e-12, atol=1e-14)


def test_attention_two_keys_closed_form():
    q, kc, vc, bt, sl = _case(B=1)
    qf = oracle.bf16_bits_to_f32(q).astype(np.float64)
    kf = oracle.bf16_bits_to_f32(kc).astype(np.float64)
    vf = oracle.bf16_bits_to_f32(vc).astype(np.float64)
    sl2 = np.array([2], np.int32)
    p0, p1 = bt[0, 0], bt[0, 0]
    for impl in (oracle.paged_decode_np, oracle.paged_decode_c):
        out = impl(q, kc, vc, bt, sl2, 0.5, 1)
        for h in range(8):
            g = h // 4
            s0 = 0.5 * kf[p0, 0, g] @ qf[0, h]
            s1 = 0.5 * kf[p1, 1, g] @ qf[0, h]
            w1 = 1.0 / (1.0 + math.exp(s0 - s1))
            want = (1 - w1) * vf[p0, 0, g] + w1 * vf[p1, 1, g]
            np.testing.assert_allclose(out[0, h], want, rtol=1e-12, atol=1e-14)


def test_attention_matches_scipy_and_restatements():
    q, kc, vc, bt, sl = _case(B=4, L=200, BS=16, H=8, KV=2, D=64, seed=1)
    a = oracle.paged_decode_np(q, kc, vc, bt, sl, 0.125, 4)
    c = oracle.paged_decode_c(q, kc, vc, bt, sl, 0.125, 4)
    np.testing.assert_allclose(a, c, rtol=1e-12, atol=1e-14)
    qf = oracle.bf16_bits_to_f32(q).astype(np.float64)
    kf = oracle.bf16_bits_to_f32(kc).astype(np.float64)
    vf = oracle.bf16_bits_to_f32(vc).astype(np.float64)
    for b in range(4):
        L = sl[b]
        pos = np.arange(L)
        k = kf[bt[b, pos // 16], pos % 16]
        v = vf[bt[b, pos // 16], pos % 16]
        for h in range(8):
            p = scipy.special.softmax(0.125 * (k[:, h // 4] @ qf[b, h]))
            np.testing.assert_allclose(c[b, h], p @ v[:, h // 4], rtol=1e-10, atol=1e-13)


def test_attention_page_permutation_invariant():
    q, kc, vc, bt, sl = _case(B=2, L=90, BS=16, H=4, KV=1, D=32, seed=2)
    base = oracle.paged_decode_c(q, kc, vc, bt, sl, 0.2, 2)
    rng = np.random.default_rng(0)
    perm = rng.permutation(kc.shape[0])
    kc2 = np.empty_like(kc)
    vc2 = np.empty_like(vc)
    kc2[perm] = kc
    vc2[perm] = vc
    moved = oracle.paged_decode_c(q, kc2, vc2, perm[bt].astype(np.int32), sl, 0.2, 2)
    assert np.array_equal(base, moved)
