"""GPU checks of the fixed-order paged decode attention.

Restates the reference's tests/test_gpu.py:46-78 (error against a float reference,
computing only the first n requests leaves them bitwise unchanged, moving physical pages
with the block table remapped leaves the output bitwise unchanged) and adds the decode
shapes of a ~9B model's full-attention layer (H=32, KV=8, D=128, block size 16 at batch 64 x 8K, 16 x 16K and 256 x 1K), where each
request run alone must give the bits it gets inside mixed batches.

Stated tolerance against the float64 oracle (V ~ N(0, 1) or 0.5 N(0, 1)):
* fp32 output: max |o - o64| <= 2e-5;
* bf16 output: |o - o64| <= 2^-8 |o64| + 2e-5 (one bf16 rounding on top of the fp32 error).
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import bf16_bits, kv_views, make_paged
from vllm_exact import paged_attn as P

pytestmark = pytest.mark.gpu
DEV = "cuda"
ATOL_F32 = 2e-5
RTOL_BF16 = 2.0 ** -8


def _run(q, kv, bt, sl, scale, n, D, out_dtype=torch.float32, **kw):
    kc, vc = kv_views(kv, D)
    out = torch.full((q.shape[0], q.shape[1], D), float("nan"), device=DEV, dtype=out_dtype)
    P.paged_decode(q, kc, vc, bt, sl, scale, out, n, int(sl.max()), **kw)
    return out


def _oracle(q, kv, bt, sl, scale, n, D, rows=None):
    """float64 oracle output for requests `rows` (default 0..n-1), built from the host copies."""
    rows = list(range(n)) if rows is None else list(rows)
    kc, vc = kv_views(kv.cpu(), D)
    qb = bf16_bits(q.cpu()[rows])
    return oracle.paged_decode_c(qb, bf16_bits(kc), bf16_bits(vc), bt.cpu().numpy()[rows], sl.cpu().numpy()[rows],
                                 scale, len(rows))


def _check_tol(got, want):
    err = np.abs(got.astype(np.float64) - want)
    assert err.max() <= ATOL_F32, err.max()


def _check_tol_bf16(got, want):
    err = np.abs(got.astype(np.float64) - want)
    assert (err <= RTOL_BF16 * np.abs(want) + ATOL_F32).all(), (err - RTOL_BF16 * np.abs(want)).max()


@pytest.mark.parametrize("L", [300, 5000])
def test_device_count_limits_the_requests(L):
    """paged_decode with n_live (vxa_paged_decode_prefix): the grid covers n requests, the
    count on the GPU picks the first n_live; those rows are bitwise the plain entry point's
    and the others are never written. L = 5000 spans several segments (merge kernel)."""
    B, H, KV, D = 6, 8, 2, 128
    q, kv, bt, sl = make_paged(B, L, 16, H, KV, D, seed=21)
    q, kv, bt, sl = (t.to(DEV) for t in (q, kv, bt, sl))
    scale = D ** -0.5
    ref = _run(q, kv, bt, sl, scale, B, D)
    kc, vc = kv_views(kv, D)
    for live in (0, 3, 6):
        out = torch.full((B, H, D), float("nan"), device=DEV)
        P.paged_decode(q, kc, vc, bt, sl, scale, out, B, int(sl.max()),
                       n_live=torch.tensor([live], dtype=torch.int32, device=DEV))
        assert torch.equal(out[:live].view(torch.int32), ref[:live].view(torch.int32)), live
        assert torch.isnan(out[live:]).all(), live
    # the count as install() makes it on the GPU: 3 single-token requests, then a prefill
    qsl = torch.tensor([0, 1, 2, 3, 40, 41, 42], dtype=torch.int32, device=DEV)
    n_live = P.leading_decodes(qsl)
    assert n_live.is_cuda and n_live.dtype == torch.int32 and int(n_live) == 3
    out = torch.full((B, H, D), float("nan"), device=DEV)
    P.paged_decode(q, kc, vc, bt, sl, scale, out, B, int(sl.max()), n_live=n_live)
    assert torch.equal(out[:3].view(torch.int32), ref[:3].view(torch.int32)) and torch.isnan(out[3:]).all()
    with pytest.raises(ValueError, match="n_live"):
        P.paged_decode(q, kc, vc, bt, sl, scale, out, B, 0, n_live=torch.tensor([1], device=DEV))


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_length_bound_trims_the_grid_without_changing_bits(out_dtype):
    """max_seq_len as a bound on the batch's lengths (0: none, the grid of MAX_LEN): the grid
    then covers only the segments the bound reaches, 3 of the 8 at 5000 keys and 1 at 2048 (no
    merge launch). Requests within the bound keep the full grid's bits, single- and
    multi-segment alike; a request longer than the bound gets NaN rows and leaves the others
    unchanged. The same through the device-count entry point."""
    B, H, KV, D = 6, 8, 2, 128
    q, kv, bt, sl = make_paged(B, 9000, 16, H, KV, D, seed=31)
    sl = torch.tensor([100, 2048, 2049, 4096, 5000, 9000], dtype=torch.int32)
    q, kv, bt, sl = (t.to(DEV) for t in (q, kv, bt, sl))
    kc, vc = kv_views(kv, D)
    scale = D ** -0.5
    assert P.MAX_LEN == 16384 and P.SPLIT == 2048

    def run(bound, n_live=None):
        out = torch.full((B, H, D), float("nan"), device=DEV, dtype=out_dtype)
        P.paged_decode(q, kc, vc, bt, sl, scale, out, B, bound, n_live=n_live)
        return out.view(torch.int32 if out_dtype == torch.float32 else torch.int16)

    full = run(0)
    assert not torch.isnan(full.view(out_dtype)).any()
    assert torch.equal(run(9000), full)
    assert torch.equal(run(16384), full)
    for bound, within in ((5000, 5), (2048, 2)):
        for n_live in (None, torch.tensor([B], dtype=torch.int32, device=DEV)):
            got = run(bound, n_live)
            assert torch.equal(got[:within], full[:within]), (bound, n_live)
            assert torch.isnan(got[within:].view(out_dtype)).all(), (bound, n_live)
    want = _oracle(q, kv, bt, sl, scale, 5, D)
    got = run(5000)[:5].view(out_dtype).float().cpu().numpy()
    (_check_tol if out_dtype == torch.float32 else _check_tol_bf16)(got, want)


@pytest.mark.parametrize("B,L,BS", [(8, 300, 16), (8, 5000, 528), (4, 9000, 528), (64, 8192, 528), (8, 3000, 8),
                                    (6, 2000, 24)])
def test_paged_attention_reference_cases(B, L, BS):
    """tests/test_gpu.py:57-78: H=16, KV=4, D=256, cache x0.5, scale 1/16. Page sizes 8 and 24
    (below 16, and not a power of two) take the per-key page lookup."""
    H, KV, D = 16, 4, 256
    q, kv, bt, sl = make_paged(B, L, BS, H, KV, D, seed=0, kv_scale=0.5)
    q, kv, bt, sl = q.to(DEV), kv.to(DEV), bt.to(DEV), sl.to(DEV)
    o = _run(q, kv, bt, sl, 1 / 16, B, D)
    n = min(B, 4)
    want = _oracle(q, kv, bt, sl, 1 / 16, n, D)
    _check_tol(o[:n].cpu().numpy(), want)
    ob = _run(q, kv, bt, sl, 1 / 16, B, D, out_dtype=torch.bfloat16)
    _check_tol_bf16(ob[:n].float().cpu().numpy(), want)
    assert torch.equal(ob, o.to(torch.bfloat16))  # bf16 output == fp32 output rounded once
    o2 = _run(q, kv, bt, sl, 1 / 16, n, D)
    assert torch.equal(o[:n], o2[:n])
    g = torch.Generator().manual_seed(3)
    newpos = torch.randperm(kv.shape[0], generator=g).to(DEV)
    kv2 = torch.empty_like(kv)
    kv2[newpos] = kv
    o3 = _run(q, kv2, newpos[bt.long()].to(torch.int32), sl, 1 / 16, B, D)
    assert torch.equal(o, o3)


CONFIG4 = [(64, 8192), (16, 16384), (256, 1024)]


def _gpu_paged(B, L, seed, var_len):
    """Config-4 inputs generated on the device (bf16 N(0,1) K/V and q), block tables from
    random permutations of one shared pool."""
    H, KV, D, BS = 32, 8, 128, 16
    g = torch.Generator(device=DEV).manual_seed(seed)
    nbp = (L + BS - 1) // BS
    nblocks = B * nbp + 8
    kv = torch.randn(nblocks, KV, BS, 2 * D, device=DEV, generator=g, dtype=torch.bfloat16)
    bt = torch.randperm(nblocks, device=DEV, generator=g)[:B * nbp].view(B, nbp).to(torch.int32)
    q = torch.randn(B, H, D, device=DEV, generator=g, dtype=torch.bfloat16)
    if var_len:
        sl = torch.randint(L // 2, L + 1, (B,), device=DEV, generator=g).to(torch.int32)
    else:
        sl = torch.full((B,), L, device=DEV, dtype=torch.int32)
    return q, kv, bt, sl


@pytest.mark.parametrize("B,L", CONFIG4)
def test_config4_batch_invariance_and_tolerance(B, L):
    D, scale = 128, 128 ** -0.5
    q, kv, bt, sl = _gpu_paged(B, L, seed=B, var_len=True)
    full = _run(q, kv, bt, sl, scale, B, D, out_dtype=torch.bfloat16)
    # each sampled request alone (batch of one) gives its in-batch bits
    for b in (0, B // 2, B - 1):
        alone = _run(q[b:b + 1], kv, bt[b:b + 1], sl[b:b + 1], scale, 1, D, out_dtype=torch.bfloat16)
        assert torch.equal(alone[0], full[b]), b
    # a mixed batch: the requests in another order, with other requests around them
    g = torch.Generator().manual_seed(7)
    perm = torch.randperm(B, generator=g).to(DEV)
    mixed = _run(q[perm], kv, bt[perm], sl[perm], scale, B, D, out_dtype=torch.bfloat16)
    assert torch.equal(mixed, full[perm])
    # only the first n requests
    n = max(1, B // 3)
    part = _run(q, kv, bt, sl, scale, n, D, out_dtype=torch.bfloat16)
    assert torch.equal(part[:n], full[:n])
    # tolerance against the float64 oracle on sampled requests
    rows = [0, B - 1]
    want = _oracle(q, kv, bt, sl, scale, B, D, rows=rows)
    f32 = _run(q, kv, bt, sl, scale, B, D)
    _check_tol(f32[rows].cpu().numpy(), want)
    _check_tol_bf16(full[rows].float().cpu().numpy(), want)


def test_short_and_single_key_sequences():
    H, KV, D, BS = 32, 8, 128, 16
    q, kv, bt, sl = make_paged(6, 64, BS, H, KV, D, seed=5)
    sl = torch.tensor([1, 2, 15, 16, 17, 64], dtype=torch.int32)
    q, kv, bt, sl = q.to(DEV), kv.to(DEV), bt.to(DEV), sl.to(DEV)
    o = _run(q, kv, bt, sl, 0.1, 6, D)
    want = _oracle(q, kv, bt, sl, 0.1, 6, D)
    _check_tol(o.cpu().numpy(), want)
    # a single key returns that key's value row exactly (softmax weight 1)
    kc, vc = kv_views(kv, D)
    v0 = vc[bt[0, 0].long(), 0].float()  # (KV, D)
    assert torch.equal(o[0], v0[torch.arange(H, device=DEV) // (H // KV)])


@pytest.mark.parametrize("blk,waves,split", [(16, 4, 1024), (32, 8, 2048), (64, 8, 512)])
def test_other_constant_sets_are_invariant_too(blk, waves, split):
    """Other (split, blk, waves) constants change the float order but keep each request's bits
    independent of the batch."""
    D = 128
    q, kv, bt, sl = _gpu_paged(12, 3000, seed=11, var_len=True)
    full = _run(q, kv, bt, sl, 0.09, 12, D, blk=blk, warps=waves, split=split)
    for b in (0, 5, 11):
        alone = _run(q[b:b + 1], kv, bt[b:b + 1], sl[b:b + 1], 0.09, 1, D, blk=blk, warps=waves, split=split)
        assert torch.equal(alone[0], full[b])
    want = _oracle(q, kv, bt, sl, 0.09, 12, D, rows=[0, 11])
    _check_tol(full[[0, 11]].cpu().numpy(), want)


def test_merge_of_more_segments_than_one_pass_loads():
    """The merge loads eight segments a pass: requests of 1, 2, 8, 9, 16, 17 and 18 segments of
    512 keys (pass boundaries on both sides) against the float64 oracle, each request's bits the
    same alone as in the batch, and the same with the batch's length passed as the bound (a grid
    of 18 segments instead of 32) as with none."""
    D, split = 128, 512
    q, kv, bt, sl = _gpu_paged(7, 9216, seed=23, var_len=False)
    sl = torch.tensor([512, 513, 4096, 4097, 8192, 8193, 9216], device=DEV, dtype=torch.int32)
    kc, vc = kv_views(kv, D)
    full = torch.full((7, 32, D), float("nan"), device=DEV)
    P.paged_decode(q, kc, vc, bt, sl, 0.09, full, 7, 0, split=split)
    bounded = _run(q, kv, bt, sl, 0.09, 7, D, split=split)
    assert torch.equal(bounded, full)
    for b in range(7):
        alone = _run(q[b:b + 1], kv, bt[b:b + 1], sl[b:b + 1], 0.09, 1, D, split=split)
        assert torch.equal(alone[0], full[b]), b
    _check_tol(full.cpu().numpy(), _oracle(q, kv, bt, sl, 0.09, 7, D))


@pytest.mark.parametrize("D,H,KV", [(64, 8, 8), (128, 16, 8), (256, 32, 4)])
def test_head_dims_and_groups(D, H, KV):
    q, kv, bt, sl = make_paged(5, 700, 32, H, KV, D, seed=D + H)
    q, kv, bt, sl = q.to(DEV), kv.to(DEV), bt.to(DEV), sl.to(DEV)
    o = _run(q, kv, bt, sl, D ** -0.5, 5, D)
    want = _oracle(q, kv, bt, sl, D ** -0.5, 5, D)
    _check_tol(o.cpu().numpy(), want)


def test_random_shapes_against_the_oracle():
    """A seeded sweep of 30 random cases over what the kernel accepts: head dims 64 / 128 / 256,
    groups 1 / 2 / 4 / 8 (H <= 32), page sizes 8 / 16 / 32 / 528, 1-6 requests of 1-3000 keys,
    (blk, waves, split) from {16, 32, 64} x {4, 8} x {512, 1024, 2048}, fp32 and bf16 output.
    Every request is within the stated tolerance of the float64 oracle, and one random request
    run alone gives the bits it gets in the batch."""
    import random

    rng = random.Random(4321)
    for case in range(30):
        D = rng.choice([64, 128, 256])
        KV = rng.choice([1, 2, 4, 8])
        G = rng.choice([g for g in (1, 2, 4, 8) if g * KV <= 32])
        BS = rng.choice([8, 16, 32, 528])
        B, L = rng.randint(1, 6), rng.randint(1, 3000)
        blk, waves, split = rng.choice([16, 32, 64]), rng.choice([4, 8]), rng.choice([512, 1024, 2048])
        out_dtype = rng.choice([torch.float32, torch.bfloat16])
        scale = D ** -0.5 * rng.uniform(0.5, 1.5)
        what = (case, D, G * KV, KV, BS, B, L, blk, waves, split, out_dtype)
        print(what, flush=True)
        q, kv, bt, sl = make_paged(B, L, BS, G * KV, KV, D, seed=case, var_len=L > 1)
        q, kv, bt, sl = q.to(DEV), kv.to(DEV), bt.to(DEV), sl.to(DEV)
        kw = dict(blk=blk, warps=waves, split=split)
        o = _run(q, kv, bt, sl, scale, B, D, out_dtype, **kw)
        want = _oracle(q, kv, bt, sl, scale, B, D)
        got = o.float().cpu().numpy()
        if out_dtype == torch.float32:
            _check_tol(got, want)
        else:
            _check_tol_bf16(got, want)
        b = rng.randrange(B)
        alone = _run(q[b:b + 1], kv, bt[b:b + 1], sl[b:b + 1], scale, 1, D, out_dtype, **kw)
        assert torch.equal(alone[0], o[b]), what
