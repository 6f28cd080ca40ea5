"""GPU parity of the packed (fragment-major) path.

The packed layout has no counterpart in the reference; tests/helpers.pack_np states it
independently in numpy. Checks: GPU packing matches it byte for byte; digitize_packed equals
pack(digitize) and the oracle's digits; the packed GEMM equals the oracle bitwise for every
kernel family (small-M, LDS ring, x through LDS with weights in registers, K split over the
waves of a workgroup), ragged M/N/K, every split-K factor, F=14 (3 and 4 dots) and F=15; the
one-launch digitize + GEMM path equals the oracle at 1-64 rows; the exactmm::linear op on
load-time packed weights, with and without the shipped table (which picks the one-launch
path at 16 rows for some shapes and not for others), equals the oracle.
"""
import itertools

import numpy as np
import pytest
import torch

import oracle
import vllm_exact
from helpers import f32_bits, np_digits, pack_np, stress_xw, xw
from vllm_exact import kernels as K
from vllm_exact import plugin

pytestmark = pytest.mark.gpu
DEV = "cuda"

PACKED_CFGS = ((16, 16, 128, 16, 4, 8), (16, 32, 128, 8, 2, 8), (16, 64, 128, 4, 1, 8), (32, 64, 128, 8, 1, 8),
               (64, 32, 128, 4, 2, 8), (64, 64, 128, 4, 1, 8), (64, 64, 128, 4, 8, 8), (128, 64, 128, 4, 6, 8),
               (64, 128, 128, 4, 4, 8), (128, 128, 128, 4, 4, 8), (128, 128, 128, 4, 2, 8)) + tuple(
    (bm, bn, 64, nw, r, 8) for bm, bn, r, nw in K.XW_SHAPES)  # BK = 64: x through LDS, weights in registers


@pytest.mark.parametrize("R,Kd", [(16, 4096), (37, 1000), (5, 64), (300, 12288), (3, 40000)])
def test_pack_matches_layout_and_digitize_packed(R, Kd):
    x, _ = xw(R, 1, Kd, seed=R)
    for F in (14, 15):
        d = K.digitize(x.to(DEV), F)
        packed, cs, sh = K.pack_digits(d)
        dn = np_digits(d)
        want = pack_np(dn[0], dn[1])
        assert np.array_equal(packed.cpu().numpy(), want)
        pd, pcs, psh = K.digitize_packed(x.to(DEV).to(torch.bfloat16).float(), F)
        xbd = oracle.digitize_c(x.to(torch.bfloat16).float().numpy(), F)
        assert np.array_equal(pd.cpu().numpy(), pack_np(xbd[0], xbd[1]))
        assert np.array_equal(pcs.cpu().numpy(), xbd[2]) and np.array_equal(psh.cpu().numpy(), xbd[3])
        # bf16 input directly gives the same packed digits
        pd2, _, _ = K.digitize_packed(x.to(DEV).to(torch.bfloat16), F)
        assert torch.equal(pd2, pd)


@pytest.mark.parametrize("F,tr", [(14, True), (14, False), (15, False)])
@pytest.mark.parametrize("M,N,Kd", [(1, 64, 4096), (16, 4096, 4096), (24, 384, 4096), (5, 200, 12288),
                                    (256, 1024, 4096), (300, 256, 12288), (33, 130, 1000)])
def test_packed_gemm_bitwise(F, tr, M, N, Kd):
    x, w = stress_xw(M, N, Kd, seed=M + N)
    xd, wd = K.digitize(x.to(DEV), F), K.digitize(w.to(DEV), F)
    ref = f32_bits(oracle.exact_linear_c(np_digits(xd), np_digits(wd), F, tr))
    xp, wp = K.pack_digits(xd), K.pack_digits(wd)
    for base, sk in itertools.product(PACKED_CFGS, (1, 2, 4, 8)):
        cfg = base + (sk,)
        y = K.exact_linear_packed(xp, wp, Kd, F, tr, cfg=cfg)
        assert np.array_equal(f32_bits(y.cpu().numpy()), ref), cfg
    yb = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
    K.exact_linear_packed(xp, wp, Kd, F, tr, out=yb, cfg=(16, 64, 128, 4, 1, 8, 2))
    want_b = oracle.bf16_rne_c(oracle.exact_linear_c(np_digits(xd), np_digits(wd), F, tr)).reshape(M, N)
    assert np.array_equal(yb.cpu().view(torch.int16).numpy().view(np.uint16), want_b)


@pytest.mark.parametrize("tr", [True, False])
def test_xw_two_byte_outputs_every_tile(tr):
    """The x-through-LDS kernels write a 2-byte output without a K split through an LDS-staged
    tile and 16-byte row pieces. Every tile shape, at ragged M, N and K: bf16 into a view
    whose row stride is a multiple of 8 (whole pieces, then an element-wise tail: 203 columns)
    and fp16 into a contiguous 203-column tensor (row starts not 16-byte aligned: every piece
    element-wise), both equal to the oracle's fp32 rounded once to nearest even."""
    M, N, Kd, F = 70, 203, 1000, 14
    x, w = stress_xw(M, N, Kd, seed=7)
    xd, wd = K.digitize(x.to(DEV), F), K.digitize(w.to(DEV), F)
    ref = oracle.exact_linear_c(np_digits(xd), np_digits(wd), F, tr)
    want_b = oracle.bf16_rne_c(ref).reshape(M, N)
    want_h = ref.astype(np.float16).view(np.uint16)
    xp, wp = K.pack_digits(xd), K.pack_digits(wd)
    for bm, bn, r, nw in K.XW_SHAPES:
        cfg = (bm, bn, 64, nw, r, 8, 1)
        full = torch.full((M, N + 5), -1.0, device=DEV, dtype=torch.bfloat16)  # row stride 208
        K.exact_linear_packed(xp, wp, Kd, F, tr, out=full[:, :N], cfg=cfg)
        got = full.cpu()
        assert np.array_equal(got[:, :N].view(torch.int16).numpy().view(np.uint16), want_b), ("bf16", cfg)
        assert torch.equal(got[:, N:], torch.full((M, 5), -1.0, dtype=torch.bfloat16)), ("bf16 padding", cfg)
        fullh = torch.full((M, N + 3), -1.0, device=DEV, dtype=torch.float16)  # odd row stride: every piece element-wise
        K.exact_linear_packed(xp, wp, Kd, F, tr, out=fullh[:, :N], cfg=cfg)
        goth = fullh.cpu()
        assert np.array_equal(goth[:, :N].numpy().view(np.uint16), want_h), ("fp16", cfg)
        assert torch.equal(goth[:, N:], torch.full((M, 3), -1.0, dtype=torch.float16)), ("fp16 padding", cfg)


XK_CFGS = tuple((bm, bn, 64 * kg, 8, 2, 8) for bm, bn, kg in K.XK_SHAPES)


@pytest.mark.parametrize("F,tr", [(14, True), (14, False), (15, False)])
@pytest.mark.parametrize("M,N,Kd", [(256, 384, 4096), (70, 203, 1000), (130, 1000, 512), (200, 96, 640)])
def test_xk_kernel_bitwise(F, tr, M, N, Kd):
    """The K-split kernel (K groups of waves reducing in LDS) for every instantiated tile, at 3
    and 4 dots (shapes without a 4-dot instantiation, K splits that are not whole rounds and
    K = 640, which has none, take the LDS-ring kernel) and split-K 1, 2, 4: fp32 output (lane
    stores; int64 partials when split), bf16 into a strided view (staged tile; the padding
    columns stay untouched), fp16 (staged, rows not 16-byte aligned) and F = 15 (offset terms),
    every one equal to the oracle rounded once."""
    x, w = stress_xw(M, N, Kd, seed=M + 3 * N)
    xd, wd = K.digitize(x.to(DEV), F), K.digitize(w.to(DEV), F)
    ref = oracle.exact_linear_c(np_digits(xd), np_digits(wd), F, tr)
    ref_bits = f32_bits(ref)
    want_b = oracle.bf16_rne_c(ref).reshape(M, N)
    want_h = ref.astype(np.float16).view(np.uint16)
    xp, wp = K.pack_digits(xd), K.pack_digits(wd)
    for base, sk in itertools.product(XK_CFGS, (1, 2, 4)):
        cfg = base + (sk,)
        y = K.exact_linear_packed(xp, wp, Kd, F, tr, cfg=cfg)
        assert np.array_equal(f32_bits(y.cpu().numpy()), ref_bits), ("fp32", cfg)
        if sk == 1:
            full = torch.full((M, N + 5), -1.0, device=DEV, dtype=torch.bfloat16)
            K.exact_linear_packed(xp, wp, Kd, F, tr, out=full[:, :N], cfg=cfg)
            got = full.cpu()
            assert np.array_equal(got[:, :N].view(torch.int16).numpy().view(np.uint16), want_b), ("bf16", cfg)
            assert torch.equal(got[:, N:], torch.full((M, 5), -1.0, dtype=torch.bfloat16)), ("bf16 padding", cfg)
            yh = torch.empty(M, N, device=DEV, dtype=torch.float16)
            K.exact_linear_packed(xp, wp, Kd, F, tr, out=yh, cfg=cfg)
            assert np.array_equal(yh.cpu().numpy().view(np.uint16), want_h), ("fp16", cfg)


FUSED_CFGS = tuple((16, 16 * nt, 128, nwk, c, 8, 1) for mt, nt, c, nwk in K.SMALL_SHAPES if mt == 1)


@pytest.mark.parametrize("F,tr", [(14, True), (14, False), (12, True), (15, False)])
@pytest.mark.parametrize("M,N,Kd", [(1, 64, 4096), (2, 200, 1000), (3, 96, 4104), (4, 48, 64), (4, 16, 12288), (2, 5000, 4096),
                                    (1, 130, 40), (16, 64, 4096), (37, 80, 1000), (64, 48, 12288), (20, 32, 8)])
def test_fused_digitize_gemm_bitwise(F, tr, M, N, Kd):
    """exact_linear_bf16x (x digitized inside the GEMM launch, each workgroup its own 16 rows)
    gives the oracle's bits for every one-row-tile config, with ragged M, N and K (K not a
    multiple of 64, 16 or 8), rows of magnitudes 1e-3 to 1e3 and a zero row; the
    exactmm::linear op takes this path and gives the same bits. F = 15 (offset digits, 4 dots,
    the row digit sums in the epilogue) runs in one launch on both kernels, x in registers and
    the row pass; it declines (NotImplementedError) only the 16-wave shapes with four column
    tiles times steps per round, whose digit sum would spill, and what it takes must match."""
    x, w = stress_xw(M, N, Kd, seed=M * 7 + Kd)
    x = (x * (10.0 ** torch.linspace(-3, 3, M))[:, None]).to(torch.bfloat16)
    if M >= 3:
        x[1] = 0  # sh = F, zero digits
    wb = w.to(torch.bfloat16)
    xd_np = oracle.digitize_c(x.float().numpy(), F)
    wd_np = oracle.digitize_c(wb.float().numpy(), F)
    ref32 = oracle.exact_linear_c(xd_np, wd_np, F, tr)
    wp = K.digitize_packed(wb.to(DEV), F)
    xg = x.to(DEV)
    taken = []
    for cfg in FUSED_CFGS:
        try:
            y = K.exact_linear_bf16x(xg, wp, Kd, F, tr, cfg=cfg)
        except NotImplementedError:
            assert F == 15 and cfg[3] == 16 and cfg[1] // 16 * cfg[4] >= 4, cfg
            continue
        taken.append(cfg)
        assert np.array_equal(f32_bits(y.cpu().numpy()), f32_bits(ref32)), cfg
    assert taken
    want_b = oracle.bf16_rne_c(ref32).reshape(M, N)
    if taken:
        yb = torch.empty(M, N + 8, device=DEV, dtype=torch.bfloat16)[:, :N]  # row stride N + 8
        K.exact_linear_bf16x(xg, wp, Kd, F, tr, out=yb, cfg=taken[0])
        assert np.array_equal(yb.cpu().contiguous().view(torch.int16).numpy().view(np.uint16), want_b)
    if (F, tr) in ((plugin.F, plugin.TRUNC), (15, False)):
        saved = plugin.F, plugin.TRUNC
        plugin.F, plugin.TRUNC = F, tr
        try:
            y_op = torch.ops.exactmm.linear(xg, *plugin.pack_weight(wb.to(DEV)))
        finally:
            plugin.F, plugin.TRUNC = saved
        assert np.array_equal(y_op.cpu().view(torch.int16).numpy().view(np.uint16), want_b)


def test_random_shapes_one_and_two_launch_bitwise():
    """A seeded sweep of 160 random cases (M 1-64, N 1-900, K 8-12288 including K not a
    multiple of 16 or 64, F = 12 / 14 / 15 with and without truncation, rows scaled by 1e-3 to
    1e3): a random one-row-tile cfg on the one-launch path and a random packed cfg and split-K
    factor on the two-launch path, both equal to the oracle bit for bit. The one-launch path
    declines only the F = 15 16-wave cfgs with four column tiles times steps per round."""
    import random

    rng = random.Random(1234)
    n_taken = 0
    for case in range(160):
        M = rng.choice([1, 2, 3, 4, 5, 8, 13, 16, 17, 31, 40, 64])
        N = rng.randint(1, 900)
        Kd = rng.choice([8, 16, 40, 64, 72, 128, 520, 1000, 2048, 4096, 4104, 8192, 12288])
        F, tr = rng.choice([(14, True), (14, False), (12, True), (15, False)])
        cfg = rng.choice(FUSED_CFGS)
        cfg2 = rng.choice(PACKED_CFGS) + (rng.choice([1, 2, 4, 8]),)
        x, w = stress_xw(M, N, Kd, seed=case)
        scale = 10.0 ** torch.empty(M).uniform_(-3, 3, generator=torch.Generator().manual_seed(case))
        x = (x * scale[:, None]).to(torch.bfloat16)
        wb = w.to(torch.bfloat16)
        ref = f32_bits(oracle.exact_linear_c(oracle.digitize_c(x.float().numpy(), F),
                                             oracle.digitize_c(wb.float().numpy(), F), F, tr))
        wp = K.digitize_packed(wb.to(DEV), F)
        xg = x.to(DEV)
        what = (case, M, N, Kd, F, tr)
        try:
            y = K.exact_linear_bf16x(xg, wp, Kd, F, tr, cfg=cfg)
        except NotImplementedError:
            assert F == 15 and cfg[3] == 16 and cfg[1] // 16 * cfg[4] >= 4, what + (cfg,)
        else:
            assert np.array_equal(f32_bits(y.cpu().numpy()), ref), what + (cfg,)
            n_taken += 1
        y2 = K.exact_linear_packed(K.digitize_packed(xg, F), wp, Kd, F, tr, cfg=cfg2)
        assert np.array_equal(f32_bits(y2.cpu().numpy()), ref), what + (cfg2,)
    assert n_taken >= 140


@pytest.mark.parametrize("F,tr", [(14, True), (15, False), (12, True)])
def test_rows_at_the_edge_of_the_scale_exponent(F, tr):
    """Rows so small that 2^sh, built from exponent bits, leaves the float range: shifts
    124 ... 133 around sh = 128 (the scale is +inf there, x * scale is +-inf, and
    NaN where x = 0; beyond it the exponent field wraps) and bf16 subnormal rows, with zeros
    and both signs in every row. float -> int32 saturates with NaN -> 0, as the device cast
    does (oracle trunc_i32). Digits and shifts from fp32 and bf16 input, packed digits, and
    both GEMM paths equal the oracle bit for bit."""
    g = torch.Generator().manual_seed(F)
    Kd, N = 200, 48
    exps = [F - 1 - sh for sh in range(124, 134)] + [-126, -130, -133]  # absmax 2^e: sh = F - e - 1
    x = torch.randn(len(exps) + 1, Kd, generator=g)
    x[:, ::7] = 0
    x = x / x.abs().amax(dim=1, keepdim=True)
    x[:len(exps)] *= torch.tensor([2.0 ** e for e in exps])[:, None]
    xb = x.to(torch.bfloat16)
    w = (torch.randn(N, Kd, generator=g) * 0.02).to(torch.bfloat16)
    for src in (x, xb.float()):
        want = oracle.digitize_c(src.numpy(), F)
        got = np_digits(K.digitize(src.to(DEV), F))
        for a, b, name in zip(got, want, ("h", "l", "cs", "sh")):
            assert np.array_equal(a, b), name
    xd_np = oracle.digitize_c(xb.float().numpy(), F)
    assert xd_np[3][:10].tolist() == list(range(124, 134))
    px, pcx, psx = K.digitize_packed(xb.to(DEV), F)
    assert np.array_equal(px.cpu().numpy(), pack_np(xd_np[0], xd_np[1]))
    assert np.array_equal(pcx.cpu().numpy(), xd_np[2]) and np.array_equal(psx.cpu().numpy(), xd_np[3])
    ref = f32_bits(oracle.exact_linear_c(xd_np, oracle.digitize_c(w.float().numpy(), F), F, tr))
    wp = K.digitize_packed(w.to(DEV), F)
    y = K.exact_linear_packed((px, pcx, psx), wp, Kd, F, tr, cfg=(16, 64, 128, 4, 1, 8, 1))
    assert np.array_equal(f32_bits(y.cpu().numpy()), ref)
    taken = 0
    for cfg in FUSED_CFGS:
        try:
            y = K.exact_linear_bf16x(xb.to(DEV), wp, Kd, F, tr, cfg=cfg)
        except NotImplementedError:
            assert F == 15 and cfg[3] == 16 and cfg[1] // 16 * cfg[4] >= 4, cfg
            continue
        taken += 1
        assert np.array_equal(f32_bits(y.cpu().numpy()), ref), cfg
    assert taken


def test_fused_path_declines_and_the_op_falls_back():
    """Where one launch does not apply (x rows not 16-byte aligned, at F = 14 and 15; a split-K
    or wide-tile cfg) exact_linear_bf16x raises NotImplementedError, and the op's two-launch
    path still gives the oracle's bits."""
    g = torch.Generator().manual_seed(5)
    N, Kd = 96, 1001  # K = 1001: bf16 rows of 2002 bytes, not 16-byte aligned
    w = (torch.randn(N, Kd, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(5, Kd, generator=g).to(torch.bfloat16)
    wp = K.digitize_packed(w.to(DEV), 14)
    xg = x.to(DEV)
    cfg = FUSED_CFGS[0]
    for args, kw in (((xg[:2], wp, Kd, 15, False), dict(cfg=cfg)), ((xg[:2], wp, Kd, 14, True), dict(cfg=cfg)),
                     ((xg[:2], wp, Kd, 14, True), dict(cfg=(16, 32, 128, 8, 1, 8, 2))),
                     ((xg[:2], wp, Kd, 14, True), dict(cfg=(64, 96, 64, 6, 6, 8, 1)))):
        with pytest.raises(NotImplementedError):
            K.exact_linear_bf16x(*args, **kw)
    wbuf = plugin.pack_weight(w.to(DEV))
    wd_np = oracle.digitize_c(w.float().numpy(), plugin.F)
    for M in (2, 5):
        y = torch.ops.exactmm.linear(xg[:M], *wbuf)
        ref = oracle.exact_linear_c(oracle.digitize_c(x[:M].float().numpy(), plugin.F), wd_np, plugin.F, plugin.TRUNC)
        assert np.array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16),
                              oracle.bf16_rne_c(ref).reshape(ref.shape)), M


@pytest.mark.parametrize("shape", [(6144, 4096), (4096, 4096), (24576, 4096), (4096, 12288)])
def test_op_with_packed_weights_matches_oracle(shape):
    N, Kd = shape
    g = torch.Generator().manual_seed(3)
    w = (torch.randn(N, Kd, generator=g) * 0.02).to(torch.bfloat16)
    wbuf = plugin.pack_weight(w.to(DEV))
    wd_np = oracle.digitize_c(w.float().numpy(), plugin.F)
    for table in (None, vllm_exact.TABLES["mi355x"]):
        plugin.load_table(table)
        try:
            for M in (1, 16, 64, 256):
                x = torch.randn(M, Kd, generator=g).to(torch.bfloat16)
                y = torch.ops.exactmm.linear(x.to(DEV), *wbuf)
                rows = np.arange(M) if M <= 64 else np.array([0, 100, 255])
                xd_np = oracle.digitize_c(x.float().numpy()[rows], plugin.F)
                ref = oracle.exact_linear_c(xd_np, wd_np, plugin.F, plugin.TRUNC)
                got = y.cpu().view(torch.int16).numpy().view(np.uint16)[rows]
                assert np.array_equal(got, oracle.bf16_rne_c(ref).reshape(ref.shape)), (M, table,
                                                                                         plugin._one_launch(M, N, Kd))
        finally:
            plugin.load_table(None)


def test_layer_digitize_and_weight_release():
    """process_weights_after_loading's packing of a layer (plugin.py:72-79): the op on the
    layer's buffers gives the oracle's bits, and releasing the bf16 weight afterwards
    (enable(release_weights=True)) frees its memory and changes no bit."""
    g = torch.Generator().manual_seed(13)
    w = (torch.randn(160, 512, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(3, 512, generator=g).to(torch.bfloat16)
    kept, freed = torch.nn.Linear(512, 160, bias=False), torch.nn.Linear(512, 160, bias=False)
    for layer in (kept, freed):
        layer.weight.data = w.to(DEV)
    plugin._digitize_layer(kept)
    plugin._digitize_layer(freed, release=True)
    assert kept.weight.numel() == 160 * 512
    assert freed.weight.numel() == 0 and freed.weight.dtype == torch.bfloat16 and freed.weight.is_cuda
    ys = [plugin._apply(layer, x.to(DEV), None) for layer in (kept, freed)]
    assert torch.equal(ys[0].view(torch.int16), ys[1].view(torch.int16))
    ref = oracle.exact_linear_c(oracle.digitize_c(x.float().numpy(), plugin.F),
                                oracle.digitize_c(w.float().numpy(), plugin.F), plugin.F, plugin.TRUNC)
    assert np.array_equal(ys[1].cpu().view(torch.int16).numpy().view(np.uint16), oracle.bf16_rne_c(ref).reshape(3, 160))


def test_op_row_blocks_and_input_layouts():
    """exactmm::linear cuts M into RB-row blocks (plugin.py:60-63), each with the config of its
    own size; rows are independent, so any blocking, a 3-D input and a transposed (strided)
    input give the same bits as one block, and those bits equal the oracle."""
    g = torch.Generator().manual_seed(11)
    w = (torch.randn(192, 1024, generator=g) * 0.02).to(torch.bfloat16)
    wbuf = plugin.pack_weight(w.to(DEV))
    x = torch.randn(257, 1024, generator=g).to(torch.bfloat16).to(DEV)
    full = torch.ops.exactmm.linear(x, *wbuf)
    rb = plugin.RB
    try:
        plugin.RB = 100  # blocks of 100, 100 and 57 rows
        blocked = torch.ops.exactmm.linear(x, *wbuf)
    finally:
        plugin.RB = rb
    assert torch.equal(blocked, full)
    assert torch.equal(torch.ops.exactmm.linear(x.view(1, 257, 1024), *wbuf).view(257, 192), full)
    xt = x.t().contiguous().t()  # same values, column-major storage
    assert xt.stride(-1) != 1 and torch.equal(torch.ops.exactmm.linear(xt, *wbuf), full)
    rows = np.array([0, 99, 100, 256])
    ref = oracle.exact_linear_c(oracle.digitize_c(x.float().cpu().numpy()[rows], plugin.F),
                                oracle.digitize_c(w.float().numpy(), plugin.F), plugin.F, plugin.TRUNC)
    got = full.cpu().view(torch.int16).numpy().view(np.uint16)[rows]
    assert np.array_equal(got, oracle.bf16_rne_c(ref).reshape(ref.shape))


@pytest.mark.parametrize("M", [3, 64, 257])
def test_op_fp16_activations(M):
    """fp16 activations, the reference's other supported dtype (plugin.py:113-114): the op
    digitizes the fp16 values and writes fp16 output (x.dtype), the fp32 result rounded once
    to nearest even. 3 rows would take the one-launch path for bf16; fp16 goes in two."""
    g = torch.Generator().manual_seed(12)
    w = (torch.randn(200, 1024, generator=g) * 0.02).to(torch.bfloat16)
    wbuf = plugin.pack_weight(w.to(DEV))
    x = (torch.randn(M, 1024, generator=g) * 4).to(torch.float16)
    y = torch.ops.exactmm.linear(x.to(DEV), *wbuf)
    assert y.dtype == torch.float16 and y.shape == (M, 200)
    ref = oracle.exact_linear_c(oracle.digitize_c(x.float().numpy(), plugin.F),
                                oracle.digitize_c(w.float().numpy(), plugin.F), plugin.F, plugin.TRUNC)
    assert np.array_equal(y.cpu().numpy().view(np.uint16), ref.astype(np.float16).view(np.uint16))


def _shipped_entries(path):
    """Distinct (M, K, cfg, one_launch) of a shipped table: cfgs only change speed, so each
    runs on a small ragged N instead of its shape's."""
    import json
    raw = json.loads(path.read_text())
    out = set()
    for nk, row in raw.items():
        kd = int(nk.split(",")[1])
        marks = set(row.get("one_launch", ()))
        for m, cfg in row.items():
            if m not in ("one_launch", "n_split"):
                out.add((int(m), kd, tuple(cfg), int(m) in marks))
        for m, split in row.get("n_split", {}).items():  # the second launch of a column split
            out.add((int(m), kd, tuple(split[1:]), False))
    return sorted(out)


@pytest.mark.parametrize("which,F,tr", [("F14", 14, True), ("F15", 15, False)])
def test_every_shipped_table_entry_is_exact(which, F, tr):
    """Every entry of a shipped gfx950 table (the one tuned at F = 14, and the one tuned at
    F = 15 with 4 dots), at its own row count and K, gives the oracle's bits; the entries
    marked one-launch also through the one-launch kernel."""
    N = 200  # ragged against every BN in the table
    entries = _shipped_entries((vllm_exact.TABLES if which == "F14" else vllm_exact.TABLES_F15)["mi355x"])
    data = {}
    for M, Kd, cfg, one in entries:
        if (M, Kd) not in data:
            x, w = stress_xw(M, N, Kd, seed=M + Kd)
            x = x.to(torch.bfloat16)
            xd_np = oracle.digitize_c(x.float().numpy(), F)
            wd = K.digitize_packed(w.to(torch.bfloat16).to(DEV), F)
            wd_np = oracle.digitize_c(w.to(torch.bfloat16).float().numpy(), F)
            want = oracle.bf16_rne_c(oracle.exact_linear_c(xd_np, wd_np, F, tr)).reshape(M, N)
            data[(M, Kd)] = (x.to(DEV), wd, want)
        xg, wd, want = data[(M, Kd)]
        out = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
        K.exact_linear_packed(K.digitize_packed(xg, F), wd, Kd, F, tr, out=out, cfg=cfg)
        assert np.array_equal(out.cpu().view(torch.int16).numpy().view(np.uint16), want), (M, Kd, cfg)
        if one:
            out.zero_()
            K.exact_linear_bf16x(xg, wd, Kd, F, tr, out=out, cfg=cfg)
            assert np.array_equal(out.cpu().view(torch.int16).numpy().view(np.uint16), want), (M, Kd, cfg, "one")
    assert len(entries) > 50


def test_packed_entry_points_reject_malformed_inputs():
    """Shapes, dtypes and devices the kernels would read out of bounds are refused on the host
    (ValueError) before any launch."""
    x, w = xw(8, 64, 256, seed=2)
    xp = K.digitize_packed(x.to(DEV), 14)
    wp = K.digitize_packed(w.to(DEV), 14)
    cfg = (16, 64, 128, 4, 1, 8, 1)
    ok = K.exact_linear_packed(xp, wp, 256, 14, True, cfg=cfg)
    assert ok.shape == (8, 64)
    bad = [
        ((xp[0], xp[1][:4], xp[2]), wp),                          # cx shorter than M
        (xp, (wp[0], wp[1], wp[2].to(torch.int64))),              # sw not int32
        ((xp[0].view(torch.uint8), xp[1], xp[2]), wp),            # packed digits not int8
        (xp, (wp[0][:2], wp[1], wp[2])),                          # packed rows do not match N
    ]
    for a, b in bad:
        with pytest.raises(ValueError):
            K.exact_linear_packed(a, b, 256, 14, True, cfg=cfg)
    with pytest.raises(ValueError):
        K.exact_linear_packed(xp, wp, 320, 14, True, cfg=cfg)   # K disagrees with the packed shape
    with pytest.raises(ValueError):
        K.digitize_packed(x.to(DEV), 14, out=(xp[0], xp[1][:3], xp[2]))
