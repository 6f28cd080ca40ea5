"""Exact INT8 two-digit linear layers on MI355X: digitization and exact matmul.

Numerical spec (the reference's kernels.py:3-9):
- activations and weights are converted per row to F-bit fixed point with one power-of-two
  scale per row and split into two INT8 digits, q = 256*h + l. F = 15 uses offset digits
  with a row-sum correction; F < 15 uses balanced digits. trunc=True drops the l*l term.
- digit products are exact on INT8 matrix cores and accumulate in int32 then int64, so the
  result does not depend on tiling, split-K partition, batch size or the other rows.
  int64 -> fp64 is exact, fp64 -> fp32 rounds once, fp32 -> bf16/fp16 rounds once more.

Entry points keep the reference's names and signatures (kernels.py:22-43, 74-100, 250-316):
digitize_torch, digitize_weight, digitize, exact_linear_torch, exact_linear,
autotune_exact, EXACT_CFGS. `digitize` and `exact_linear` run the gfx950 HIP kernels of
libvllm_exact_amd.so and accept only GPU tensors; the *_torch functions are the plain
torch statements of the same integer arithmetic (the reference's CPU path).
"""
import torch

from . import _native as _nx

HAVE_HIP = _nx.available() and torch.cuda.is_available()
HAVE_TRITON = False  # the reference's backend flag (kernels.py:13-18); this build has no Triton path


# ======================= fixed-point digitization =======================
def digitize_torch(x, F):
    """(R, K) float -> (h int8, l int8, cs int32, sh int32) in plain torch (kernels.py:22-39).

    e is the frexp exponent of the row absmax (0 for a zero row), sh = F - e, 2^sh is built
    from its fp32 bit pattern, and q = trunc(x * 2^sh) (the float -> int cast truncates).
    """
    x = x.float()
    amax = x.abs().amax(dim=1)
    e = torch.frexp(amax).exponent
    e = torch.where(amax > 0, e, torch.zeros_like(e)).to(torch.int32)
    sh = (F - e).to(torch.int32)
    two_sh = ((sh + 127) << 23).view(torch.float32)
    q = (x * two_sh.unsqueeze(1)).to(torch.int32)
    if F == 15:
        lo = (q & 255) - 128
        hi = (q - lo - 128) >> 8
        cs = (256 * hi + lo).sum(dim=1, dtype=torch.int32)
    else:
        lo = ((q + 128) & 255) - 128
        hi = (q - lo) >> 8
        cs = torch.zeros_like(sh)
    return hi.to(torch.int8), lo.to(torch.int8), cs.to(torch.int32), sh


def digitize_weight(w, F):
    return digitize_torch(w.float(), F)


def _require_gpu(t, what):
    if not t.is_cuda:
        raise ValueError(
            f"{what} runs the gfx950 HIP kernels and needs GPU tensors; "
            f"use {what}_torch for the CPU statement of the same arithmetic")
    _nx.lib()  # raises if the HIP library is missing


def digitize(x, F, out=None):
    """Digitize the rows of a GPU tensor x (R, K) (fp32, bf16 or fp16) with the HIP kernel.

    Returns (h, l, cs, sh) like digitize_torch; bf16 input gives the same digits as its fp32
    upcast (kernels.py:74-85)."""
    _require_gpu(x, "digitize")
    if x.dim() != 2:
        raise ValueError(f"digitize expects a 2-D tensor, got shape {tuple(x.shape)}")
    if x.stride(1) != 1:
        x = x.contiguous()
    R, K = x.shape
    dev = x.device
    if out is None:
        out = (torch.empty((R, K), dtype=torch.int8, device=dev), torch.empty((R, K), dtype=torch.int8, device=dev),
               torch.empty(R, dtype=torch.int32, device=dev), torch.empty(R, dtype=torch.int32, device=dev))
    h, l, cs, sh = out
    if h.shape != (R, K) or l.shape != (R, K) or h.dtype != torch.int8 or l.dtype != torch.int8:
        raise ValueError("digitize: h/l must be int8 tensors of shape (R, K)")
    if h.stride(1) != 1 or l.stride(1) != 1 or h.stride(0) != l.stride(0):
        raise ValueError("digitize: h/l must be row-major with equal row strides")
    if cs.numel() != R or sh.numel() != R or cs.dtype != torch.int32 or sh.dtype != torch.int32:
        raise ValueError("digitize: cs/sh must be int32 tensors of R elements")
    if not (cs.is_contiguous() and sh.is_contiguous()):
        raise ValueError("digitize: cs/sh must be contiguous")
    with torch.cuda.device(dev):
        st = _nx.stream_handle(dev)
        _nx.check(_nx.lib().vxa_digitize(x.data_ptr(), _nx.dtype_enum(x.dtype), R, K, x.stride(0), h.data_ptr(),
                                         l.data_ptr(), h.stride(0), cs.data_ptr(), sh.data_ptr(), F, st),
                  "digitize")
    return out


# ======================= exact linear layer =======================
def exact_linear_torch(xd, wd, F, trunc=False):
    """Integer closed form in torch int64 (kernels.py:89-100); returns fp32 (M, N)."""
    xh, xl, cx, sx = (t.long() for t in xd)
    wh, wl, cw, sw = (t.long() for t in wd)
    K = xh.shape[1]
    tot = (xh @ wh.T) * 65536 + (xh @ wl.T + xl @ wh.T) * 256
    if not trunc:
        tot = tot + xl @ wl.T
    if F == 15:
        tot = tot + 128 * (cx[:, None] + cw[None, :]) + 128 * 128 * K
    e = -(sx[:, None] + sw[None, :])
    two_e = ((e + 1023) << 52).view(torch.float64)
    return (tot.double() * two_e).float()


def _check_sums(name, cs, sh, rows):
    """The per-row digit sums and scale exponents the kernels read: int32, contiguous, `rows` each."""
    if cs.dtype != torch.int32 or sh.dtype != torch.int32 or cs.numel() != rows or sh.numel() != rows:
        raise ValueError(f"{name}: cs/sh must be int32 tensors of {rows} elements")
    if not (cs.is_contiguous() and sh.is_contiguous()):
        raise ValueError(f"{name}: cs/sh must be contiguous")


# ======================= packed (fragment-major) digits =======================
# A [R, K] digit matrix packs into int8 [cdiv(R,16), cdiv(K,64), 2, 1024]: block (rt, kt) holds
# the h then l fragment of rows 16rt..16rt+15 and columns 64kt..64kt+63 in the operand order of
# the int8 MFMA (lane l's 16 bytes: row l & 15, columns 16*(l >> 4)..+16), zero-padded. Every
# MFMA operand is then one contiguous 1 KiB load. The weights of the plugin are packed once at
# load time; activations are digitized straight into this form.
def packed_shape(R, K):
    return ((R + 15) // 16, (K + 63) // 64, 2, 1024)


def pack_digits(d):
    """Row-major digits (h, l, cs, sh) -> (packed, cs, sh) on the GPU."""
    h, l, cs, sh = d
    _require_gpu(h, "pack_digits")
    R, K = h.shape
    if h.stride(1) != 1 or l.stride(1) != 1 or h.stride(0) != l.stride(0) or l.shape != h.shape:
        raise ValueError("pack_digits: h/l must be row-major int8 planes of one shape")
    packed = torch.empty(packed_shape(R, K), dtype=torch.int8, device=h.device)
    with torch.cuda.device(h.device):
        _nx.check(_nx.lib().vxa_pack_digits(h.data_ptr(), l.data_ptr(), R, K, h.stride(0), packed.data_ptr(),
                                            _nx.stream_handle(h.device)), "pack_digits")
    return packed, cs, sh


def digitize_packed(x, F, out=None):
    """digitize() writing packed digits: returns (packed, cs, sh), the same digits as
    pack_digits(digitize(x, F))."""
    _require_gpu(x, "digitize_packed")
    if x.dim() != 2:
        raise ValueError(f"digitize_packed expects a 2-D tensor, got shape {tuple(x.shape)}")
    if x.stride(1) != 1:
        x = x.contiguous()
    R, K = x.shape
    dev = x.device
    if out is None:
        out = (torch.empty(packed_shape(R, K), dtype=torch.int8, device=dev),
               torch.empty(R, dtype=torch.int32, device=dev), torch.empty(R, dtype=torch.int32, device=dev))
    packed, cs, sh = out
    if packed.shape != packed_shape(R, K) or not packed.is_contiguous() or packed.dtype != torch.int8:
        raise ValueError("digitize_packed: packed must be a contiguous int8 tensor of packed_shape(R, K)")
    _check_sums("digitize_packed", cs, sh, R)
    if any(t.device != dev for t in out):
        raise ValueError("digitize_packed: outputs must be on the input's device")
    with torch.cuda.device(dev):
        _nx.check(_nx.lib().vxa_digitize_packed(x.data_ptr(), _nx.dtype_enum(x.dtype), R, K, x.stride(0),
                                                packed.data_ptr(), cs.data_ptr(), sh.data_ptr(), F,
                                                _nx.stream_handle(dev)), "digitize_packed")
    return out


def exact_linear_packed(xp, wp, K, F, trunc=False, out=None, cfg=None):
    """exact_linear on packed digits xp = (packed_x, cx, sx), wp = (packed_w, cw, sw) with
    inner dimension K: the same bits as exact_linear on the row-major digits."""
    px, cx, sx = xp
    pw, cw, sw = wp
    _require_gpu(px, "exact_linear_packed")
    M, N = sx.numel(), sw.numel()
    if px.dtype != torch.int8 or pw.dtype != torch.int8:
        raise ValueError("exact_linear_packed: packed digits must be int8")
    if px.shape != packed_shape(M, K) or pw.shape != packed_shape(N, K):
        raise ValueError("exact_linear_packed: packed shapes do not match (M, K) and (N, K)")
    if not (px.is_contiguous() and pw.is_contiguous()):
        raise ValueError("exact_linear_packed: packed digits must be contiguous")
    _check_sums("exact_linear_packed (x)", cx, sx, M)
    _check_sums("exact_linear_packed (w)", cw, sw, N)
    dev = px.device
    if any(t.device != dev for t in (*xp, *wp)):
        raise ValueError("exact_linear_packed: all digit tensors must be on one device")
    if out is None:
        out = torch.empty((M, N), device=dev, dtype=torch.float32)
    if out.shape != (M, N) or out.stride(1) != 1 or out.device != dev:
        raise ValueError("exact_linear_packed: out must be an (M, N) row-major tensor")
    if cfg is None:
        raise ValueError("exact_linear_packed: pass a cfg (plugin._cfg or a tuning-table entry)")
    kpad = ((K + 63) // 64) * 64
    _, _, ws_bytes = _nx.exact_plan(M, N, kpad, cfg)
    ws = torch.empty(ws_bytes // 8, dtype=torch.int64, device=dev) if ws_bytes else None
    arr, n = _nx.cfg_array(cfg)
    with torch.cuda.device(dev):
        _nx.check(_nx.lib().vxa_exact_linear_packed(
            px.data_ptr(), cx.data_ptr(), sx.data_ptr(), pw.data_ptr(), cw.data_ptr(), sw.data_ptr(),
            out.data_ptr(), _nx.dtype_enum(out.dtype), out.stride(0), M, N, K, int(F), int(bool(trunc)), arr, n,
            _nx.ptr(ws), ws_bytes, _nx.stream_handle(dev)), "exact_linear_packed")
    return out


# Without a tuning-table entry that says otherwise, the exactmm::linear op digitizes inside the
# GEMM launch (exact_linear_bf16x) up to this many rows. Measured on MI355X the one launch
# saves 2-6 µs per op at 1-4 rows at every decode shape. Above that it depends on the shape:
# every workgroup reads its x rows twice (row pass, then K loop), so at 16 rows it still wins
# where K = 4096 and loses where K = 12288, and at 64 rows it loses. The tuner times both.
ONE_LAUNCH_MAX_ROWS = 4


def bf16x_rows_aligned(x):
    """True when x's rows can be read 16 bytes at a time (what exact_linear_bf16x needs)."""
    return x.data_ptr() % 16 == 0 and x.stride(0) % 8 == 0


def exact_linear_bf16x(x, wp, K, F, trunc=False, out=None, cfg=None):
    """Digitize x (bf16 [M, K]) and run exact_linear_packed in one launch: the bits of
    exact_linear_packed(digitize_packed(x, F), wp, K, F, trunc, cfg=cfg). Raises
    NotImplementedError where the one-launch path does not apply (a cfg outside the
    one-row-tile small-M family or with split-K, x rows not 16-byte aligned, or F = 15 with
    3 dots or on a 16-wave cfg with four column tiles times steps per round, whose digit sum
    would spill); the two-launch path covers those."""
    pw, cw, sw = wp
    _require_gpu(x, "exact_linear_bf16x")
    if x.dim() != 2 or x.dtype != torch.bfloat16 or x.stride(1) != 1:
        raise ValueError("exact_linear_bf16x: x must be a 2-D bf16 tensor with contiguous rows")
    M, N = x.shape[0], sw.numel()
    if x.shape[1] != K:
        raise ValueError(f"exact_linear_bf16x: x has {x.shape[1]} columns, K is {K}")
    if pw.dtype != torch.int8 or pw.shape != packed_shape(N, K) or not pw.is_contiguous():
        raise ValueError("exact_linear_bf16x: weights must be contiguous int8 of packed_shape(N, K)")
    _check_sums("exact_linear_bf16x (w)", cw, sw, N)
    dev = x.device
    if any(t.device != dev for t in wp):
        raise ValueError("exact_linear_bf16x: x and the weights must be on one device")
    if out is None:
        out = torch.empty((M, N), device=dev, dtype=torch.float32)
    if out.shape != (M, N) or out.stride(1) != 1 or out.device != dev:
        raise ValueError("exact_linear_bf16x: out must be an (M, N) row-major tensor")
    if cfg is None:
        raise ValueError("exact_linear_bf16x: pass a cfg (plugin._cfg or a tuning-table entry)")
    arr, n = _nx.cfg_array(cfg)
    with torch.cuda.device(dev):
        _nx.check(_nx.lib().vxa_exact_linear_bf16x(
            x.data_ptr(), x.stride(0), pw.data_ptr(), cw.data_ptr(), sw.data_ptr(), out.data_ptr(),
            _nx.dtype_enum(out.dtype),
            out.stride(0), M, N, K, int(F), int(bool(trunc)), arr, n, _nx.stream_handle(dev)), "exact_linear_bf16x")
    return out


# gfx950 kernel shapes, as cfg tuples (BM, BN, BK, warps, stages, GM). Three families:
# * small-M register-streaming kernel: BM = 16*MT rows, BN = 16*NT columns per workgroup,
#   `warps` waves splitting K, `stages` = K steps whose loads are issued together;
# * LDS-ring kernel (BM, BN >= 64, 4 waves, stages >= 2): BM x BN tile, `stages`-deep ring
#   of direct-to-LDS loads;
# * x-through-LDS kernel (BK = 64, packed digits): BM x BN tile, `warps` = 4 or 8 waves,
#   `stages` = weight register sets in flight per wave;
# * K-split kernel (BM >= 64, BK = 64 * KG with KG = 2 or 4 K groups, 8 waves, stages = 2,
#   packed digits): BM x BN tile, the waves of a K group covering all BM rows of BN / (8 / KG)
#   columns each over every KG-th pair of K steps.
# BK otherwise only rounds split-K chunks; GM is accepted for the reference's format.
SMALL_SHAPES = [(1, 1, 1, 4), (1, 1, 1, 8), (1, 1, 1, 16), (1, 1, 2, 4), (1, 1, 2, 8), (1, 1, 2, 16), (1, 1, 4, 4),
                (1, 1, 4, 8), (1, 1, 4, 16), (1, 2, 1, 4), (1, 2, 1, 8), (1, 2, 1, 16), (1, 2, 2, 4), (1, 2, 2, 8),
                (1, 2, 2, 16), (1, 2, 4, 4), (1, 2, 4, 8), (1, 4, 1, 4), (1, 4, 1, 8), (1, 4, 1, 16), (1, 4, 2, 4),
                (1, 4, 2, 8), (2, 1, 1, 4), (2, 1, 1, 8), (2, 1, 1, 16), (2, 1, 2, 4), (2, 1, 2, 8), (2, 2, 1, 4),
                (2, 2, 1, 8), (2, 2, 1, 16), (2, 2, 2, 4), (2, 2, 2, 8), (2, 4, 1, 4), (2, 4, 1, 8), (4, 1, 1, 4),
                (4, 1, 1, 8), (4, 1, 2, 4), (4, 1, 2, 8), (4, 2, 1, 4), (4, 2, 1, 8), (4, 4, 1, 4)]  # (MT, NT, C, NWK)
LDS_SHAPES = [(64, 64, 2), (64, 64, 4), (64, 64, 8), (128, 64, 2), (128, 64, 4), (128, 64, 6), (64, 128, 2),
              (64, 128, 4), (64, 128, 6), (128, 128, 2), (128, 128, 3), (128, 128, 4)]  # (BM, BN, stages)
XW_SHAPES = [(32, 128, 4, 4), (32, 256, 4, 4), (64, 64, 4, 4), (64, 128, 4, 4), (64, 192, 4, 4), (64, 256, 3, 4),
             (64, 256, 4, 4), (128, 64, 4, 4), (128, 128, 3, 4), (128, 128, 4, 4), (128, 192, 3, 4),
             (128, 192, 4, 4), (64, 128, 4, 8), (64, 192, 4, 8), (64, 256, 4, 8), (128, 128, 4, 8),
             (128, 192, 3, 8), (128, 192, 4, 8), (128, 256, 2, 8), (64, 96, 4, 6), (64, 96, 6, 6), (64, 96, 8, 6),
             (64, 96, 4, 3), (64, 96, 6, 3)]  # (BM, BN, weight sets, waves); BK = 64
XK_SHAPES = [(128, 192, 2), (128, 128, 2), (64, 96, 4), (64, 64, 4), (64, 128, 2), (64, 192, 2)]  # (BM, BN, KG)
XK_FOUR_DOTS = [(128, 128, 2), (64, 96, 4), (64, 64, 4), (64, 128, 2), (64, 192, 2)]  # the shapes with 4-dot instantiations
EXACT_CFGS = ([(16 * mt, 16 * nt, 128, nwk, c, 8) for mt, nt, c, nwk in SMALL_SHAPES]
              + [(bm, bn, 128, 4, st, 8) for bm, bn, st in LDS_SHAPES]
              + [(bm, bn, 64, nw, r, 8) for bm, bn, r, nw in XW_SHAPES]
              + [(bm, bn, 64 * kg, 8, 2, 8) for bm, bn, kg in XK_SHAPES])
AUTOTUNE_SPLITS = (1, 2, 4)
_CFG_CACHE = {}


def _check_digits(name, d, rows, K):
    h, l, c, s = d
    if h.dtype != torch.int8 or l.dtype != torch.int8 or c.dtype != torch.int32 or s.dtype != torch.int32:
        raise ValueError(f"exact_linear: {name} digits must be (int8, int8, int32, int32)")
    if h.shape != (rows, K) or l.shape != (rows, K) or c.numel() != rows or s.numel() != rows:
        raise ValueError(f"exact_linear: {name} digit shapes disagree")
    if h.stride(1) != 1 or l.stride(1) != 1 or h.stride(0) != l.stride(0):
        raise ValueError(f"exact_linear: {name} digit planes must be row-major with equal row strides")
    if not (c.is_contiguous() and s.is_contiguous()):
        raise ValueError(f"exact_linear: {name} cs/sh must be contiguous")


def exact_linear(xd, wd, F, trunc=False, out=None, cfg=None):
    """Exact two-digit matmul of digitized x (M, K) and w (N, K) on the HIP kernels.

    out: optional (M, N) fp32/bf16/fp16 GPU tensor (default fp32). cfg: the reference's tuple
    (BM, BN, BK, warps, stages, GM[, SK[, mma]]); it changes speed only, never bits
    (kernels.py:257-289). Without cfg the cached or autotuned config is used."""
    xh, xl, cx, sx = xd
    wh, wl, cw, sw = wd
    _require_gpu(xh, "exact_linear")
    M, K = xh.shape
    N = wh.shape[0]
    if wh.shape[1] != K:
        raise ValueError(f"exact_linear: K mismatch, x has {K}, w has {wh.shape[1]}")
    _check_digits("x", xd, M, K)
    _check_digits("w", wd, N, K)
    dev = xh.device
    for t in (*xd, *wd):
        if t.device != dev:
            raise ValueError("exact_linear: all digit tensors must be on one device")
    if out is None:
        out = torch.empty((M, N), device=dev, dtype=torch.float32)
    if out.shape != (M, N) or out.stride(1) != 1 or out.device != dev:
        raise ValueError("exact_linear: out must be an (M, N) row-major tensor on the digits' device")
    key = (M, N, K, F, bool(trunc))
    cfg = tuple(cfg or _CFG_CACHE.get(key) or autotune_exact(xd, wd, F, trunc))
    _, _, ws_bytes = _nx.exact_plan(M, N, K, cfg)
    ws = torch.empty(ws_bytes // 8, dtype=torch.int64, device=dev) if ws_bytes else None
    arr, n = _nx.cfg_array(cfg)
    with torch.cuda.device(dev):
        st = _nx.stream_handle(dev)
        _nx.check(_nx.lib().vxa_exact_linear(
            xh.data_ptr(), xl.data_ptr(), cx.data_ptr(), sx.data_ptr(), xh.stride(0),
            wh.data_ptr(), wl.data_ptr(), cw.data_ptr(), sw.data_ptr(), wh.stride(0),
            out.data_ptr(), _nx.dtype_enum(out.dtype), out.stride(0), M, N, K, int(F), int(bool(trunc)),
            arr, n, _nx.ptr(ws), ws_bytes, st), "exact_linear")
    return out


def _next_pow2(v):
    return 1 << max(0, (int(v) - 1).bit_length())


def autotune_exact(xd, wd, F, trunc):
    """Time every candidate (and split-K factor) and cache the fastest (kernels.py:292-316).
    Each candidate is timed by HIP-graph replay on the weights as given, the method of the
    reference's tuner (scripts/tune_table.py:38-57): a loop of launches timed with events
    favours configs with fewer launches and never picks split-K, where a graph, as vLLM's
    decode runs the op, does not. Candidates the kernels reject are skipped."""
    from .graph_timing import time_graph

    M, K = xd[0].shape
    N = wd[0].shape[0]
    key = (M, N, K, F, bool(trunc))
    out = torch.empty((M, N), device=xd[0].device, dtype=torch.float32)
    best = None
    for c in EXACT_CFGS:
        if c[0] > max(16, _next_pow2(M)):
            continue
        for sk in AUTOTUNE_SPLITS:
            cand = tuple(c) + (sk,)
            try:
                exact_linear(xd, wd, F, trunc, out=out, cfg=cand)
                torch.cuda.synchronize()
                t = time_graph(lambda i, cand=cand: exact_linear(xd, wd, F, trunc, out=out, cfg=cand),
                               calls_per_replay=10, replays=5)
            except (NotImplementedError, ValueError, RuntimeError):
                continue
            if best is None or t < best[0]:
                best = (t, cand)
    if best is None:
        raise RuntimeError(f"autotune_exact: no candidate config ran for M={M} N={N} K={K}")
    _CFG_CACHE[key] = best[1]
    return best[1]


__all__ = ["HAVE_HIP", "HAVE_TRITON", "digitize_torch", "digitize_weight", "digitize", "exact_linear_torch",
           "exact_linear", "autotune_exact", "EXACT_CFGS", "pack_digits", "digitize_packed", "exact_linear_packed",
           "packed_shape", "exact_linear_bf16x", "bf16x_rows_aligned", "ONE_LAUNCH_MAX_ROWS"]
