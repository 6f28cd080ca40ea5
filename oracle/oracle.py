"""CPU oracle for the exact linear path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module,
and only to check results (or as the timed CPU baseline); the product never does.

Two independent restatements of the reference's CPU arithmetic:
* numpy (this file): digitize_np <- kernels.py:22-39, exact_linear_np <- kernels.py:89-100,
  bf16_rne_np <- fp32 -> bf16 RNE, paged_decode_np <- paged_attn.py:117-132 in float64;
* C with OpenMP (exact_oracle.c, loaded through ctypes as liboracle.so): the same functions,
  fast enough for full-size sampled checks and the CPU baseline.
tests/test_oracle.py pins both against closed forms, hand-computed known answers, exact
integer brute force and library routines.
"""
import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"


# ----------------------------------------------------------------------------- numpy
def digitize_np(x, F):
    """(R, K) float32 -> (h int8, l int8, cs int32, sh int32) (kernels.py:22-39)."""
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x).max(axis=1) if x.shape[1] else np.zeros(x.shape[0], np.float32)
    _, e = np.frexp(a)
    e = np.where(a > 0, e, 0).astype(np.int32)
    sh = (F - e).astype(np.int32)
    scale = ((sh.astype(np.int64) + 127) << 23).astype(np.uint32).view(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        q = np.trunc(x * scale[:, None]).astype(np.int64)
    if F == 15:
        lo = (q & 255) - 128
        hi = (q - lo - 128) >> 8
        cs = (256 * hi + lo).sum(axis=1).astype(np.int32)
    else:
        lo = ((q + 128) & 255) - 128
        hi = (q - lo) >> 8
        cs = np.zeros_like(sh)
    return hi.astype(np.int8), lo.astype(np.int8), cs, sh


def exact_tot_np(xd, wd, F, trunc):
    """int64 tot[m, n] of the integer closed form (kernels.py:93-97)."""
    xh, xl, cx, _ = (np.asarray(t, np.int64) for t in xd)
    wh, wl, cw, _ = (np.asarray(t, np.int64) for t in wd)
    K = xh.shape[1]
    tot = (xh @ wh.T) * 65536 + (xh @ wl.T + xl @ wh.T) * 256
    if not trunc:
        tot = tot + xl @ wl.T
    if F == 15:
        tot = tot + 128 * (cx[:, None] + cw[None, :]) + 128 * 128 * K
    return tot


def exact_linear_np(xd, wd, F, trunc):
    """fp32 (M, N) result: fp64(tot) * 2^-(sx+sw), then one rounding to fp32 (kernels.py:98-100)."""
    tot = exact_tot_np(xd, wd, F, trunc)
    e = -(np.asarray(xd[3], np.int64)[:, None] + np.asarray(wd[3], np.int64)[None, :])
    scale = ((e + 1023) << 52).astype(np.uint64).view(np.float64)
    return (tot.astype(np.float64) * scale).astype(np.float32)


def bf16_rne_np(x):
    """fp32 -> bf16 bit patterns (uint16), round to nearest even; NaN -> 0x7FC0."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def bf16_bits_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def paged_decode_np(q_bits, kc_bits, vc_bits, block_table, seq_lens, scale, n):
    """Float64 decode attention (paged_attn.py:117-132).

    q_bits (B, H, D) and kc_bits / vc_bits (num_blocks, BS, KV, D) are bf16 bit patterns
    (uint16); returns (n, H, D) float64."""
    q = bf16_bits_to_f32(q_bits).astype(np.float64)
    kc = bf16_bits_to_f32(kc_bits).astype(np.float64)
    vc = bf16_bits_to_f32(vc_bits).astype(np.float64)
    BS, KV = kc.shape[1], kc.shape[2]
    H, D = q.shape[1], q.shape[2]
    G = H // KV
    out = np.zeros((n, H, D))
    for b in range(n):
        L = int(seq_lens[b])
        pos = np.arange(L)
        pages = np.asarray(block_table)[b, pos // BS].astype(np.int64)
        k = kc[pages, pos % BS]  # (L, KV, D)
        v = vc[pages, pos % BS]
        for h in range(H):
            s = (k[:, h // G] @ q[b, h]) * scale
            p = np.exp(s - s.max())
            out[b, h] = (p / p.sum()) @ v[:, h // G]
    return out


# ----------------------------------------------------------------------------- C library
def build(force=False):
    """Compile exact_oracle.c into liboracle.so with the recipe in oracle/Makefile."""
    if LIB_PATH.exists() and not force:
        return LIB_PATH
    subprocess.run(["make", "-C", str(HERE)] + (["-B"] if force else []), check=True, capture_output=True)
    return LIB_PATH


_clib = None


def clib():
    global _clib
    if _clib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P, i64, i32, f64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double
        L.oracle_digitize_f32.argtypes = [P, i64, i64, i32, P, P, P, P]
        L.oracle_digitize_f32.restype = i32
        L.oracle_exact_linear.argtypes = [P, P, P, P, P, P, P, P, i64, i64, i64, i32, i32, P]
        L.oracle_exact_linear.restype = i32
        L.oracle_exact_entries.argtypes = [P, P, P, P, P, P, P, P, i64, i32, i32, P, P, i64, P]
        L.oracle_exact_entries.restype = i32
        L.oracle_f32_to_bf16.argtypes = [P, i64, P]
        L.oracle_f32_to_bf16.restype = None
        L.oracle_paged_decode_f64.argtypes = [P, i64, i64, P, i64, i64, i64, P, i64, i64, i64, P, i64, P, f64, i64,
                                              i64, i64, i64, i64, P]
        L.oracle_paged_decode_f64.restype = i32
        _clib = L
    return _clib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def digitize_c(x, F):
    x = np.ascontiguousarray(x, dtype=np.float32)
    R, K = x.shape
    h = np.empty((R, K), np.int8)
    l = np.empty((R, K), np.int8)
    cs = np.empty(R, np.int32)
    sh = np.empty(R, np.int32)
    if clib().oracle_digitize_f32(_p(x), R, K, F, _p(h), _p(l), _p(cs), _p(sh)) != 0:
        raise ValueError(f"oracle digitize: bad F={F}")
    return h, l, cs, sh


def _digits(d):
    h, l, c, s = d
    return (np.ascontiguousarray(h, np.int8), np.ascontiguousarray(l, np.int8), np.ascontiguousarray(c, np.int32),
            np.ascontiguousarray(s, np.int32))


def exact_linear_c(xd, wd, F, trunc):
    xh, xl, cx, sx = _digits(xd)
    wh, wl, cw, sw = _digits(wd)
    M, K = xh.shape
    N = wh.shape[0]
    out = np.empty((M, N), np.float32)
    clib().oracle_exact_linear(_p(xh), _p(xl), _p(cx), _p(sx), _p(wh), _p(wl), _p(cw), _p(sw), M, N, K, F,
                               int(bool(trunc)), _p(out))
    return out


def exact_entries_c(xd, wd, F, trunc, rows, cols):
    xh, xl, cx, sx = _digits(xd)
    wh, wl, cw, sw = _digits(wd)
    rows = np.ascontiguousarray(rows, np.int64)
    cols = np.ascontiguousarray(cols, np.int64)
    out = np.empty(rows.shape[0], np.float32)
    clib().oracle_exact_entries(_p(xh), _p(xl), _p(cx), _p(sx), _p(wh), _p(wl), _p(cw), _p(sw), xh.shape[1], F,
                                int(bool(trunc)), _p(rows), _p(cols), rows.shape[0], _p(out))
    return out


def bf16_rne_c(x):
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.empty(x.shape[0], np.uint16)
    clib().oracle_f32_to_bf16(_p(x), x.shape[0], _p(out))
    return out


def paged_decode_c(q_bits, kc_bits, vc_bits, block_table, seq_lens, scale, n):
    """Same contract as paged_decode_np; q (B, H, D) and caches (num_blocks, BS, KV, D) as
    contiguous uint16 bf16 bit arrays."""
    q = np.ascontiguousarray(q_bits, np.uint16)
    kc = np.ascontiguousarray(kc_bits, np.uint16)
    vc = np.ascontiguousarray(vc_bits, np.uint16)
    bt = np.ascontiguousarray(block_table, np.int32)
    sl = np.ascontiguousarray(seq_lens, np.int32)
    B, H, D = q.shape
    nb, BS, KV, _ = kc.shape
    out = np.empty((n, H, D), np.float64)
    clib().oracle_paged_decode_f64(_p(q), H * D, D, _p(kc), BS * KV * D, KV * D, D, _p(vc), BS * KV * D, KV * D, D,
                                   _p(bt), bt.shape[1], _p(sl), float(scale), n, H, KV, D, BS, _p(out))
    return out


def cpu_threads():
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
