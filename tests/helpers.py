"""Shared test data: seeded CPU generators (device RNG streams are not portable), conversions
between torch tensors and the oracle's numpy arrays."""
import numpy as np
import torch


def xw(M, N, K, seed=0, outlier=True, x_scale=1.0, w_scale=0.02):
    """x ~ N(0, 1), w ~ N(0, 0.02) drawn in that order from one CPU generator
    (tests/test_reference_cpu.py:7-13 of the reference)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g) * x_scale
    if outlier:
        x[:, 3 % max(K, 1)] *= 500
    w = torch.randn(N, K, generator=g) * w_scale
    return x, w


def stress_xw(M, N, K, seed=0):
    """Outlier columns push digits to |d| ~ 128 (tests/test_gpu.py:19-23 of the reference)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    x[:, 7 % K] *= 300
    w = torch.randn(N, K, generator=g) * 0.02
    w[:, 3 % K] *= 300
    return x, w


def np_digits(d):
    return tuple(t.detach().cpu().numpy() for t in d)


def torch_digits(d, device=None):
    return tuple(torch.from_numpy(np.ascontiguousarray(t)).to(device) for t in d)


def bf16_bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def f32_bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def make_paged(B, L, BS, H, KV, D, seed=0, spare=7, var_len=True, kv_scale=1.0):
    """Synthetic paged cache in vLLM's FlashAttention layout [num_blocks, KV, BS, 2D] bf16,
    a block table of random page permutations of a shared pool, and seq_lens in [L/2, L]
    (tests/test_gpu.py:46-54 of the reference), all drawn on the CPU."""
    g = torch.Generator().manual_seed(seed)
    nbp = (L + BS - 1) // BS
    nblocks = B * nbp + spare
    kv = (torch.randn(nblocks, KV, BS, 2 * D, generator=g) * kv_scale).to(torch.bfloat16)
    bt = torch.randperm(nblocks, generator=g)[:B * nbp].view(B, nbp).to(torch.int32)
    q = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
    if var_len:
        sl = torch.randint(L // 2, L + 1, (B,), generator=g).to(torch.int32)
    else:
        sl = torch.full((B,), L, dtype=torch.int32)
    return q, kv, bt, sl


def kv_views(kv, D):
    """key/value views (num_blocks, BS, KV, D) of a [num_blocks, KV, BS, 2D] cache."""
    return kv.transpose(1, 2).split(D, dim=-1)


def pack_np(h, l):
    """Fragment-major layout written out in numpy, as documented for vxa_pack_digits:
    block (rt, kt) = [h fragment | l fragment], fragment byte 16*lane + j = row 16rt + (lane & 15),
    column 64kt + 16(lane >> 4) + j; padding rows/columns are zero."""
    R, K = h.shape
    RT, KT = (R + 15) // 16, (K + 63) // 64
    out = np.zeros((RT, KT, 2, 64, 16), np.int8)
    hp = np.zeros((RT * 16, KT * 64), np.int8)
    lp = np.zeros((RT * 16, KT * 64), np.int8)
    hp[:R, :K] = h
    lp[:R, :K] = l
    lane = np.arange(64)
    for plane, src in ((0, hp), (1, lp)):
        blk = src.reshape(RT, 16, KT, 4, 16)  # rt, r16, kt, kq, j
        # lane = 16*kq + r16
        out[:, :, plane] = blk.transpose(0, 2, 3, 1, 4).reshape(RT, KT, 64, 16)[:, :, lane]
    return out.reshape(RT, KT, 2, 1024)
