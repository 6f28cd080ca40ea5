"""Paged decode attention with a fixed reduction order on MI355X, and the vLLM patch.

Kernel (libvllm_exact_amd.so, paged_decode.hip): one workgroup per (request, KV head,
segment of SPLIT keys). The segment length is fixed and the segment count is fixed by the
model's max length (paged_attn.py:3-5), so the grid is the same for every batch and the
floating-point order of a request depends only on its own length. QK^T runs on bf16
matrix cores (exact products, fp32 sums); the softmax is online in base 2; P V runs in fp32.
Segments are merged in segment order.

KV layout follows vLLM FlashAttention (paged_attn.py:8-9):
kv_cache [num_blocks, num_kv_heads, block_size, 2*head_size];
key_cache = kv_cache.transpose(1, 2)[..., :D], value_cache = [..., D:] (strided views).

SPLIT, BLK and WARPS change the floating-point order: one deployment uses one fixed set.
STAGES is accepted for the reference's signature and has no effect here.
"""
import math

import torch

from . import _native as _nx

# gfx950 defaults, measured at H32/KV8/D128/BS16 (64x8K, 16x16K, 256x1K): one 16-key tile per
# wave step keeps the kernel at 4 waves per SIMD, and 2048-key segments keep enough
# workgroups in flight at 16x16K.
SPLIT = 2048
BLK = 16
WARPS = 4
STAGES = 1
MAX_LEN = 16384  # fixes the number of segments; enable() sets it to max_model_len


def paged_decode(query, key_cache, value_cache, block_table, seq_lens, scale, out, n, max_seq_len, blk=None,
                 warps=None, stages=None, split=None):
    """query (>=n, H, D) bf16; key/value_cache (num_blocks, block_size, KV, D) bf16 views;
    block_table (B, max_blocks) int32; seq_lens (B,) int32; out (>=n, H, D).
    Computes the first n requests only (paged_attn.py:97-114). max_seq_len is accepted and
    unused, as in the reference: the grid is fixed by MAX_LEN."""
    del max_seq_len, stages
    n = int(n)
    if n <= 0:
        return out
    blk, warps, split = int(blk or BLK), int(warps or WARPS), int(split or SPLIT)
    for t in (query, key_cache, value_cache, block_table, seq_lens, out):
        if not t.is_cuda:
            raise ValueError("paged_decode runs the gfx950 HIP kernel and needs GPU tensors; "
                             "use paged_decode_torch for the CPU statement")
    _nx.lib()
    if query.dtype != torch.bfloat16 or key_cache.dtype != torch.bfloat16 or value_cache.dtype != torch.bfloat16:
        raise NotImplementedError("paged_decode: query and KV cache must be bf16")
    if block_table.dtype != torch.int32 or seq_lens.dtype != torch.int32:
        raise ValueError("paged_decode: block_table and seq_lens must be int32")
    if query.stride(2) != 1 or key_cache.stride(3) != 1 or value_cache.stride(3) != 1 or out.stride(2) != 1:
        raise ValueError("paged_decode: the head dimension must be contiguous")
    if block_table.stride(1) != 1 or not seq_lens.is_contiguous():
        raise ValueError("paged_decode: block_table rows and seq_lens must be contiguous")
    H, D = query.shape[1], query.shape[2]
    KV = key_cache.shape[2]
    BS = key_cache.shape[1]
    if value_cache.shape != key_cache.shape or out.shape[1:] != (H, D) or query.shape[0] < n or out.shape[0] < n:
        raise ValueError("paged_decode: inconsistent shapes")
    if seq_lens.shape[0] < n or block_table.shape[0] < n:
        raise ValueError("paged_decode: fewer block-table rows or lengths than requests")
    ws_bytes = _nx.paged_workspace(n, H, D, MAX_LEN, split)
    ws = torch.empty(ws_bytes // 4, dtype=torch.float32, device=query.device) if ws_bytes else None
    dev = query.device
    with torch.cuda.device(dev):
        st = _nx.stream_handle(dev)
        _nx.check(_nx.lib().vxa_paged_decode(
            query.data_ptr(), query.stride(0), query.stride(1),
            key_cache.data_ptr(), key_cache.stride(0), key_cache.stride(1), key_cache.stride(2),
            value_cache.data_ptr(), value_cache.stride(0), value_cache.stride(1), value_cache.stride(2),
            block_table.data_ptr(), block_table.stride(0), seq_lens.data_ptr(), float(scale),
            out.data_ptr(), _nx.dtype_enum(out.dtype), out.stride(0), out.stride(1),
            n, H, KV, D, BS, int(MAX_LEN), split, blk, warps, _nx.ptr(ws), ws_bytes, st), "paged_decode")
    return out


def paged_decode_torch(query, key_cache, value_cache, block_table, seq_lens, scale, n):
    """fp32 torch statement of the same attention (paged_attn.py:117-132): per request,
    gather its keys/values through the block table, softmax(K q * scale) V per head."""
    BS = key_cache.shape[1]
    H, D = query.shape[1], query.shape[2]
    KV = key_cache.shape[2]
    G = H // KV
    out = torch.empty(n, H, D, device=query.device, dtype=torch.float32)
    for b in range(n):
        L = int(seq_lens[b])
        pos = torch.arange(L, device=query.device)
        pages = block_table[b, pos // BS].long()
        k = key_cache[pages, pos % BS].float()  # (L, KV, D)
        v = value_cache[pages, pos % BS].float()
        for h in range(H):
            logits = (k[:, h // G] @ query[b, h].float()) * scale
            out[b, h] = torch.softmax(logits, 0) @ v[:, h // G]
    return out


def install():
    """Patch vLLM's FlashAttentionImpl.forward so every decode token goes through
    paged_decode and every prefill token through vLLM's own implementation
    (paged_attn.py:135-163). Call before creating the LLM, with the engine in-process."""
    from vllm.v1.attention.backends import flash_attn as fa

    orig = fa.FlashAttentionImpl.forward
    decoder = fa.AttentionType.DECODER

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output, output_scale=None,
                output_block_scale=None):
        if attn_metadata is None or self.attn_type != decoder:
            return orig(self, layer, query, key, value, kv_cache, attn_metadata, output, output_scale,
                        output_block_scale)
        D = self.head_size
        key_cache, value_cache = kv_cache.transpose(1, 2).split(D, dim=-1)
        out3 = output.view(output.shape[0], self.num_heads, D)
        if attn_metadata.max_query_len == 1:
            n = attn_metadata.num_actual_tokens
            if n > 0:
                paged_decode(query, key_cache, value_cache, attn_metadata.block_table, attn_metadata.seq_lens,
                             self.scale, out3, n, attn_metadata.max_seq_len)
            return output
        res = orig(self, layer, query, key, value, kv_cache, attn_metadata, output, output_scale,
                   output_block_scale)
        qsl = attn_metadata.query_start_loc
        qlen = qsl[1:] - qsl[:-1]
        # leading decode requests (vLLM orders decodes first); mixed steps run eagerly
        nd = int(torch.cumprod((qlen == 1).to(torch.int32), 0).sum().item())
        if nd > 0:
            paged_decode(query, key_cache, value_cache, attn_metadata.block_table, attn_metadata.seq_lens,
                         self.scale, out3, nd, attn_metadata.max_seq_len)
        return res

    fa.FlashAttentionImpl.forward = forward
    return orig


def default_scale(head_dim):
    return 1.0 / math.sqrt(head_dim)
