"""Paged decode attention with a fixed reduction order on MI355X, and the vLLM patch.

Kernel (libvllm_exact_amd.so, paged_decode.hip): one workgroup per (request, KV head,
segment of SPLIT keys). The segment length is fixed and the segment count is fixed by the
model's max length (paged_attn.py:3-5), so the grid is the same for every batch and the
floating-point order of a request depends only on its own length. QK^T runs on bf16
matrix cores (exact products, fp32 sums); the softmax is online in base 2; P V runs in fp32.
Segments are merged in segment order.

The kernel reads key/value caches as strided views (num_blocks, block_size, KV, D) with the
head dimension contiguous. The reference's vLLM FlashAttention cache (paged_attn.py:8-9),
kv_cache [num_blocks, num_kv_heads, block_size, 2*head_size], is one such pair of views;
install() derives the views from whichever backend it wraps (kv_cache_views).

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
                 warps=None, stages=None, split=None, n_live=None):
    """query (>=n, H, D) bf16; key/value_cache (num_blocks, block_size, KV, D) bf16 views;
    block_table (B, max_blocks) int32; seq_lens (B,) int32; out (>=n, H, D).
    Computes the first n requests only (paged_attn.py:97-114). The segments of SPLIT keys, and
    so the bits of every request, are fixed by MAX_LEN as in the reference. max_seq_len, which
    the reference accepts and leaves unused, is taken as a bound on seq_lens[:n] (vLLM's
    metadata keeps it one, also under graph capture): the grid then covers only the segments
    the bound can reach, which changes no bit of a request within it, and a request longer
    than the bound gets NaN rows rather than a sum over fewer keys. 0 or None: no bound.

    n_live: optional int32 GPU tensor of one element holding a count <= n. Only the first
    n_live requests are then computed and written, the count read by the kernel itself, so a
    count produced on the GPU needs no host round trip (n still sizes the grid)."""
    del stages
    n = int(n)
    bound = int(max_seq_len or 0)
    if bound < 0:
        raise ValueError(f"paged_decode: max_seq_len must be >= 0, got {bound}")
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
    if n_live is not None and (not n_live.is_cuda or n_live.dtype != torch.int32 or n_live.numel() != 1
                               or n_live.device != query.device):
        raise ValueError("paged_decode: n_live must be a one-element int32 tensor on the query's GPU")
    ws_bytes = _nx.paged_workspace(n, H, D, min(MAX_LEN, bound) if bound else MAX_LEN, split)
    ws = torch.empty(ws_bytes // 4, dtype=torch.float32, device=query.device) if ws_bytes else None
    dev = query.device
    with torch.cuda.device(dev):
        st = _nx.stream_handle(dev)
        head = (query.data_ptr(), query.stride(0), query.stride(1),
                key_cache.data_ptr(), key_cache.stride(0), key_cache.stride(1), key_cache.stride(2),
                value_cache.data_ptr(), value_cache.stride(0), value_cache.stride(1), value_cache.stride(2),
                block_table.data_ptr(), block_table.stride(0), seq_lens.data_ptr(), float(scale),
                out.data_ptr(), _nx.dtype_enum(out.dtype), out.stride(0), out.stride(1), n)
        tail = (H, KV, D, BS, int(MAX_LEN), bound, split, blk, warps, _nx.ptr(ws), ws_bytes, st)
        if n_live is None:
            _nx.check(_nx.lib().vxa_paged_decode(*head, *tail), "paged_decode")
        else:
            _nx.check(_nx.lib().vxa_paged_decode_prefix(*head, n_live.data_ptr(), *tail), "paged_decode")
    return out


def paged_decode_torch(query, key_cache, value_cache, block_table, seq_lens, scale, n):
    """fp32 torch statement of the same attention (paged_attn.py:117-132): for each request,
    the keys and values of its seq_lens[b] tokens are collected once through its block-table
    row, and each KV head's G query heads attend to them together as one batched product,
    softmax(q_g K_g^T * scale) V_g. Returns fp32 (n, H, D)."""
    page = key_cache.shape[1]
    H, D = query.shape[1], query.shape[2]
    KV = key_cache.shape[2]
    G = H // KV
    out = torch.empty(n, H, D, device=query.device, dtype=torch.float32)
    for b in range(n):
        L = int(seq_lens[b])
        tok = torch.arange(L, device=query.device)
        blk = block_table[b].long()[tok // page]
        slot = tok % page
        # (KV, L, D) per cache: token rows of each KV head
        keys = key_cache[blk, slot].float().permute(1, 0, 2).contiguous()
        vals = value_cache[blk, slot].float().permute(1, 0, 2).contiguous()
        q = query[b].float().view(KV, G, D)
        scores = torch.bmm(q, keys.transpose(1, 2).contiguous()) * scale  # (KV, G, L)
        out[b] = torch.bmm(torch.softmax(scores, dim=-1), vals).reshape(H, D)
    return out


# vLLM attention backends install() can wrap: name -> (module, impl class, backend class).
# The reference patches FLASH_ATTN only (paged_attn.py:135-163); on ROCm vLLM may route
# decode through TRITON_ATTN, whose KV cache stacks K and V on an axis of its own. vLLM's
# ROCM_ATTN backend is not offered: it declares a (2, blocks, page, heads, dim) shape but
# reads and writes K through an x-packed layout ([blocks, heads, dim / x, page, x]), so views
# taken from its declared shape would read K at the wrong offsets.
BACKENDS = {
    "FLASH_ATTN": ("vllm.v1.attention.backends.flash_attn", "FlashAttentionImpl", "FlashAttentionBackend"),
    "TRITON_ATTN": ("vllm.v1.attention.backends.triton_attn", "TritonAttentionImpl", "TritonAttentionBackend"),
}


def writes_cache_outside_forward(backend_cls, impl_cls):
    """True when the backend stores new keys and values in the KV cache outside its forward:
    it declares forward_includes_kv_cache_update = False, or, where vLLM has no such flag,
    its impl has the separate do_kv_cache_update step. install() skips the backend's forward
    on decode-only steps (as the reference does), so a backend that writes the cache inside
    forward would never store the new token's key and value."""
    flag = getattr(backend_cls, "forward_includes_kv_cache_update", None)
    if flag is not None:
        return not flag
    return callable(getattr(impl_cls, "do_kv_cache_update", None))


def kv_cache_views(shape_of, num_kv_heads, head_size):
    """Split function for a backend's KV cache: kv_cache -> (key_cache, value_cache), both
    views (num_blocks, block_size, num_kv_heads, head_size) as paged_decode takes them.

    shape_of is the backend's get_kv_cache_shape(num_blocks, block_size, num_kv_heads,
    head_size). Two probes with different sizes name its axes: the block, page and head axes
    change between them, and what stays is either a size-2 axis plus a head_size axis (K and
    V stacked) or one 2 * head_size axis (K then V per row, the layout paged_attn.py:8-9
    describes). Views only: the kernel reads the cache through their strides. Layouts that
    merge axes raise NotImplementedError."""
    a = tuple(int(v) for v in shape_of(7, 16, num_kv_heads, head_size))
    b = tuple(int(v) for v in shape_of(11, 32, num_kv_heads + 1, head_size))

    def axis(x, y, what):
        hits = [i for i in range(len(a)) if a[i] == x and b[i] == y]
        if len(a) != len(b) or len(hits) != 1:
            raise NotImplementedError(f"KV cache shape {a}: no single {what} axis")
        return hits[0]

    blocks, pages, heads = axis(7, 11, "block"), axis(16, 32, "page"), axis(num_kv_heads, num_kv_heads + 1, "head")
    rest = [i for i in range(len(a)) if i not in (blocks, pages, heads)]
    sizes = sorted(a[i] for i in rest)
    if len(rest) == 1 and sizes == [2 * head_size]:
        dim = rest[0]
        order = (blocks, pages, heads, dim)
        return lambda t: tuple(t.narrow(dim, j * head_size, head_size).permute(*order) for j in (0, 1))
    if len(rest) == 2 and head_size != 2 and sizes == sorted((2, head_size)):
        kv = next(i for i in rest if a[i] == 2)
        dim = next(i for i in rest if a[i] == head_size)
        order = tuple(i - (i > kv) for i in (blocks, pages, heads, dim))  # axes once kv is selected away
        return lambda t: tuple(t.select(kv, j).permute(*order) for j in (0, 1))
    raise NotImplementedError(f"KV cache shape {a}: K and V are neither a size-2 axis nor a 2*head_size axis")


def leading_decodes(query_start_loc):
    """Number of leading requests with one query token, as a one-element int32 tensor on the
    same device (vLLM orders decode requests first; paged_attn.py:154-156). Nothing is read
    back to the host."""
    one = (query_start_loc[1:] - query_start_loc[:-1]) == 1
    return torch.cumprod(one.to(torch.int32), 0).sum().to(torch.int32).reshape(1)


def install(backend="FLASH_ATTN"):
    """Wrap the forward of a vLLM attention backend (BACKENDS) so that every decode token goes
    through paged_decode and every other token through the backend itself (paged_attn.py:
    135-163). Call before creating the LLM, with the engine in-process; returns the original
    forward.

    * No metadata (profiling) or a non-decoder layer: the backend alone.
    * Decode-only step (max_query_len == 1): paged_decode alone, for num_actual_tokens
      requests (graph-capturable, no host synchronisation).
    * Mixed step: the backend first, then paged_decode over the leading decode requests,
      overwriting their rows. Their count stays on the GPU (leading_decodes): the grid covers
      every request and the kernel skips those past the count.
    A request's attention output is then always computed by the same kernel in the same
    order, whatever the rest of the batch is. The wrapped backend must write new keys and
    values to the cache outside forward, as the reference's vLLM does: on decode-only steps
    the backend's forward is not called. A backend that does not say so
    (writes_cache_outside_forward) is refused with NotImplementedError."""
    import importlib

    if backend not in BACKENDS:
        raise ValueError(f"install: backend must be one of {sorted(BACKENDS)}, got {backend!r}")
    module_name, impl_name, backend_name = BACKENDS[backend]
    module = importlib.import_module(module_name)
    impl_cls = getattr(module, impl_name)
    backend_cls = getattr(module, backend_name)
    if not writes_cache_outside_forward(backend_cls, impl_cls):
        raise NotImplementedError(
            f"install: {backend_name} does not declare that it writes the KV cache outside forward; decode-only "
            "steps skip its forward, so the new token's key and value would never be stored")
    decoder = module.AttentionType.DECODER
    original = impl_cls.forward
    splits = {}

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None, *args, **kwargs):
        md = attn_metadata
        if md is None or getattr(self, "attn_type", decoder) != decoder:
            return original(self, layer, query, key, value, kv_cache, md, output, *args, **kwargs)
        shape = (self.num_kv_heads, self.head_size)
        if shape not in splits:
            splits[shape] = kv_cache_views(backend_cls.get_kv_cache_shape, *shape)
        key_cache, value_cache = splits[shape](kv_cache)
        rows = output.view(output.shape[0], self.num_heads, self.head_size)
        if md.max_query_len == 1:
            if md.num_actual_tokens > 0:
                paged_decode(query, key_cache, value_cache, md.block_table, md.seq_lens, self.scale, rows,
                             md.num_actual_tokens, md.max_seq_len)
            return output
        result = original(self, layer, query, key, value, kv_cache, md, output, *args, **kwargs)
        n_req = md.query_start_loc.shape[0] - 1
        if n_req > 0:
            paged_decode(query, key_cache, value_cache, md.block_table, md.seq_lens, self.scale, rows, n_req,
                         md.max_seq_len, n_live=leading_decodes(md.query_start_loc))
        return result

    impl_cls.forward = forward
    return original


def default_scale(head_dim):
    return 1.0 / math.sqrt(head_dim)
