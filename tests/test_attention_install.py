"""CPU checks of the vLLM wiring of the paged decode kernel (paged_attn.py:135-163 of the
reference): the KV-cache views derived from a backend's declared layout, the routing of
decode-only, mixed and other steps, and the on-GPU count of leading decode requests. vLLM is
not installed here: a stand-in backend module with the same names is registered in
sys.modules, and paged_decode is replaced by a recorder (the kernel itself is checked on the
GPU in test_gpu_attention.py)."""
import sys
import types

import pytest
import torch

import vllm_exact
from vllm_exact import paged_attn as P

NB, BS, KV, D, H = 5, 16, 2, 8, 4

LAYOUTS = {
    # declared shape, and where key / value element (block b, page slot p, head h, dim d) lives
    "blocks, heads, page, 2*dim (the reference's)": (
        lambda nb, bs, kv, d: (nb, kv, bs, 2 * d), lambda b, p, h, d: (b, h, p, d), lambda b, p, h, d: (b, h, p, D + d)),
    "K/V first": (
        lambda nb, bs, kv, d: (2, nb, bs, kv, d), lambda b, p, h, d: (0, b, p, h, d), lambda b, p, h, d: (1, b, p, h, d)),
    "K/V second": (
        lambda nb, bs, kv, d: (nb, 2, bs, kv, d), lambda b, p, h, d: (b, 0, p, h, d), lambda b, p, h, d: (b, 1, p, h, d)),
    "K/V first, heads before page": (
        lambda nb, bs, kv, d: (2, nb, kv, bs, d), lambda b, p, h, d: (0, b, h, p, d), lambda b, p, h, d: (1, b, h, p, d)),
}


@pytest.mark.parametrize("name", sorted(LAYOUTS))
@pytest.mark.parametrize("kv_heads", [KV, 16])
def test_kv_cache_views_follow_the_declared_layout(name, kv_heads):
    shape_of, kpos, vpos = LAYOUTS[name]
    t = torch.arange(int(torch.tensor(shape_of(NB, BS, kv_heads, D)).prod())).view(*shape_of(NB, BS, kv_heads, D))
    key, value = P.kv_cache_views(shape_of, kv_heads, D)(t)
    assert key.shape == value.shape == (NB, BS, kv_heads, D)
    assert key.stride(-1) == 1 and value.stride(-1) == 1  # views, head dim contiguous
    assert key.untyped_storage().data_ptr() == t.untyped_storage().data_ptr()
    g = torch.Generator().manual_seed(0)
    for _ in range(50):
        b, p, h, d = (int(torch.randint(0, s, (1,), generator=g)) for s in (NB, BS, kv_heads, D))
        assert key[b, p, h, d] == t[kpos(b, p, h, d)]
        assert value[b, p, h, d] == t[vpos(b, p, h, d)]


def test_kv_cache_views_refuse_merged_layouts():
    with pytest.raises(NotImplementedError):
        P.kv_cache_views(lambda nb, bs, kv, d: (2, nb, bs * kv * d), KV, D)
    with pytest.raises(NotImplementedError):
        P.kv_cache_views(lambda nb, bs, kv, d: (nb, bs, kv * d * 2), KV, D)


@pytest.mark.parametrize("qsl,want", [([0, 1, 2, 5, 9], 2), ([0, 1, 4, 5], 1), ([0, 3, 4], 0), ([0, 1, 2, 3], 3)])
def test_leading_decodes_counts_on_device(qsl, want):
    n = P.leading_decodes(torch.tensor(qsl, dtype=torch.int32))
    assert n.dtype == torch.int32 and n.shape == (1,) and int(n) == want


@pytest.fixture
def backend(monkeypatch):
    """A stand-in vllm.v1.attention.backends.flash_attn with the reference's cache layout."""
    for name in ("vllm", "vllm.v1", "vllm.v1.attention", "vllm.v1.attention.backends"):
        monkeypatch.setitem(sys.modules, name, types.ModuleType(name))
    mod = types.ModuleType("vllm.v1.attention.backends.flash_attn")

    class AttentionType:
        DECODER = "decoder"
        ENCODER_ONLY = "encoder_only"

    class FlashAttentionBackend:
        forward_includes_kv_cache_update = False  # new keys/values are stored outside forward

        @staticmethod
        def get_kv_cache_shape(num_blocks, block_size, num_kv_heads, head_size, cache_dtype_str="auto"):
            if block_size % 16:
                raise ValueError("block size must be a multiple of 16")
            return (num_blocks, num_kv_heads, block_size, 2 * head_size)

    class FlashAttentionImpl:
        calls = []

        def __init__(self, attn_type=AttentionType.DECODER):
            self.num_heads, self.num_kv_heads, self.head_size, self.scale = H, KV, D, 0.25
            self.attn_type = attn_type

        def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None, output_scale=None,
                    output_block_scale=None):
            FlashAttentionImpl.calls.append((attn_metadata, output_scale))
            output.fill_(3.0)
            return output

    mod.AttentionType, mod.FlashAttentionBackend, mod.FlashAttentionImpl = (AttentionType, FlashAttentionBackend,
                                                                              FlashAttentionImpl)
    monkeypatch.setitem(sys.modules, mod.__name__, mod)
    decodes = []

    def record(query, key_cache, value_cache, block_table, seq_lens, scale, out, n, max_seq_len, n_live=None, **kw):
        decodes.append(dict(key=key_cache, value=value_cache, n=n, n_live=None if n_live is None else int(n_live),
                            out=out, scale=scale))
        return out

    monkeypatch.setattr(P, "paged_decode", record)
    return mod, decodes


def _md(max_query_len, num_actual_tokens, qsl):
    return types.SimpleNamespace(max_query_len=max_query_len, num_actual_tokens=num_actual_tokens,
                                 query_start_loc=torch.tensor(qsl, dtype=torch.int32),
                                 block_table=torch.zeros(len(qsl) - 1, 4, dtype=torch.int32),
                                 seq_lens=torch.ones(len(qsl) - 1, dtype=torch.int32), max_seq_len=64)


def test_install_routes_each_kind_of_step(backend):
    mod, decodes = backend
    impl_cls = mod.FlashAttentionImpl
    original = impl_cls.forward
    assert P.install("FLASH_ATTN") is original
    impl = impl_cls()
    kv_cache = torch.arange(NB * KV * BS * 2 * D, dtype=torch.float32).view(NB, KV, BS, 2 * D)
    q = torch.zeros(9, H, D)

    def call(md, impl=impl, **kw):
        out = torch.zeros(9, H * D)
        res = impl.forward(None, q, None, None, kv_cache, md, out, **kw)
        return out, res

    # profiling pass (no metadata) and a non-decoder layer: the backend alone
    call(None)
    call(_md(1, 2, [0, 1, 2]), impl=impl_cls(attn_type=mod.AttentionType.ENCODER_ONLY))
    assert len(impl_cls.calls) == 2 and not decodes

    # decode-only step: the kernel alone, for num_actual_tokens requests, no count tensor
    out, res = call(_md(1, 3, [0, 1, 2, 3]))
    assert res is out and len(impl_cls.calls) == 2 and len(decodes) == 1
    d = decodes[-1]
    assert d["n"] == 3 and d["n_live"] is None and d["scale"] == 0.25
    assert d["out"].shape == (9, H, D) and d["out"].data_ptr() == out.data_ptr()
    assert torch.equal(d["key"], kv_cache.transpose(1, 2)[..., :D])
    assert torch.equal(d["value"], kv_cache.transpose(1, 2)[..., D:])
    call(_md(1, 0, [0]))  # empty step: nothing launched
    assert len(decodes) == 1 and len(impl_cls.calls) == 2

    # mixed step: the backend, then the kernel over every request with the leading-decode
    # count left on the device; extra keyword arguments reach the backend unchanged
    out, res = call(_md(4, 9, [0, 1, 2, 5, 9]), output_scale="s")
    assert len(impl_cls.calls) == 3 and impl_cls.calls[-1][1] == "s"
    assert res is out and torch.all(out == 3.0)
    assert decodes[-1]["n"] == 4 and decodes[-1]["n_live"] == 2
    call(_md(3, 5, [0, 3, 4, 5]))  # a prefill first: no leading decodes, the kernel skips all
    assert decodes[-1]["n"] == 3 and decodes[-1]["n_live"] == 0


def test_enable_checks_the_backend_name(monkeypatch):
    monkeypatch.delitem(sys.modules, "vllm", raising=False)
    with pytest.raises(ValueError, match="attention_backend"):
        vllm_exact.enable(1024, attention_backend="NO_SUCH_BACKEND")
    assert not vllm_exact._ENABLED


def test_install_refuses_backends_that_write_the_cache_in_forward(backend):
    """Decode-only steps skip the backend's forward, so a backend whose forward stores the new
    token's key and value (or that does not say where it stores them) is refused."""
    mod, _ = backend
    original = mod.FlashAttentionImpl.forward
    mod.FlashAttentionBackend.forward_includes_kv_cache_update = True
    with pytest.raises(NotImplementedError, match="outside forward"):
        P.install("FLASH_ATTN")
    del mod.FlashAttentionBackend.forward_includes_kv_cache_update  # older vLLM: no flag at all
    with pytest.raises(NotImplementedError, match="outside forward"):
        P.install("FLASH_ATTN")
    mod.FlashAttentionImpl.do_kv_cache_update = lambda self, *a: None  # ... but a separate cache step
    assert P.install("FLASH_ATTN") is original
    mod.FlashAttentionImpl.forward = original


def test_install_offers_no_backend_with_an_undeclared_physical_layout():
    """vLLM's ROCM_ATTN reads K through an x-packed layout its declared shape does not show."""
    assert "ROCM_ATTN" not in P.BACKENDS
    with pytest.raises(ValueError, match="backend must be one of"):
        P.install("ROCM_ATTN")
