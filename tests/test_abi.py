"""CPU checks of the C ABI: the library loads, exports every symbol include/*.h declares, and
its host-only entry points (plans, workspace sizes, argument validation) behave as
documented. No kernel is launched here."""
import ctypes
import re
from pathlib import Path

import pytest

from vllm_exact import _native as nx

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    names = set()
    for hdr in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", hdr.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(vxa_\w+)\s*\(", text))
    return names


def test_library_loads_and_exports_every_declared_symbol():
    assert nx.available(), "build the HIP library first (make -C vllm-exact_amd)"
    lib = ctypes.CDLL(str(nx.LIB_PATH))
    declared = declared_functions()
    assert declared == set(nx.EXPORTED), declared ^ set(nx.EXPORTED)
    for name in declared:
        assert hasattr(lib, name), name


def test_version_and_status_strings():
    assert "gfx950" in nx.version()
    L = nx.lib()
    assert L.vxa_status_string(nx.VXA_OK) == b"ok"
    assert b"workspace" in L.vxa_status_string(nx.VXA_ERR_WORKSPACE)


def _plan(M, N, K, cfg):
    return nx.exact_plan(M, N, K, cfg)


def test_split_k_plan_follows_reference_arithmetic():
    # kernels.py:271-272: KCH = cdiv(cdiv(K, SK), BK) * BK, SK = cdiv(K, KCH)
    assert _plan(16, 4096, 4096, (16, 64, 128, 4, 3, 8, 1)) == (1, 4096, 0)
    assert _plan(16, 4096, 4096, (16, 64, 128, 4, 3, 8, 4)) == (4, 1024, 4 * 16 * 4096 * 8)
    assert _plan(5, 200, 12288, (16, 128, 256, 8, 3, 8, 8)) == (8, 1536, 8 * 5 * 200 * 8)
    # K = 4096 split 8 ways with BK = 256 -> KCH = 512
    assert _plan(1, 64, 4096, (16, 64, 256, 4, 3, 8, 8))[:2] == (8, 512)
    # uneven: K = 1000, SK = 3, BK = 128 -> KCH = 384, SK = 3
    assert _plan(2, 64, 1000, (16, 64, 128, 4, 3, 8, 3))[:2] == (3, 384)
    # BK below one MFMA step (64) rounds chunks up to 64
    assert _plan(2, 64, 4096, (16, 64, 32, 4, 3, 8, 8))[:2] == (8, 512)
    # a single int32 accumulator never spans more than 32768 terms
    sk, kch, _ = _plan(1, 64, 65536, (16, 64, 128, 4, 3, 8, 1))
    assert kch <= 32768 and sk * kch >= 65536
    # BK = 64 (x through LDS, weights in registers): chunks of whole 64-wide steps
    assert _plan(256, 24576, 4096, (128, 192, 64, 4, 4, 8, 1)) == (1, 4096, 0)
    assert _plan(33, 130, 1000, (64, 128, 64, 4, 3, 8, 3))[:2] == (3, 384)
    # mma (8th field) is accepted and does not change the plan
    assert _plan(24, 384, 4096, (64, 128, 128, 4, 4, 8, 2, 1)) == _plan(24, 384, 4096, (64, 128, 128, 4, 4, 8, 2, 0))


def test_plan_rejects_bad_cfgs():
    with pytest.raises(ValueError):
        nx.cfg_array((16, 64, 128, 4, 3))
    with pytest.raises(ValueError):
        _plan(1, 64, 4096, (0, 64, 128, 4, 3, 8))
    with pytest.raises(ValueError):
        _plan(-1, 64, 4096, (16, 64, 128, 4, 3, 8))


def test_paged_workspace_sizes():
    # paged_attn.py:105-108: NS = max(1, cdiv(MAX_LEN, split)); partials only when NS > 1
    assert nx.paged_workspace(64, 32, 128, 1024, 1024) == 0
    assert nx.paged_workspace(64, 32, 128, 16784, 1024) == 64 * 32 * 17 * 130 * 4
    assert nx.paged_workspace(4, 16, 256, 9000, 4096) == 4 * 16 * 3 * 258 * 4


def test_entry_points_validate_before_launching():
    L = nx.lib()
    # digitize: F outside 1..15 and negative sizes are argument errors; zero rows is a no-op
    assert L.vxa_digitize(None, nx.VXA_F32, 4, 64, 64, None, None, 64, None, None, 16, None) == nx.VXA_ERR_ARG
    assert L.vxa_digitize(None, nx.VXA_F32, -1, 64, 64, None, None, 64, None, None, 14, None) == nx.VXA_ERR_ARG
    assert L.vxa_digitize(None, nx.VXA_F32, 0, 64, 64, None, None, 64, None, None, 14, None) == nx.VXA_OK
    assert L.vxa_digitize(None, 7, 4, 64, 64, None, None, 64, None, None, 14, None) == nx.VXA_ERR_ARG
    arr, n = nx.cfg_array((16, 64, 128, 4, 3, 8, 4))
    # exact_linear: an empty output is a no-op; missing workspace for split-K is reported
    assert L.vxa_exact_linear(None, None, None, None, 64, None, None, None, None, 64, None, nx.VXA_F32, 64,
                              0, 64, 64, 14, 1, arr, n, None, 0, None) == nx.VXA_OK
    fake = 16  # never dereferenced: validation fails first
    assert L.vxa_exact_linear(fake, fake, fake, fake, 4096, fake, fake, fake, fake, 4096, fake, nx.VXA_F32, 4096,
                              16, 4096, 4096, 14, 1, arr, n, None, 0, None) == nx.VXA_ERR_WORKSPACE
    assert L.vxa_exact_linear(fake, fake, fake, fake, 4096, fake, fake, fake, fake, 4096, fake, 9, 4096,
                              16, 4096, 4096, 14, 1, arr, n, None, 0, None) == nx.VXA_ERR_ARG
    # paged decode: unsupported head size / group / split are reported as unsupported
    args = dict(q=fake, sqt=4096, sqh=128, kc=fake, skb=4096, skp=2048, skh=256, vc=fake, svb=4096, svp=2048,
                svh=256, bt=fake, sbt=8, sl=fake, scale=0.1, out=fake, od=nx.VXA_BF16, sot=4096, soh=128, n=2,
                H=32, KV=8, D=128, BS=16, max_len=1024, max_seq_len=0, split=1024, blk=64, waves=4, ws=None, wsb=0,
                st=None)

    def call(**over):
        a = dict(args, **over)
        return L.vxa_paged_decode(*a.values())

    assert call(D=96) == nx.VXA_ERR_UNSUPPORTED
    assert call(H=24, KV=8) == nx.VXA_ERR_UNSUPPORTED  # G = 3
    assert call(split=1000) == nx.VXA_ERR_UNSUPPORTED
    assert call(blk=48) == nx.VXA_ERR_UNSUPPORTED
    assert call(split=131072) == nx.VXA_ERR_UNSUPPORTED  # a segment's block-table entries must fit in LDS
    assert call(H=30, KV=8) == nx.VXA_ERR_ARG
    assert call(max_len=4096) == nx.VXA_ERR_WORKSPACE
    # a bound on the batch's lengths trims the grid to the segments it reaches (here two, whose
    # partials need a workspace); a negative bound is refused
    assert call(max_len=4096, max_seq_len=3000) == nx.VXA_ERR_WORKSPACE
    assert call(max_seq_len=-1) == nx.VXA_ERR_ARG
    assert call(n=0) == nx.VXA_OK

    # the device-count variant: the same checks, and the count pointer is required
    def call_prefix(n_live=fake, **over):
        a = list(dict(args, **over).values())
        return L.vxa_paged_decode_prefix(*a[:20], n_live, *a[20:])

    assert call_prefix(n_live=None) == nx.VXA_ERR_ARG
    assert call_prefix(D=96) == nx.VXA_ERR_UNSUPPORTED
    assert call_prefix(max_len=4096) == nx.VXA_ERR_WORKSPACE
    assert call_prefix(n=0) == nx.VXA_OK


def test_fused_entry_point_validates_before_launching():
    # vxa_exact_linear_bf16x refuses what its one launch does not cover (the op then takes the
    # two-launch path) and bad arguments, all before any launch: the pointers are never read
    L = nx.lib()
    fake = 16
    sm, sm_n = nx.cfg_array((16, 32, 128, 8, 1, 8, 1))

    def call(m=1, n=4096, k=4096, f=14, cfg=(sm, sm_n), x=fake, ldx=4096, od=nx.VXA_BF16, ldo=4096, w=fake,
             cw=fake, trunc=1):
        return L.vxa_exact_linear_bf16x(x, ldx, w, cw, fake, fake, od, ldo, m, n, k, f, trunc, cfg[0], cfg[1], None)

    assert call(f=15) == nx.VXA_ERR_UNSUPPORTED  # offset digits run 4 dots in one launch, not 3
    assert call(f=15, trunc=0, cw=None) == nx.VXA_ERR_ARG  # their epilogue needs the weight digit sums
    assert call(cfg=nx.cfg_array((64, 96, 64, 6, 6, 8, 1))) == nx.VXA_ERR_UNSUPPORTED  # not a small-M cfg
    assert call(cfg=nx.cfg_array((32, 32, 128, 8, 1, 8, 1))) == nx.VXA_ERR_UNSUPPORTED  # two row tiles
    assert call(cfg=nx.cfg_array((16, 32, 128, 8, 1, 8, 2))) == nx.VXA_ERR_UNSUPPORTED  # split-K
    assert call(x=fake + 2) == nx.VXA_ERR_UNSUPPORTED  # rows not 16-byte aligned
    assert call(ldx=4100) == nx.VXA_ERR_UNSUPPORTED
    assert call(k=0) == nx.VXA_ERR_UNSUPPORTED
    assert call(k=40000, ldx=40000) == nx.VXA_ERR_UNSUPPORTED  # two K splits (32768 per split)
    assert call(m=0) == nx.VXA_OK
    assert call(f=16) == nx.VXA_ERR_ARG
    assert call(od=9) == nx.VXA_ERR_ARG
    assert call(ldo=100) == nx.VXA_ERR_ARG
    assert call(ldx=100) == nx.VXA_ERR_ARG
    assert call(x=None) == nx.VXA_ERR_ARG
    assert call(w=fake + 8) == nx.VXA_ERR_ARG


def test_noalloc_entry_refuses_problems_beyond_its_scratch():
    """vxa_exact_linear_op_noalloc checks its scratch need on the host and returns
    VXA_ERR_TOO_LARGE before touching the device: 4096 rows of 4096 columns with a two-way
    split over 4096 outputs needs 32 MiB of digits and 256 MiB of partials."""
    L = nx.lib()
    fake = ctypes.c_void_p(0x1000)
    cfg = (ctypes.c_int32 * 7)(64, 64, 128, 4, 1, 8, 2)
    rc = L.vxa_exact_linear_op_noalloc(fake, nx.VXA_BF16, 4096, fake, fake, fake, fake, nx.VXA_BF16, 4096, 4096,
                                       4096, 4096, 14, 1, cfg, 7, None)
    assert rc == nx.VXA_ERR_TOO_LARGE
    assert b"scratch" in L.vxa_status_string(nx.VXA_ERR_TOO_LARGE)
    with pytest.raises(ValueError, match="scratch"):
        nx.check(rc, "exact_linear_op_noalloc")
    # bad arguments are still refused first
    assert L.vxa_exact_linear_op_noalloc(fake, nx.VXA_BF16, 64, fake, fake, fake, fake, nx.VXA_BF16, 64, 1, 64,
                                         64, 16, 1, cfg, 7, None) == nx.VXA_ERR_ARG


def test_noalloc_entry_checks_every_argument_before_launching():
    """A call the GEMM stage would refuse is refused before the digitize stage writes the shared
    scratch: the pointers below are never dereferenced (no GPU is needed), so a launch would
    show up as a crash or a launch error, not as VXA_ERR_ARG."""
    L = nx.lib()
    fake = 0x1000
    cfg = (ctypes.c_int32 * 7)(16, 64, 128, 4, 1, 8, 1)

    def call(x=fake, xd=nx.VXA_BF16, ldx=64, wp=fake, cw=fake, sw=fake, out=fake, od=nx.VXA_BF16, ldo=64, m=2, n=64,
             k=64, f=14, trunc=1):
        return L.vxa_exact_linear_op_noalloc(x, xd, ldx, wp, cw, sw, out, od, ldo, m, n, k, f, trunc, cfg, 7, None)

    assert call(od=9) == nx.VXA_ERR_ARG
    assert call(ldo=10) == nx.VXA_ERR_ARG
    assert call(out=None) == nx.VXA_ERR_ARG
    assert call(wp=None) == nx.VXA_ERR_ARG
    assert call(wp=fake + 8) == nx.VXA_ERR_ARG  # packed weights are read 16 bytes at a time
    assert call(sw=None) == nx.VXA_ERR_ARG
    assert call(f=15, trunc=0, cw=None) == nx.VXA_ERR_ARG
    assert call(xd=7) == nx.VXA_ERR_ARG
    assert call(ldx=10) == nx.VXA_ERR_ARG
    assert call(x=None) == nx.VXA_ERR_ARG
    assert call(m=0) == nx.VXA_OK
