"""The probe library behind `bench.py --floors` (vllm-exact_amd/floors/floors.hip): it loads,
exports its nine probes, and refuses malformed arguments before launching anything (no GPU
needed: every refusal happens on the host)."""
import ctypes
from pathlib import Path

import pytest

LIB = Path(__file__).resolve().parents[1] / "vllm-exact_amd" / "vllm_exact" / "libvxa_floors.so"
pytestmark = pytest.mark.skipif(not LIB.exists(), reason="floors library not built (make -C vllm-exact_amd)")

vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
SIGS = {
    "vxf_stream": [vp, i64, i64, i32, i32, i32, i32, vp, vp, vp],
    "vxf_pages": [vp, i64, vp, i32, i32, i32, i32, vp, vp, vp],
    "vxf_wave_pages": [vp, i64, vp, i32, i32, i32, i32, vp, vp, vp],
    "vxf_l2": [vp, i64, i32, i32, i32, i32, i32, vp, vp, vp],
    "vxf_lds": [i32, i32, i32, vp, vp, vp],
    "vxf_mfma": [i32, i32, i32, vp, vp, vp],
    "vxf_mfma_mix": [vp, i64, vp, i64, i32, i32, i32, i32, i32, vp, vp, vp],
    "vxf_mfma_shape": [i32, i32, i32, i32, vp, vp, vp],
    "vxf_rowcopy": [vp, i64, i64, i64, vp, i64, vp],
}


@pytest.fixture(scope="module")
def lib():
    L = ctypes.CDLL(str(LIB))
    for name, args in SIGS.items():
        getattr(L, name).argtypes = args
        getattr(L, name).restype = i32
    return L


def test_exports_every_probe(lib):
    for name in SIGS:
        assert hasattr(lib, name), name


def test_probes_refuse_malformed_arguments(lib):
    p = 16  # never dereferenced: every call below is refused on the host
    # stream: per-workgroup bytes not a multiple of 16 * threads; more bytes than the buffer;
    # an unsupported depth or thread count
    assert lib.vxf_stream(p, 1 << 20, 100, 4, 256, 4, 1, p, p, None) == 1
    assert lib.vxf_stream(p, 1 << 20, 1 << 20, 4, 256, 4, 1, p, p, None) == 1
    assert lib.vxf_stream(p, 1 << 20, 4096, 4, 256, 3, 0, p, p, None) == 1
    assert lib.vxf_stream(p, 1 << 20, 4096, 4, 128, 4, 0, p, p, None) == 1
    # pages: unsupported depth, a page count per workgroup not divisible by it, no buffer
    assert lib.vxf_pages(p, 1 << 20, p, 4, 8, 3, 1, p, p, None) == 1
    assert lib.vxf_pages(p, 1 << 20, p, 4, 3, 2, 1, p, p, None) == 1
    assert lib.vxf_pages(None, 1 << 20, p, 4, 8, 2, 1, p, p, None) == 1
    # wave pages: LDS padding outside 1 KiB .. 64 KiB, empty grid
    assert lib.vxf_wave_pages(p, 1 << 20, p, 4, 8, 1, 100, p, p, None) == 1
    assert lib.vxf_wave_pages(p, 1 << 20, p, 4, 8, 1, 1 << 17, p, p, None) == 1
    assert lib.vxf_wave_pages(p, 1 << 20, p, 0, 8, 1, 0, p, p, None) == 1
    # l2: buffer not a power of two, unsupported wave count
    assert lib.vxf_l2(p, 3 << 20, 0, 4, 4, 1, 1, p, p, None) == 1
    assert lib.vxf_l2(p, 1 << 21, 0, 4, 5, 1, 1, p, p, None) == 1
    # mfma_mix: neither loads nor MFMAs, an MFMA count not a multiple of 8, no clock buffer, HBM
    # loads without a buffer or with less than 8 KiB per workgroup, an unknown operand mode
    assert lib.vxf_mfma_mix(p, 1 << 21, p, 1 << 30, 0, 0, 0, 1, 1, p, p, None) == 1
    assert lib.vxf_mfma_mix(p, 1 << 21, p, 1 << 30, 1, 12, 0, 1, 1, p, p, None) == 1
    assert lib.vxf_mfma_mix(p, 1 << 21, p, 1 << 30, 1, 56, 0, 1, 1, p, None, None) == 1
    assert lib.vxf_mfma_mix(p, 1 << 21, None, 1 << 30, 2, 56, 0, 1, 1, p, p, None) == 1
    assert lib.vxf_mfma_mix(p, 1 << 21, p, 4096, 2, 56, 0, 1, 1, p, p, None) == 1
    assert lib.vxf_mfma_mix(p, 1 << 21, p, 1 << 30, 1, 56, 2, 1, 1, p, p, None) == 1
    # mfma_shape: an unknown shape or operand mode, an odd round count, no clock buffer
    assert lib.vxf_mfma_shape(24, 0, 1, 2, p, p, None) == 1
    assert lib.vxf_mfma_shape(16, 2, 1, 2, p, p, None) == 1
    assert lib.vxf_mfma_shape(32, 1, 1, 3, p, p, None) == 1
    assert lib.vxf_mfma_shape(16, 1, 1, 2, p, None, None) == 1
    # rowcopy: rows not a multiple of 16, K not a multiple of 64 or past 16384, buffers too small
    assert lib.vxf_rowcopy(p, 1 << 30, 17, 4096, p, 1 << 30, None) == 1
    assert lib.vxf_rowcopy(p, 1 << 30, 16, 4100, p, 1 << 30, None) == 1
    assert lib.vxf_rowcopy(p, 1 << 30, 16, 32768, p, 1 << 30, None) == 1
    assert lib.vxf_rowcopy(p, 1000, 16, 4096, p, 1 << 30, None) == 1
    assert lib.vxf_rowcopy(p, 1 << 30, 16, 4096, p, 1000, None) == 1
