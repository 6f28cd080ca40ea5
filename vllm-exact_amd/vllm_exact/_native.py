"""ctypes binding of libvllm_exact_amd.so, the gfx950 HIP library behind this package.

The library exposes a plain C ABI (include/vllm_exact_amd.h): device pointers, 64-bit sizes
and strides, dtype enums, a hipStream_t, an int status. This module loads it, declares the
argument types, and turns status codes into Python exceptions:

* VXA_ERR_ARG         -> ValueError
* VXA_ERR_UNSUPPORTED -> NotImplementedError (autotune and tuners skip such configs, as the
                         reference skips configs that fail, kernels.py:313-314)
* VXA_ERR_TOO_LARGE   -> ValueError (a problem beyond vxa_exact_linear_op_noalloc's fixed scratch)
* VXA_ERR_WORKSPACE / VXA_ERR_LAUNCH -> RuntimeError

There is no fallback: if the library is missing, every GPU entry point raises.
"""
import ctypes
from pathlib import Path

import torch  # loads torch's HIP runtime first, so the library binds to that same runtime

LIB_NAME = "libvllm_exact_amd.so"
LIB_PATH = Path(__file__).with_name(LIB_NAME)

VXA_OK, VXA_ERR_ARG, VXA_ERR_UNSUPPORTED, VXA_ERR_WORKSPACE, VXA_ERR_LAUNCH, VXA_ERR_TOO_LARGE = range(6)
NOALLOC_SCRATCH_BYTES = 64 << 20  # VXA_NOALLOC_SCRATCH_BYTES
VXA_F32, VXA_BF16, VXA_F16 = 0, 1, 2

DTYPE_ENUM = {torch.float32: VXA_F32, torch.bfloat16: VXA_BF16, torch.float16: VXA_F16}

# Every symbol include/vllm_exact_amd.h declares.
EXPORTED = (
    "vxa_version",
    "vxa_status_string",
    "vxa_digitize",
    "vxa_exact_linear_plan",
    "vxa_exact_linear",
    "vxa_packed_bytes",
    "vxa_pack_digits",
    "vxa_digitize_packed",
    "vxa_exact_linear_packed",
    "vxa_exact_linear_bf16x",
    "vxa_paged_decode_workspace",
    "vxa_paged_decode",
    "vxa_paged_decode_prefix",
    "vxa_exact_linear_op_noalloc",
)

_i64, _i32, _int, _vp, _sz = ctypes.c_int64, ctypes.c_int32, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t
_SIGNATURES = {
    "vxa_version": (ctypes.c_char_p, []),
    "vxa_status_string": (ctypes.c_char_p, [_int]),
    "vxa_digitize": (_int, [_vp, _int, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _int, _vp]),
    "vxa_exact_linear_plan": (
        _int,
        [_i64, _i64, _i64, ctypes.POINTER(_i32), _int, ctypes.POINTER(_i32), ctypes.POINTER(_i64),
         ctypes.POINTER(_sz)],
    ),
    "vxa_exact_linear": (
        _int,
        [_vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _i64, _vp, _int, _i64, _i64, _i64, _i64, _int, _int,
         ctypes.POINTER(_i32), _int, _vp, _sz, _vp],
    ),
    "vxa_packed_bytes": (_sz, [_i64, _i64]),
    "vxa_pack_digits": (_int, [_vp, _vp, _i64, _i64, _i64, _vp, _vp]),
    "vxa_digitize_packed": (_int, [_vp, _int, _i64, _i64, _i64, _vp, _vp, _vp, _int, _vp]),
    "vxa_exact_linear_packed": (
        _int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _int, _int, ctypes.POINTER(_i32), _int,
         _vp, _sz, _vp],
    ),
    "vxa_exact_linear_bf16x": (
        _int,
        [_vp, _i64, _vp, _vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _int, _int, ctypes.POINTER(_i32), _int, _vp],
    ),
    "vxa_paged_decode_workspace": (_int, [_i64, _i64, _i64, _i64, _i64, ctypes.POINTER(_sz)]),
    "vxa_exact_linear_op_noalloc": (
        _int,
        [_vp, _int, _i64, _vp, _vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _int, _int, ctypes.POINTER(_i32), _int,
         _vp],
    ),
    "vxa_paged_decode": (
        _int,
        [_vp, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _vp, ctypes.c_float, _vp,
         _int, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _sz, _vp],
    ),
    "vxa_paged_decode_prefix": (
        _int,
        [_vp, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _vp, ctypes.c_float, _vp,
         _int, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _sz, _vp],
    ),
}

_lib = None
_load_error = None


def _load():
    global _lib, _load_error
    if _lib is not None or _load_error is not None:
        return _lib
    try:
        if not LIB_PATH.exists():
            raise OSError(f"{LIB_PATH} does not exist")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    except OSError as e:  # not built, or built for another ABI
        _load_error = e
    return _lib


def available():
    """True when the HIP library is built and loadable (it does not need a GPU to load)."""
    return _load() is not None


def lib():
    """The loaded library; raises RuntimeError when it is missing (no silent fallback)."""
    L = _load()
    if L is None:
        raise RuntimeError(
            f"vllm_exact: the HIP library {LIB_NAME} is not available ({_load_error}). "
            "Build it with `make -C vllm-exact_amd` (gfx950).")
    return L


def check(status, what):
    if status == VXA_OK:
        return
    msg = f"{what}: {lib().vxa_status_string(status).decode()} (status {status})"
    if status in (VXA_ERR_ARG, VXA_ERR_TOO_LARGE):
        raise ValueError(msg)
    if status == VXA_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


def version():
    return lib().vxa_version().decode()


def stream_handle(device):
    """hipStream_t of torch's current stream on `device`, as an integer."""
    return torch.cuda.current_stream(device).cuda_stream


def dtype_enum(dtype):
    try:
        return DTYPE_ENUM[dtype]
    except KeyError:
        raise ValueError(f"unsupported floating dtype {dtype}") from None


def ptr(t):
    return None if t is None else t.data_ptr()


def cfg_array(cfg):
    cfg = tuple(int(c) for c in cfg)
    if not 6 <= len(cfg) <= 8:
        raise ValueError(f"cfg must have 6 to 8 entries (BM, BN, BK, warps, stages, GM[, SK[, mma]]), got {cfg}")
    return (_i32 * len(cfg))(*cfg), len(cfg)


def exact_plan(M, N, K, cfg):
    """(sk, kch, ws_bytes) for one exact_linear call (the split-K arithmetic of kernels.py:271-273)."""
    arr, n = cfg_array(cfg)
    sk, kch, ws = _i32(), _i64(), _sz()
    check(lib().vxa_exact_linear_plan(M, N, K, arr, n, ctypes.byref(sk), ctypes.byref(kch), ctypes.byref(ws)),
          "exact_linear_plan")
    return sk.value, kch.value, ws.value


def paged_workspace(n, H, D, max_len, split):
    ws = _sz()
    check(lib().vxa_paged_decode_workspace(n, H, D, max_len, split, ctypes.byref(ws)), "paged_decode_workspace")
    return ws.value
