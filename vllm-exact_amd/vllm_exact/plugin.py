"""vLLM quantization plugin quantization="exact_int8" (plugin.py of the reference).

Every linear layer (optionally lm_head) goes through the exact two-digit matmul. The
pieces that do not need vLLM (tuning-table lookup, the `exactmm::linear` custom op, weight
digitization) are always defined; the vLLM classes are defined when vLLM is importable.
Globals F, TRUNC, LMHEAD, RB are set by vllm_exact.enable().
"""
import json
from pathlib import Path

import torch

from . import kernels as K

# set by enable()
F = 14
TRUNC = True
LMHEAD = True
RELEASE_WEIGHTS = False  # free each linear layer's bf16 weight once its digits are packed
_TABLE = None
RB = 16384  # rows per block: rows are independent, so blocking bounds temporaries without changing bits
WEIGHT_RB = 32768  # weight rows digitized per block at load time (plugin.py:74)


_ONE_LAUNCH_ROWS = {}  # (N, K) -> tuned row counts whose calls digitize inside the GEMM launch
_N_SPLIT = {}  # (N, K) -> {tuned row count: (N1, cfg of columns N1..N)}


def load_table(path):
    """Tuning table {"N,K": {"M": [BM, BN, BK, warps, stages, GM, SK(, mma)]}} (plugin.py:27-34).
    Configs change speed only, never results. A row may also hold "one_launch": [M, ...], the
    tuned row counts at which the op digitizes inside the GEMM launch (see _one_launch), and
    "n_split": {"M": [N1, BM, BN, ...]}, the tuned row counts at which the GEMM runs as two
    launches over columns [0, N1) and [N1, N), the second with its own cfg (see _n_split)."""
    global _TABLE
    _ONE_LAUNCH_ROWS.clear()
    _ONE_LAUNCH_CFG.clear()
    _N_SPLIT.clear()
    if path is None:
        _TABLE = None
        return
    raw = json.loads(Path(path).read_text())
    _TABLE = {}
    for nk, row in raw.items():
        key = tuple(int(v) for v in nk.split(","))
        _TABLE[key] = {int(m): tuple(c) for m, c in row.items() if m not in ("one_launch", "n_split")}
        if "one_launch" in row:
            _ONE_LAUNCH_ROWS[key] = frozenset(int(m) for m in row["one_launch"])
        if "n_split" in row:
            split = {}
            for m, v in row["n_split"].items():
                n1, cfg2 = int(v[0]), tuple(v[1:])
                if int(m) not in _TABLE[key] or n1 <= 0 or n1 % 16 or n1 >= key[0] or len(cfg2) < 6:
                    raise ValueError(f"load_table: bad n_split entry {m}: {v} for shape {nk}")
                split[int(m)] = (n1, cfg2)
            _N_SPLIT[key] = split


# Built-in gfx950 configs when a shape has no table entry (speed only).
DEFAULT_CFGS = ((16, (16, 64, 128, 8, 1, 8, 1)), (32, (32, 64, 128, 8, 1, 8, 1)), (64, (64, 64, 128, 4, 1, 8, 1)))
LARGE_M_CFG = (64, 64, 128, 4, 1, 8, 1)


def _cfg(M, N, Kd):
    """Config for an (M, N, K) call: the table row of the smallest tuned M >= M; beyond the
    largest tuned M the largest row with SK = 1; otherwise a built-in (plugin.py:37-48)."""
    if _TABLE is not None and (N, Kd) in _TABLE:
        row = _TABLE[(N, Kd)]
        ms = sorted(row)
        if M > ms[-1]:
            return tuple(row[ms[-1]][:6]) + (1,)
        return row[next(m for m in ms if m >= M)]
    for bound, cfg in DEFAULT_CFGS:
        if M <= bound:
            return cfg
    return LARGE_M_CFG


def _one_launch(M, N, Kd):
    """Whether an (M, N, K) call takes the one-launch digitize + GEMM path: as the table row
    that _cfg picks says when the shape's row has a "one_launch" list, else M <= 4
    (K.ONE_LAUNCH_MAX_ROWS). Either way the bits are those of the two-launch path."""
    if _TABLE is not None and (N, Kd) in _ONE_LAUNCH_ROWS:
        ms = sorted(_TABLE[(N, Kd)])
        if M > ms[-1]:
            return False
        return next(m for m in ms if m >= M) in _ONE_LAUNCH_ROWS[(N, Kd)]
    return M <= K.ONE_LAUNCH_MAX_ROWS


def _n_split(M, N, Kd):
    """(N1, cfg2) when the table row that _cfg picks for an (M, N, K) call splits its columns:
    the GEMM then runs over columns [0, N1) with _cfg's config and over [N1, N) with cfg2, on the
    same digits of x. N1 ends the last whole round of workgroups of the first config (one per CU),
    so the last, partly filled round runs with a grid of its own. Integer sums do not depend on
    the tiling: the bits are those of one launch. None otherwise."""
    if _TABLE is None or (N, Kd) not in _N_SPLIT:
        return None
    ms = sorted(_TABLE[(N, Kd)])
    if M > ms[-1]:
        return None
    return _N_SPLIT[(N, Kd)].get(next(m for m in ms if m >= M))


# (F, trunc, cfg, N, K[, M at F = 15]) the one-launch digitize + GEMM path refused. At F < 15
# a refusal depends on the cfg and K (a K past 32768 columns needs a second K split); at F = 15
# also on the grid, hence the row count. Cleared by load_table.
_ONE_LAUNCH_CFG = {}


def _one_launch_key(cfg, M, N, Kd):
    return (F, TRUNC, tuple(cfg), N, Kd) + ((M,) if F == 15 else ())


@torch.library.custom_op("exactmm::linear", mutates_args=())
def exact_linear_op(x: torch.Tensor, wh: torch.Tensor, wl: torch.Tensor, cw: torch.Tensor,
                    sw: torch.Tensor) -> torch.Tensor:
    """y = x @ W^T through the exact path: reshape to 2-D, digitize x (bf16 read directly),
    exact matmul straight into an x.dtype output, in row blocks of RB (plugin.py:51-64). With
    packed weights, bf16 rows, a one-row-tile cfg and a row count the table marks (1-4 rows
    without a mark), digitize and GEMM share one launch (same bits).

    Weights come either as the reference's row-major digit planes wh, wl [N, K], or packed
    at load time (wh = packed [cdiv(N,16), cdiv(K,64), 2, 1024], wl empty); N is sw's length
    either way, and both give the same bits."""
    shp = x.shape
    N = sw.shape[0]
    x2 = x.reshape(-1, shp[-1])
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    M, Kd = x2.shape
    out = x.new_empty(M, N)
    packed = wh.dim() == 4
    for i in range(0, M, RB):
        xb = x2[i:i + RB]
        cfg = _cfg(xb.shape[0], N, Kd)
        if packed:
            key = _one_launch_key(cfg, xb.shape[0], N, Kd)
            if (xb.dtype == torch.bfloat16 and _one_launch(xb.shape[0], N, Kd)
                    and _ONE_LAUNCH_CFG.get(key, True)):
                # digitize inside the GEMM launch where the cfg allows it (same bits, one launch fewer)
                try:
                    K.exact_linear_bf16x(xb, (wh, cw, sw), Kd, F, TRUNC, out=out[i:i + RB], cfg=cfg)
                    continue
                except NotImplementedError:
                    if K.bf16x_rows_aligned(xb):
                        _ONE_LAUNCH_CFG[key] = False  # refused for the cfg (and shape), not for this x
            xd = K.digitize_packed(xb, F)
            split = _n_split(xb.shape[0], N, Kd)
            if split is None:
                K.exact_linear_packed(xd, (wh, cw, sw), Kd, F, TRUNC, out=out[i:i + RB], cfg=cfg)
            else:
                # the whole rounds of workgroups, then the rest of the columns with a grid of its own
                n1, cfg2 = split
                ob = out[i:i + RB]
                K.exact_linear_packed(xd, (wh[:n1 // 16], cw[:n1], sw[:n1]), Kd, F, TRUNC, out=ob[:, :n1], cfg=cfg)
                K.exact_linear_packed(xd, (wh[n1 // 16:], cw[n1:], sw[n1:]), Kd, F, TRUNC, out=ob[:, n1:], cfg=cfg2)
        else:
            K.exact_linear(K.digitize(xb, F), (wh, wl, cw, sw), F, TRUNC, out=out[i:i + RB], cfg=cfg)
    return out.reshape(*shp[:-1], N)


@exact_linear_op.register_fake
def _(x, wh, wl, cw, sw):
    return x.new_empty(*x.shape[:-1], sw.shape[0])


def digitize_weight_rows(w):
    """Digitize a weight matrix on the GPU in row blocks (plugin.py:72-79): row-major digits."""
    parts = [K.digitize(w[i:i + WEIGHT_RB].float().contiguous(), F) for i in range(0, w.shape[0], WEIGHT_RB)]
    return tuple(torch.cat([p[j] for p in parts]).contiguous() for j in range(4))


def pack_weight(w):
    """Digitize and pack a weight matrix: (packed, empty, cw, sw), the buffers the op takes.
    Row blocks of WEIGHT_RB keep the fp32 temporaries bounded (a multiple of 16 rows, so
    blocks pack independently)."""
    N, Kd = w.shape
    packed = torch.empty(K.packed_shape(N, Kd), dtype=torch.int8, device=w.device)
    cw = torch.empty(N, dtype=torch.int32, device=w.device)
    sw = torch.empty(N, dtype=torch.int32, device=w.device)
    for i in range(0, N, WEIGHT_RB):
        rows = min(WEIGHT_RB, N - i)
        src = w[i:i + rows]
        if src.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            src = src.float()  # bf16/fp16/fp32 are read directly: same digits as their fp32 value
        K.digitize_packed(src, F, out=(packed[i // 16:(i + rows + 15) // 16], cw[i:i + rows], sw[i:i + rows]))
    return packed, torch.empty(0, dtype=torch.int8, device=w.device), cw, sw


def _digitize_layer(layer, release=False):
    """Register the packed digits of layer.weight as buffers (plugin.py:72-79). With release,
    the bf16 weight's memory is freed afterwards: the Parameter stays (same dtype and device,
    no elements), so nothing that only checks for it breaks, but the op never reads it."""
    ph, pl, cs, sh = pack_weight(layer.weight.data)
    layer.register_buffer("ex_wh", ph, persistent=False)
    layer.register_buffer("ex_wl", pl, persistent=False)
    layer.register_buffer("ex_cw", cs, persistent=False)
    layer.register_buffer("ex_sw", sh, persistent=False)
    if release:
        layer.weight.data = layer.weight.data.new_empty(0)


def _apply(layer, x, bias):
    y = torch.ops.exactmm.linear(x, layer.ex_wh, layer.ex_wl, layer.ex_cw, layer.ex_sw)
    return y if bias is None else y + bias


def define_vllm_classes():
    """Define ExactLinearMethod, ExactLMHeadMethod and ExactInt8Config on vLLM's own base
    classes and register the config as quantization="exact_int8" (plugin.py:87-133). Runs at
    import when vLLM is importable (ImportError otherwise); returns the three classes."""
    from vllm.model_executor.layers.linear import LinearBase, UnquantizedLinearMethod
    from vllm.model_executor.layers.quantization import register_quantization_config
    from vllm.model_executor.layers.quantization.base_config import QuantizationConfig
    from vllm.model_executor.layers.vocab_parallel_embedding import ParallelLMHead, UnquantizedEmbeddingMethod

    class ExactLinearMethod(UnquantizedLinearMethod):
        """Every linear layer: weights digitized and packed once loaded, the product through
        the exactmm::linear op (plugin.py:87-93)."""

        def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
            _digitize_layer(layer, release=RELEASE_WEIGHTS)

        def apply(self, layer, x, bias=None):
            return _apply(layer, x, bias)

    class ExactLMHeadMethod(UnquantizedEmbeddingMethod):
        """lm_head through the exact linear layer; the embedding lookup is unchanged. Its bf16
        weight is always kept: a tied lm_head shares it with the embedding (plugin.py:96-102)."""

        def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
            _digitize_layer(layer)

        def apply(self, layer, x, bias=None):
            return _apply(layer, x, bias)

    @register_quantization_config("exact_int8")
    class ExactInt8Config(QuantizationConfig):
        def __init__(self):
            super().__init__()

        def get_name(self):
            return "exact_int8"

        def get_supported_act_dtypes(self):
            return [torch.bfloat16, torch.float16]

        @classmethod
        def get_min_capability(cls):
            return 80

        @staticmethod
        def get_config_filenames():
            return []

        @classmethod
        def from_config(cls, config):
            return cls()

        def get_quant_method(self, layer, prefix):
            if isinstance(layer, LinearBase):
                return ExactLinearMethod()
            if LMHEAD and isinstance(layer, ParallelLMHead):
                return ExactLMHeadMethod()
            return None

    return ExactLinearMethod, ExactLMHeadMethod, ExactInt8Config


try:  # vLLM is the host engine; the op and the helpers above do not need it
    ExactLinearMethod, ExactLMHeadMethod, ExactInt8Config = define_vllm_classes()
    HAVE_VLLM = True
except ImportError:
    HAVE_VLLM = False
