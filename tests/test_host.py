"""CPU checks of the host-side mirror of the reference interface: config tables and bucket
lookup (plugin.py:27-48), the custom op's registration, enable()'s guards
(__init__.py:44-47), the CPU-tensor policy of the GPU entry points, and the torch
statements (*_torch) against the oracle."""
import json
import sys

import numpy as np
import pytest
import torch

import oracle
import vllm_exact
from helpers import make_paged, xw
from vllm_exact import kernels as K
from vllm_exact import paged_attn as P
from vllm_exact import plugin


def test_table_bucket_lookup(tmp_path):
    table = {"4096,4096": {"1": [16, 64, 128, 4, 1, 8, 4], "16": [16, 128, 128, 8, 1, 8, 2],
                           "64": [64, 64, 128, 4, 1, 8, 1, 0]}}
    path = tmp_path / "t.json"
    path.write_text(json.dumps(table))
    plugin.load_table(path)
    try:
        assert plugin._cfg(1, 4096, 4096) == (16, 64, 128, 4, 1, 8, 4)
        assert plugin._cfg(2, 4096, 4096) == (16, 128, 128, 8, 1, 8, 2)  # smallest tuned M >= M
        assert plugin._cfg(16, 4096, 4096) == (16, 128, 128, 8, 1, 8, 2)
        assert plugin._cfg(17, 4096, 4096) == (64, 64, 128, 4, 1, 8, 1, 0)
        assert plugin._cfg(300, 4096, 4096) == (64, 64, 128, 4, 1, 8, 1)  # beyond: last row, SK = 1
        assert plugin._cfg(16, 6144, 4096) == plugin.DEFAULT_CFGS[0][1]  # shape not in the table
    finally:
        plugin.load_table(None)
    assert plugin._cfg(1, 4096, 4096) == plugin.DEFAULT_CFGS[0][1]
    assert plugin._cfg(4096, 4096, 4096) == plugin.LARGE_M_CFG


def test_one_launch_marks(tmp_path):
    # a row's "one_launch" list names the tuned row counts whose calls digitize inside the GEMM
    # launch, looked up like the cfg (smallest tuned M >= M); rows without one keep M <= 4
    table = {"4096,4096": {"1": [16, 16, 128, 16, 1, 8, 1], "16": [16, 16, 128, 16, 1, 8, 1],
                           "64": [32, 32, 128, 8, 2, 8, 1], "one_launch": [16]},
             "4096,12288": {"1": [16, 16, 128, 16, 1, 8, 1], "16": [16, 16, 128, 8, 2, 8, 1]}}
    path = tmp_path / "t.json"
    path.write_text(json.dumps(table))
    plugin.load_table(path)
    try:
        assert plugin._cfg(16, 4096, 4096) == (16, 16, 128, 16, 1, 8, 1)  # the list is no M row
        assert [plugin._one_launch(m, 4096, 4096) for m in (1, 2, 16, 17, 64, 65)] == [
            False, True, True, False, False, False]
        assert [plugin._one_launch(m, 4096, 12288) for m in (1, 4, 5, 16)] == [True, True, False, False]
        assert plugin._one_launch(4, 6144, 4096) and not plugin._one_launch(5, 6144, 4096)
    finally:
        plugin.load_table(None)
    assert plugin._one_launch(4, 4096, 4096) and not plugin._one_launch(16, 4096, 4096)


def test_tuner_merge_keeps_untuned_entries():
    import importlib.util
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    spec = importlib.util.spec_from_file_location("tune_mod", root / "vllm-exact_amd" / "tune_table.py")
    tune = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(tune)
    a, b, c = [16, 16, 128, 16, 1, 8, 1], [16, 32, 128, 8, 1, 8, 1], [64, 64, 128, 4, 4, 8, 1]
    # a base row without marks meant 1-4 rows: entries not retuned keep that meaning
    old = {"1": a, "4": a, "16": a, "256": c}
    got = tune.merge_row(old, {"16": b, "one_launch": [16]}, [16])
    assert got == {"1": a, "4": a, "16": b, "256": c, "one_launch": [1, 4, 16]}
    got = tune.merge_row(got, {"1": b, "4": b, "one_launch": [4]}, [1, 4])
    assert got == {"1": b, "4": b, "16": b, "256": c, "one_launch": [4, 16]}
    # a retune without marks (plain layout) leaves the base's marks alone
    assert tune.merge_row(got, {"256": a}, [256])["one_launch"] == [4, 16]
    assert tune.merge_row({}, {"64": c, "one_launch": []}, [64]) == {"64": c, "one_launch": []}
    # a column split stays with its row until that row is retuned
    split = {"256": [768] + a}
    assert tune.merge_row({"256": c, "n_split": split}, {"16": a}, [16])["n_split"] == split
    assert "n_split" not in tune.merge_row({"256": c, "n_split": split}, {"256": a}, [256])
    assert tune.merge_row({"256": c, "n_split": split}, {"256": a, "n_split": {"256": [512] + a}},
                          [256])["n_split"] == {"256": [512] + a}
    # the split the tuner searches: the last whole round of one-per-CU K-split workgroups
    xk = (128, 192, 128, 8, 2, 8, 1)
    assert tune.whole_round_columns(256, 151936, xk, 256) == 147456  # 1584 workgroups: 6 rounds + 48
    assert tune.whole_round_columns(512, 151936, xk, 256) == 147456  # 3168: 12 rounds + 96
    assert tune.whole_round_columns(128, 151936, (128, 128, 128, 8, 2, 8, 1), 256) is None  # last round 64 % full
    assert tune.whole_round_columns(256, 24576, xk, 256) is None  # exactly one round
    assert tune.whole_round_columns(256, 151936, (16, 64, 128, 4, 1, 8, 1), 256) is None  # not K-split
    assert tune.whole_round_columns(256, 151936, xk[:6] + (2,), 256) is None  # split-K


@pytest.mark.parametrize("path", [vllm_exact.TABLES["mi355x"], vllm_exact.TABLES_F15["mi355x"]])
def test_shipped_table_is_well_formed(path):
    raw = json.loads(path.read_text())
    for nk, row in raw.items():
        n, k = map(int, nk.split(","))
        assert n > 0 and k > 0
        for m, cfg in row.items():
            if m == "one_launch":
                assert all(str(r) in row for r in cfg), (nk, cfg)  # marks name tuned rows
                continue
            if m == "n_split":
                for r, split in cfg.items():  # splits name tuned rows, at a tile boundary inside N
                    assert r in row and 0 < split[0] < n and split[0] % 16 == 0 and 7 <= len(split[1:]) <= 8
                continue
            assert int(m) > 0 and 7 <= len(cfg) <= 8
    plugin.load_table(path)
    plugin.load_table(None)
    # every entry names an instantiated kernel: x-through-LDS tiles (BK = 64) exactly, the
    # other families through the plan's nearest-instantiation rule
    xw = {(bm, bn, r, nw) for bm, bn, r, nw in K.XW_SHAPES}
    for row in raw.values():
        cfgs = [c for m, c in row.items() if m not in ("one_launch", "n_split")]
        cfgs += [split[1:] for split in row.get("n_split", {}).values()]
        for cfg in cfgs:
            if cfg[2] == 64:
                assert (cfg[0], cfg[1], cfg[4], cfg[3]) in xw, cfg


def test_column_split_lookup(tmp_path):
    """A row's "n_split" entry applies to the calls whose row count _cfg maps to that tuned
    row, and to no other; malformed entries are refused when the table loads."""
    a, b = [128, 192, 128, 8, 2, 8, 1], [64, 96, 256, 8, 2, 8, 1]
    t = {"1000,4096": {"64": a, "256": a, "n_split": {"256": [768] + b}}}
    p = tmp_path / "t.json"
    p.write_text(json.dumps(t))
    try:
        plugin.load_table(p)
        assert plugin._n_split(256, 1000, 4096) == (768, tuple(b))
        assert plugin._n_split(65, 1000, 4096) == (768, tuple(b))  # M 65 .. 256 take the 256 row
        assert plugin._n_split(64, 1000, 4096) is None
        assert plugin._n_split(257, 1000, 4096) is None  # past the table: the last row, unsplit
        assert plugin._n_split(256, 2000, 4096) is None
        assert plugin._cfg(256, 1000, 4096) == tuple(a)
        for bad in ([770] + b, [1000] + b, [768, 64, 96]):
            t["1000,4096"]["n_split"] = {"256": bad}
            p.write_text(json.dumps(t))
            with pytest.raises(ValueError, match="n_split"):
                plugin.load_table(p)
        t["1000,4096"]["n_split"] = {"128": [768] + b}  # names no tuned row
        p.write_text(json.dumps(t))
        with pytest.raises(ValueError, match="n_split"):
            plugin.load_table(p)
    finally:
        plugin.load_table(None)


def test_bench_traffic_is_tied_to_cfg_and_sources(tmp_path, monkeypatch):
    # bench.py reports roofline.traffic from the rocprofv3 FETCH/WRITE summary only when it
    # was measured with the dominant GEMM's cfg on a library built from the current sources
    import importlib.util
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    spec = importlib.util.spec_from_file_location("bench_mod", root / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    sha = bench.kernel_sources_sha16()
    assert len(sha) == 16 and sha == bench.kernel_sources_sha16()
    summary = tmp_path / "traffic.md"
    monkeypatch.setattr(bench, "TRAFFIC_SUMMARY", summary)
    cfg = (128, 192, 64, 8, 3, 8, 1)

    def write(cfg_, sha_):
        summary.write_text(f"# traffic\n\n    cfg = {list(cfg_)}\n    traffic_bytes_per_launch = 231361984\n"
                           f"    kernel_sources_sha16 = {sha_}\n")

    write(cfg, sha)
    traffic, src = bench.read_traffic(cfg)
    assert traffic == 231361984 and sha in src
    assert bench.read_traffic((1, 2, 3, 4, 5, 6, 7))[0] is None
    write(cfg, "0" * 16)
    traffic, why = bench.read_traffic(cfg)
    assert traffic is None and "other sources" in why


def test_bench_per_op_traffic_is_tied_to_sources(tmp_path, monkeypatch):
    # bench.py attaches a per-op traffic figure from the counter record only when the record
    # was measured on a library built from the current sources
    import importlib.util
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    spec = importlib.util.spec_from_file_location("bench_mod2", root / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    summary = tmp_path / "counters.md"
    monkeypatch.setattr(bench, "COUNTERS_SUMMARY", summary)

    def write(sha_):
        summary.write_text("# counters\n\n| table |\n\n"
                           f"    kernel_sources_sha16 = {sha_}\n"
                           "    traffic M:1 op:qkv cfg:[16,32,128,16,1,8,1] = 50960000\n"
                           "    traffic M:256 op:down cfg:[128,128,128,8,2,8,4] = 182931202\n")

    write(bench.kernel_sources_sha16())
    got, src = bench.read_op_traffic()
    assert got == {(1, "qkv"): (50960000, [16, 32, 128, 16, 1, 8, 1]),
                   (256, "down"): (182931202, [128, 128, 128, 8, 2, 8, 4])}
    assert bench.kernel_sources_sha16() in src
    write("0" * 16)
    got, why = bench.read_op_traffic()
    assert got == {} and "other sources" in why


def test_bench_refuses_more_than_one_gpu():
    import subprocess
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stdout


def test_custom_op_is_registered_with_fake():
    op = torch.ops.exactmm.linear
    x = torch.empty(3, 5, 64, device="meta", dtype=torch.bfloat16)
    wh = torch.empty(96, 64, device="meta", dtype=torch.int8)
    cw = torch.empty(96, device="meta", dtype=torch.int32)
    y = op(x, wh, wh, cw, cw)
    assert y.shape == (3, 5, 96) and y.dtype == torch.bfloat16


def test_gpu_entry_points_refuse_cpu_tensors():
    x, w = xw(4, 8, 128)
    with pytest.raises(ValueError, match="digitize_torch"):
        K.digitize(x, 14)
    xd, wd = K.digitize_torch(x, 14), K.digitize_torch(w, 14)
    with pytest.raises(ValueError, match="exact_linear_torch"):
        K.exact_linear(xd, wd, 14, True)
    q, kv, bt, sl = make_paged(2, 40, 16, 4, 1, 64)
    kc, vc = kv.transpose(1, 2).split(64, dim=-1)
    with pytest.raises(ValueError, match="paged_decode_torch"):
        P.paged_decode(q, kc, vc, bt, sl, 0.125, torch.empty(2, 4, 64), 2, 40)


def test_enable_guards(monkeypatch):
    monkeypatch.setattr(vllm_exact, "_ENABLED", True)
    with pytest.raises(RuntimeError, match="only be called once"):
        vllm_exact.enable(1024)
    monkeypatch.setattr(vllm_exact, "_ENABLED", False)
    monkeypatch.setitem(sys.modules, "vllm", object())
    with pytest.raises(RuntimeError, match="before importing vllm"):
        vllm_exact.enable(1024)
    monkeypatch.delitem(sys.modules, "vllm")
    with pytest.raises(ValueError, match="another GPU"):
        vllm_exact.enable(1024, cfg_table="h200")
    if not plugin.HAVE_VLLM:
        with pytest.raises(ImportError):
            vllm_exact.enable(1024)
    assert vllm_exact._ENABLED is False


@pytest.mark.parametrize("F,trunc", [(14, True), (14, False), (15, False)])
def test_torch_statements_match_oracle(F, trunc):
    x, w = xw(9, 70, 1024, seed=5)
    xd, wd = K.digitize_torch(x, F), K.digitize_torch(w, F)
    y = K.exact_linear_torch(xd, wd, F, trunc).numpy()
    want = oracle.exact_linear_c(tuple(t.numpy() for t in xd), tuple(t.numpy() for t in wd), F, trunc)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))
    assert K.digitize_weight(w.to(torch.bfloat16), F)[3].dtype == torch.int32


def test_paged_decode_torch_matches_oracle():
    q, kv, bt, sl = make_paged(3, 100, 16, 8, 2, 64, seed=4)
    kc, vc = kv.transpose(1, 2).split(64, dim=-1)
    got = P.paged_decode_torch(q, kc, vc, bt, sl, 0.125, 3).double().numpy()
    bits = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)
    want = oracle.paged_decode_c(bits(q), bits(kc), bits(vc), bt.numpy(), sl.numpy(), 0.125, 3)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6)


def test_plugin_classes_register_and_dispatch(monkeypatch):
    """The vLLM side of the plugin (plugin.py:87-133 of the reference), run on stand-in vLLM
    base classes: the config registers as "exact_int8", reports bf16/fp16 activations and
    capability 80, and hands ExactLinearMethod to every linear layer and ExactLMHeadMethod to
    the lm_head only when LMHEAD is set; other layers get None."""
    import vllm_standin as V

    registry = V.install(monkeypatch)
    lin_m, head_m, cfg_cls = plugin.define_vllm_classes()
    assert registry == {"exact_int8": cfg_cls}
    assert issubclass(lin_m, V.UnquantizedLinearMethod) and issubclass(head_m, V.UnquantizedEmbeddingMethod)
    cfg = cfg_cls.from_config({})
    assert isinstance(cfg, V.QuantizationConfig) and cfg.get_name() == "exact_int8"
    assert cfg.get_supported_act_dtypes() == [torch.bfloat16, torch.float16]
    assert cfg_cls.get_min_capability() == 80 and cfg_cls.get_config_filenames() == []

    class QKV(V.LinearBase):
        pass

    monkeypatch.setattr(plugin, "LMHEAD", True)
    assert type(cfg.get_quant_method(QKV(), "model.layers.0.qkv")) is lin_m
    assert type(cfg.get_quant_method(V.ParallelLMHead(), "lm_head")) is head_m
    assert cfg.get_quant_method(V.VocabParallelEmbedding(), "embed_tokens") is None
    monkeypatch.setattr(plugin, "LMHEAD", False)
    assert cfg.get_quant_method(V.ParallelLMHead(), "lm_head") is None
    assert type(cfg.get_quant_method(QKV(), "model.layers.0.qkv")) is lin_m
