"""Build a gfx950 tuning table for the exact plugin (the reference's scripts/tune_table.py).

    python vllm-exact_amd/tune_table.py OUT.json [--f 14] [--shapes 6144x4096,4096x4096,...]
                                                 [--ms 1,16,64,256] [--report OUT_report.json]
                                                 [--merge BASE.json]

For each weight shape (N, K) and batch bucket M, every candidate config is run, checked
bitwise against the first candidate's output (exact integer accumulation makes every
tiling give the same bits; a mismatch raises), and timed by HIP-graph replay with the
weights rotated over enough copies to stream past the 256 MB MALL: a short replay of every
candidate first, then the FINALISTS fastest in full (about 4 ms of calls per replay, 25
replays, 10 for the big lm_heads; the median counts). By default the weights
are packed at load time and x is digitized packed, as exactmm::linear runs them (--layout
plain tunes the row-major kernels instead), and the GEMM on digitized x is timed alone.
Up to 64 rows on packed weights, every cfg the one-launch digitize + GEMM
kernel takes is also timed on that path; it is chosen, and M listed in the row's
"one_launch", when it beats digitize + the best two-launch GEMM timed together. The result
is {"N,K": {"M": [BM, BN, BK, waves, stages, GM, SK], "one_launch": [M, ...]}}; with
--merge the tuned (N, K, M) entries replace those of BASE and the rest of BASE is kept. Where
the chosen K-split cfg's grid ends in a round of workgroups at most half full, the columns of
the whole rounds plus the rest under a second cfg are timed as a pair, and kept as the row's
"n_split": {M: [N1, cfg...]} when 1 % faster. OUT
is rewritten after every shape. The report also records the bf16 hipBLASLt time of the same product (torch.matmul) for
comparison.
"""
import argparse
import json
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parent))
from vllm_exact import kernels as K  # noqa: E402
from vllm_exact.graph_timing import rotations_for, time_graph  # noqa: E402

# the decode sweep's qkv and lm_head, then the reference's shapes (its scripts/tune_table.py:26)
DEFAULT_SHAPES = ("6144x4096,151936x4096,10240x4096,4096x4096,12288x4096,64x4096,24576x4096,4096x12288,"
                  "248320x4096")
SPLITS = (1, 2, 4)
ONE_LAUNCH_TUNE_ROWS = 64  # the one-launch path is timed up to this many rows
FINALISTS = 6  # candidates per path re-timed in full after the first cut
SPLIT_GAIN = 1.01  # a column split is kept when it is this much faster than one launch


def whole_round_columns(M, N, cfg, ncu):
    """N1, the columns of the last whole round of workgroups when cfg runs the K-split family
    (8 waves, one workgroup per CU) with SK = 1 and its grid ends in a round at most half full;
    None otherwise."""
    bm, bn, bk, waves, stages = cfg[:5]
    if waves != 8 or stages != 2 or bk not in (128, 256) or bm < 64 or cfg[6] != 1:
        return None
    nbm, nbn = -(-M // bm), -(-N // bn)
    rounds, rest = divmod(nbm * nbn, ncu)
    if rounds == 0 or rest == 0 or rest > ncu // 2 or (rounds * ncu) % nbm:
        return None
    n1 = rounds * ncu // nbm * bn
    return n1 if 0 < n1 < N else None


def timing_for(M, N, Kd, rot):
    """(calls per replay, replays) for one timing: about 4 ms of calls per replay, at least one
    full weight rotation, and fewer replays for calls of 200 µs or more (the big lm_heads)."""
    est_us = max(2 * N * Kd / 5e6, 6 * M * N * Kd / 2e12, 5.0)  # ~5 TB/s, ~2 POP/s
    calls = max(rot, min(20, -(-4000 // int(est_us))))
    return calls, (25 if est_us < 200 else 10)


def candidates(M, Kd):
    """Every instantiated kernel shape whose M block does not exceed max(16, next_pow2(M))
    (kernels.py:298 filters the same way; the 32-row x-through-LDS tiles are kept for every M),
    times the split-K factors."""
    out = []
    for c in K.EXACT_CFGS:
        xw32 = c[2] == 64 and c[0] == 32  # the 32-row x-through-LDS tiles also serve M <= 16
        if c[0] > max(16, 1 << max(0, (M - 1).bit_length())) and not xw32:
            continue
        if M <= 16 and c[0] >= 64 and c[4] >= 2:
            continue  # the LDS-ring kernel needs a real M tile
        for sk in SPLITS:
            if sk > 1 and Kd // sk < 256:
                continue
            out.append(tuple(c) + (sk,))
    return out


def tune_shape(N, Kd, ms, F, trunc, gen, report, packed):
    w = (torch.randn(N, Kd, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
    rot = rotations_for(2 * N * Kd)
    if packed:
        wds = [K.pack_digits(K.digitize(w, F)) for _ in range(rot)]
    else:
        wds = [K.digitize(w, F) for _ in range(rot)]
    wbs = [w.clone() for _ in range(rot)]  # bf16 copies for the hipBLASLt comparison
    ncu = torch.cuda.get_device_properties(w.device).multi_processor_count
    row, one_rows, splits = {}, [], {}
    for M in ms:
        x = torch.randn(M, Kd, device="cuda", generator=gen).to(torch.bfloat16)
        xd = K.digitize_packed(x, F) if packed else K.digitize(x, F)
        try_one = packed and M <= ONE_LAUNCH_TUNE_ROWS

        def gemm(i, cfg, xd=xd):
            if packed:
                return K.exact_linear_packed(xd, wds[i], Kd, F, trunc, cfg=cfg)
            return K.exact_linear(xd, wds[i], F, trunc, cfg=cfg)

        def two_launch(i, cfg):
            return K.exact_linear_packed(K.digitize_packed(x, F), wds[i], Kd, F, trunc, cfg=cfg)

        def one_launch(i, cfg):
            return K.exact_linear_bf16x(x, wds[i], Kd, F, trunc, cfg=cfg)

        cpr, reps = timing_for(M, N, Kd, rot)

        def timed(fn, quick=False):
            if quick:  # a first cut over every candidate: one rotation's calls, 3 replays
                return time_graph(fn, rot, calls_per_replay=max(rot, 2), replays=3)
            return time_graph(fn, rot, calls_per_replay=cpr, replays=reps)

        ref, tried, tried_one = None, [], []

        def check(y, cfg):
            nonlocal ref
            if ref is None:
                ref = y
            elif not torch.equal(y.view(torch.int32), ref.view(torch.int32)):
                raise RuntimeError(f"config {cfg} changed the result (N={N} K={Kd} M={M})")

        for cfg in candidates(M, Kd):
            try:
                y = gemm(0, cfg)
            except NotImplementedError:
                continue
            check(y, cfg)
            tried.append((timed(lambda i, c=cfg: gemm(i, c), quick=True), cfg))
            if try_one:
                try:
                    y = one_launch(0, cfg)
                except NotImplementedError:
                    pass
                else:
                    check(y, cfg)
                    tried_one.append((timed(lambda i, c=cfg: one_launch(i, c), quick=True), cfg))
            if len(tried) % 40 == 0:
                print(f"  N={N} K={Kd} M={M}: {len(tried)} configs timed", file=sys.stderr, flush=True)
        n_cand = len(tried)
        # the finalists of the first cut, timed in full
        tried = sorted((timed(lambda i, c=c: gemm(i, c)), c) for _, c in sorted(tried)[:FINALISTS])
        tried_one = sorted((timed(lambda i, c=c: one_launch(i, c)), c) for _, c in sorted(tried_one)[:FINALISTS])
        best = min(tried)
        rec = dict(N=N, K=Kd, M=M, exact_us=round(best[0], 2), cfg=list(best[1]), candidates=n_cand)
        if tried_one:
            # what the op would run either way: digitize + the best GEMM, or the one launch
            t_two = timed(lambda i: two_launch(i, best[1]))
            best_one = min(tried_one)
            rec.update(two_launch_op_us=round(t_two, 2), one_launch_us=round(best_one[0], 2),
                       one_launch_cfg=list(best_one[1]), one_launch=best_one[0] < t_two)
            if best_one[0] < t_two:
                best = best_one
                one_rows.append(M)
        n1 = whole_round_columns(M, N, best[1], ncu) if packed and not rec.get("one_launch") else None
        if n1 is not None:
            # the whole rounds with the chosen cfg, the rest of the columns with a grid of its own
            # (the remainder's candidates cut on the remainder alone, then timed as the pair)
            out = torch.empty(M, N, device="cuda", dtype=torch.float32)

            def part(i, n0, n_end, cfg, xd=xd, out=out):
                pw, cw, sw = wds[i]
                return K.exact_linear_packed(xd, (pw[n0 // 16:(n_end + 15) // 16], cw[n0:n_end], sw[n0:n_end]),
                                             Kd, F, trunc, out=out[:, n0:n_end], cfg=cfg)

            rest = []
            for cfg in candidates(M, Kd):
                if cfg[6] != 1:
                    continue
                try:
                    part(0, n1, N, cfg)
                except NotImplementedError:
                    continue
                rest.append((timed(lambda i, c=cfg: part(i, n1, N, c), quick=True), cfg))
            pairs = []
            for _, cfg2 in sorted(rest)[:3]:
                part(0, 0, n1, best[1])
                part(0, n1, N, cfg2)
                check(out.clone(), (best[1], n1, cfg2))
                pairs.append((timed(lambda i, c=cfg2: (part(i, 0, n1, best[1]), part(i, n1, N, c))), cfg2))
            if pairs and min(pairs)[0] * SPLIT_GAIN < best[0]:
                splits[str(M)] = [n1] + list(min(pairs)[1])
                rec.update(n_split=splits[str(M)], split_us=round(min(pairs)[0], 2))
        t_bf16 = timed(lambda i: torch.matmul(x, wbs[i].T))
        row[str(M)] = list(best[1])
        rec.update(bf16_hipblaslt_us=round(t_bf16, 2), chosen=list(best[1]))
        print(json.dumps(rec), flush=True)
        rec["finalists"] = [[round(t, 2), list(c)] for t, c in tried]
        rec["finalists_one_launch"] = [[round(t, 2), list(c)] for t, c in tried_one]
        report.append(rec)
    if packed:
        row["one_launch"] = one_rows
    if splits:
        row["n_split"] = splits
    del wds, wbs
    torch.cuda.empty_cache()
    return row


def merge_row(old, new, ms):
    """Row `old` with the tuned entries of `new` (at the row counts `ms`) put in. A row without
    a "one_launch" list follows the op's default (1-4 rows); merged, it keeps that meaning for
    the entries that were not retuned."""
    cfgs = {m: c for m, c in old.items() if m not in ("one_launch", "n_split")}
    cfgs.update({m: c for m, c in new.items() if m not in ("one_launch", "n_split")})
    out = dict(sorted(cfgs.items(), key=lambda t: int(t[0])))
    if "one_launch" in new:
        if "one_launch" in old:
            kept = [m for m in old["one_launch"] if m not in ms]
        else:
            kept = [int(m) for m in old if int(m) <= K.ONE_LAUNCH_MAX_ROWS and int(m) not in ms]
        out["one_launch"] = sorted(set(kept) | set(new["one_launch"]))
    elif "one_launch" in old:
        out["one_launch"] = old["one_launch"]
    # column splits are measured against their row's cfg: a retuned row takes the new result
    split = {m: v for m, v in old.get("n_split", {}).items() if int(m) not in ms}
    split.update(new.get("n_split", {}))
    if split:
        out["n_split"] = split
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("out")
    ap.add_argument("--f", type=int, default=14)
    ap.add_argument("--shapes", default=DEFAULT_SHAPES)
    ap.add_argument("--ms", default="1,2,4,8,16,24,32,48,64,96,128,192,256")
    ap.add_argument("--report", default=None)
    ap.add_argument("--merge", default=None, help="existing table whose untuned entries are kept")
    ap.add_argument("--layout", default="packed", choices=["packed", "plain"],
                    help="packed: weights packed at load (the exactmm::linear path); plain: row-major digits")
    args = ap.parse_args()
    F, trunc = args.f, args.f == 14
    shapes = [tuple(map(int, s.split("x"))) for s in args.shapes.split(",")]
    ms = [int(m) for m in args.ms.split(",")]
    gen = torch.Generator(device="cuda").manual_seed(0)
    table = json.loads(Path(args.merge).read_text()) if args.merge else {}
    report = []
    for N, Kd in shapes:
        new = tune_shape(N, Kd, ms, F, trunc, gen, report, args.layout == "packed")
        table[f"{N},{Kd}"] = merge_row(table.get(f"{N},{Kd}", {}), new, ms)
        Path(args.out).write_text(json.dumps(table, indent=1))  # after every shape
    Path(args.out).write_text(json.dumps(table, indent=1))
    rep = args.report or args.out.replace(".json", "_report.json")
    Path(rep).write_text(json.dumps(report, indent=1))


if __name__ == "__main__":
    main()
