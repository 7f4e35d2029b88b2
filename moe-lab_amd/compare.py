"""A/B of two variants with launch-level replication and a 95% CI on the speedup (reference
moelab/compare.py:1-140, on torch-ROCm).

Each launch is its own process (its own weights, inputs and routing windows, seed = seed_base + launch) that
times A and B in interleaved rounds (A first on even rounds, B first on odd ones) with the chained timing of
backend.time_chained, and brackets itself with guard probes. The parent pools every launch's rounds:
    speedup = median(A_us) / median(B_us)          (B is speedup x faster than A)
    CI      = percentiles 2.5 / 97.5 of that ratio over a two-stage bootstrap: draw launches with
              replacement, then rounds with replacement inside each drawn launch (rounds of one launch share
              its routing windows, so resampling rounds alone understates the spread)
and reports the rounds-only bootstrap beside it.

    python moe-lab_amd/compare.py A.py B.py --shape qwen3-30b-a3b --tokens 1 8 32 --launches 5 --rounds 6
"""
import argparse
import json
import os
import subprocess
import sys

import numpy as np


def ratio_of_medians(a, b):
    return float(np.median(a) / np.median(b))


def boot_ci(a_us, b_us, n=4000, seed=0):
    """(point, lo, hi): the speedup and its 95% interval from resampling rounds (paired) with replacement."""
    a_us, b_us = np.asarray(a_us, float), np.asarray(b_us, float)
    rng = np.random.default_rng(seed)
    draws = rng.integers(0, a_us.size, size=(n, a_us.size))
    r = np.median(a_us[draws], axis=1) / np.median(b_us[draws], axis=1)
    lo, hi = np.percentile(r, [2.5, 97.5])
    return ratio_of_medians(a_us, b_us), float(lo), float(hi)


def hier_samples(rows, n=4000, seed=0):
    """n bootstrap replicates of the speedup: draw launches with replacement, then each drawn launch's rounds
    with replacement (rounds stay paired: A and B of one round travel together)."""
    launches = sorted({r["launch"] for r in rows})
    a = [np.asarray([r["A_us"] for r in rows if r["launch"] == L], float) for L in launches]
    b = [np.asarray([r["B_us"] for r in rows if r["launch"] == L], float) for L in launches]
    sizes = np.array([v.size for v in a])
    flat_a, flat_b = np.concatenate(a), np.concatenate(b)
    start = np.concatenate([[0], np.cumsum(sizes)[:-1]])
    rng = np.random.default_rng(seed)
    out = np.empty(n)
    for i in range(n):
        pick = rng.integers(0, len(launches), len(launches))
        idx = np.concatenate([start[g] + rng.integers(0, sizes[g], sizes[g]) for g in pick])
        out[i] = np.median(flat_a[idx]) / np.median(flat_b[idx])
    return out


def boot_ci_hier(rows, n=4000, seed=0):
    """(lo, hi): 95% interval of the speedup from the two-stage bootstrap (hier_samples)."""
    lo, hi = np.percentile(hier_samples(rows, n, seed), [2.5, 97.5])
    return float(lo), float(hi)


def summarize(rows, tokens):
    summary = []
    for T in tokens:
        rs = [r for r in rows if r["T"] == T]
        if not rs:
            continue
        sp, rlo, rhi = boot_ci([r["A_us"] for r in rs], [r["B_us"] for r in rs])
        lo, hi = boot_ci_hier(rs)
        per_launch = [ratio_of_medians([r["A_us"] for r in rs if r["launch"] == L],
                                       [r["B_us"] for r in rs if r["launch"] == L])
                      for L in sorted({r["launch"] for r in rs})]
        summary.append({"T": T, "A_us": float(np.median([r["A_us"] for r in rs])),
                        "B_us": float(np.median([r["B_us"] for r in rs])), "speedup_B_over_A": sp,
                        "ci95": [lo, hi], "ci95_rounds_only": [rlo, rhi], "per_launch": per_launch,
                        "errA": rs[0]["errA"], "errB": rs[0]["errB"], "n": len(rs)})
    return summary


def _variant_path(v):
    if os.path.exists(v):
        return v
    here = os.path.dirname(os.path.abspath(__file__))
    return os.path.join(here, "variants", v if v.endswith(".py") else v + ".py")


def child(a):
    import torch
    from moelab_amd import backend as be, guard
    from moelab_amd.shapes import SHAPES, MoEShape
    sh = SHAPES[a.shape] if not a.dims else MoEShape(a.shape, *map(int, a.dims.split(",")))
    w = be.make_weights(sh, a.dtype, seed=a.seed)
    mods = [be.load_variant(_variant_path(p)) for p in (a.A, a.B)]
    states = [m.prepare(*w) for m in mods]
    torch.cuda.synchronize()
    print(json.dumps({"probe": guard.probe()}), flush=True)
    for T in a.tokens:
        inp = [be.make_inputs(sh, T, a.dtype, a.routing, seed=a.seed * 100 + s) for s in range(a.windows)]
        x, idx, wts = inp[0]
        rw = mods[1].dequant(states[1]) if hasattr(mods[1], "dequant") else w
        ref = be.reference(*rw, x, idx, wts)
        errs = [be.errors(m.run(s, x, idx, wts), ref)["rel_fro"] for m, s in zip(mods, states)]
        for r in range(a.rounds):
            res = {}
            for i in ((0, 1) if r % 2 == 0 else (1, 0)):
                ts = be.time_chained(lambda *z: mods[i].run(states[i], *z), inp, reps=5)
                res[i] = float(np.median(ts)) * 1e6
            print(json.dumps({"T": T, "round": r, "A_us": res[0], "B_us": res[1], "errA": errs[0],
                              "errB": errs[1]}), flush=True)
    print(json.dumps({"probe": guard.probe()}), flush=True)


def parse(argv):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("A")
    ap.add_argument("B")
    ap.add_argument("--shape", default="qwen3-30b-a3b")
    ap.add_argument("--dims", default=None, help="custom shape d,f,E,k (overrides --shape)")
    ap.add_argument("--dtype", default="bfloat16")
    ap.add_argument("--routing", default="uniform")
    ap.add_argument("--tokens", type=int, nargs="+", default=[1, 2, 4, 8])
    ap.add_argument("--launches", type=int, default=5)
    ap.add_argument("--rounds", type=int, default=6)
    ap.add_argument("--windows", type=int, default=3, help="distinct (x, routing) inputs per launch")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--seed-base", type=int, default=0, help="launch L uses seed seed_base + L")
    ap.add_argument("--child", action="store_true")
    ap.add_argument("--out", default=None)
    return ap.parse_args(argv)


def main(argv=None):
    a = parse(argv)
    if a.child:
        return child(a)
    from moelab_amd import guard
    rows, probes = [], []
    for L in range(a.launches):
        cmd = [sys.executable, os.path.abspath(__file__), a.A, a.B, "--child", "--shape", a.shape, "--dtype", a.dtype,
               "--routing", a.routing, "--rounds", str(a.rounds), "--seed", str(a.seed_base + L), "--windows",
               str(a.windows), "--tokens", *map(str, a.tokens)] + (["--dims", a.dims] if a.dims else [])
        out = subprocess.run(cmd, capture_output=True, text=True, check=True).stdout
        recs = [json.loads(line) for line in out.splitlines() if line.startswith("{")]
        probes += [r["probe"] for r in recs if "probe" in r]
        rows += [dict(r, launch=L) for r in recs if "probe" not in r]
    summary = summarize(rows, a.tokens)
    print(f"A={os.path.basename(a.A)}  B={os.path.basename(a.B)}  shape={a.shape} {a.dtype} {a.routing}  "
          f"{a.launches} launches x {a.rounds} rounds")
    for s in summary:
        print(f"T={s['T']:3d}  A {s['A_us']:8.1f}us  B {s['B_us']:8.1f}us  B is {s['speedup_B_over_A']:.3f}x  "
              f"[95% CI {s['ci95'][0]:.3f}-{s['ci95'][1]:.3f}, by launch]  err A {s['errA']:.1e} B {s['errB']:.1e}")
    g = guard.verdict(probes) if probes else None
    if g:
        print(guard.report(g))
    if a.out:
        with open(a.out, "w") as f:
            json.dump({"args": vars(a), "rows": rows, "summary": summary, "guard": g, "probes": probes}, f, indent=1)
    return summary


if __name__ == "__main__":
    # run as a script (also the per-launch child): load the package from the source tree first
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import __graft_entry__
    __graft_entry__.load_package()
    from moelab_amd import compare as _pkg
    _pkg.main()
