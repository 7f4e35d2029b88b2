"""Random-shape sweep: is the default dispatch correct, and not slower than the per-slot path, away from the shapes
it was tuned on? The reference runs such a screen over random shapes, token counts, dtypes and routings
(moelab/sweep.py:1-8, 38-85); this one is its own design on this build's harness.

Each case is drawn from a seeded generator (`draw_case`): d and F multiples of 64 (the library's requirement), E a
power of two from 8 to 256, k <= E, T from 1 to 128 (small T more often), bf16 or fp16 activations, uniform, Zipf or
one-hot routing, int4 g64 or MXFP4 weights, under a cap on the dense weight bytes. For each case:
  * random dense weights go through the variant's prepare() (hip_q4_moe or hip_mxfp4_moe);
  * correctness: the default call with fp32 output against the fp32 reference on the variant's dequant() (the
    north-star gate max|y - y_ref| <= 1e-2 RMS), and the x.dtype output against the harness's rel-Fro TOL;
  * speed: the per-slot arm (fallback.gather_moe: every slot streams its own expert, the stock-gather stand-in) and
    the default arm (the variant's run()) as captured HIP-graph chains of dependent calls over two input windows,
    timed in alternating order over two rounds; the per-call time of an arm is its fastest round's median replay.
A case that fails a gate, or whose default arm is slower than the per-slot arm by more than --flag, is flagged;
timing flags are a screen, to be re-measured with compare.py. The guard's read probe brackets the run.

    python moe-lab_amd/sweep.py --n 40 --seed 7 --out sweep.json
"""
import argparse
import json
import os
import sys
from dataclasses import asdict, dataclass

import numpy as np

VARIANTS = {"int4": "hip_q4_moe", "mxfp4": "hip_mxfp4_moe"}
T_CHOICES = (1, 1, 1, 2, 3, 4, 5, 8, 12, 16, 24, 32, 48, 64, 96, 128)


@dataclass(frozen=True)
class Case:
    d: int
    F: int
    E: int
    k: int
    T: int
    dtype: str
    routing: str
    fmt: str

    @property
    def name(self):
        return f"{self.fmt}-d{self.d}-F{self.F}-E{self.E}-k{self.k}"

    def dense_bytes(self):
        return 3 * self.E * self.d * self.F * 2


def draw_case(rng, max_dense_bytes=1.5e9, fmts=("int4", "mxfp4")):
    """One random case from numpy Generator `rng` (rejection-sampled under the weight cap)."""
    while True:
        d = 64 * int(rng.integers(8, 81))           # 512 .. 5120
        F = 64 * int(rng.integers(4, 65))           # 256 .. 4096
        E = 1 << int(rng.integers(3, 9))            # 8 .. 256
        k = int(rng.choice([1, 2, 4, 6, 8]))
        if k > E:
            continue
        c = Case(d=d, F=F, E=E, k=k, T=int(rng.choice(T_CHOICES)),
                 dtype=str(rng.choice(["bfloat16", "float16"])),
                 routing=str(rng.choice(["uniform", "uniform", "zipf", "one_hot"])), fmt=str(rng.choice(list(fmts))))
        if c.dense_bytes() <= max_dense_bytes:
            return c


def draw_cases(n, seed, **kw):
    rng = np.random.default_rng(seed)
    return [draw_case(rng, **kw) for _ in range(n)]


def arm_seconds(graphs, rounds=2, replays=5):
    """Per-call seconds of each arm: graphs {name: (graph, calls per replay)} replayed in alternating order for
    `rounds` rounds of `replays`; an arm's time is its fastest round's median replay over its call count."""
    from .backend import replay_seconds
    names = list(graphs)
    best = {n: float("inf") for n in names}
    for r in range(rounds):
        for n in (names if r % 2 == 0 else names[::-1]):
            g, calls = graphs[n]
            best[n] = min(best[n], float(np.median(replay_seconds(g, replays))) / calls)
    return best


def run_case(case, seed, chain=8, rounds=2, replays=5):
    """Build, check and time one case; returns its row."""
    import torch
    from . import backend as be
    from .fallback import gather_moe
    from .shapes import MoEShape
    mod = be.load_variant(os.path.join(os.path.dirname(os.path.abspath(__file__)), "variants",
                                       VARIANTS[case.fmt] + ".py"))
    sh = MoEShape(case.name, d=case.d, f=case.F, E=case.E, k=case.k)
    w = be.make_weights(sh, case.dtype, seed=seed)
    s = mod.prepare(*w)
    del w
    windows = [be.make_inputs(sh, case.T, case.dtype, case.routing, seed=(seed, i)) for i in range(2)]
    x, idx, wts = windows[0]
    ref = be.reference(*mod.dequant(s), x, idx, wts)
    y32 = mod.run(s, x, idx, wts, out_dtype=torch.float32)
    yd = mod.run(s, x, idx, wts)
    e32, ed = be.errors(y32, ref), be.errors(yd, ref)
    ok = e32["finite"] and e32["max_over_rms"] <= be.NORTH_STAR_GATE and ed["rel_fro"] < be.TOL[case.dtype]
    arms = {"slots": lambda x, i, w_: gather_moe(s, x, i, w_), "default": lambda x, i, w_: mod.run(s, x, i, w_)}
    graphs = {n: (be.capture(be.chain_of(fn, windows, chain))[0], chain) for n, fn in arms.items()}
    t = arm_seconds(graphs, rounds, replays)
    del graphs, s
    torch.cuda.empty_cache()
    return {**asdict(case), "case": case.name, "seed": seed, "slots_us": t["slots"] * 1e6,
            "default_us": t["default"] * 1e6, "slots_over_default": t["slots"] / t["default"],
            "max_over_rms": e32["max_over_rms"], "rel_fro": ed["rel_fro"], "ok": bool(ok)}


def flagged(row, flag):
    return (not row["ok"]) or row["slots_over_default"] < flag


def summary(rows, flag):
    sp = np.array([r["slots_over_default"] for r in rows]) if rows else np.array([np.nan])
    return {"cases": len(rows), "all_correct": all(r["ok"] for r in rows),
            "worst_max_over_rms": max((r["max_over_rms"] for r in rows), default=float("nan")),
            "slots_over_default_median": float(np.median(sp)), "slots_over_default_min": float(np.min(sp)),
            "flagged": [r["case"] + f" T={r['T']}" for r in rows if flagged(r, flag)]}


def run(n, seed, flag=0.95, fmts=("int4", "mxfp4"), max_dense_bytes=1.5e9, probe=True, emit=print):
    """The sweep: n cases from `seed`; returns (rows, summary, guard verdict or None)."""
    from . import guard
    cases = draw_cases(n, seed, max_dense_bytes=max_dense_bytes, fmts=fmts)
    probes = [guard.probe()] if probe else []
    rows = []
    for i, c in enumerate(cases):
        emit(f"case {i} {c.name} T={c.T} {c.dtype} {c.routing}")
        row = run_case(c, seed=1000 * seed + i)
        rows.append(row)
        emit(f"  per-slot {row['slots_us']:9.1f} us  default {row['default_us']:9.1f} us  "
             f"{row['slots_over_default']:6.2f}x  max/RMS {row['max_over_rms']:.1e}  rel-Fro {row['rel_fro']:.1e}"
             + ("  FLAG" if flagged(row, flag) else ""))
        if probe and i % 10 == 9:
            probes.append(guard.probe())
    g = None
    if probe:
        probes.append(guard.probe())
        g = guard.verdict(probes)
    return rows, summary(rows, flag), g


def main(argv=None):
    from . import guard
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--n", type=int, default=40)
    ap.add_argument("--seed", type=int, default=7)
    ap.add_argument("--fmt", nargs="+", default=["int4", "mxfp4"], choices=list(VARIANTS))
    ap.add_argument("--flag", type=float, default=0.95,
                    help="flag cases whose per-slot / default time ratio is below this")
    ap.add_argument("--max-dense-gb", type=float, default=1.5)
    ap.add_argument("--out", default=None)
    a = ap.parse_args(argv)
    rows, summ, g = run(a.n, a.seed, a.flag, tuple(a.fmt), a.max_dense_gb * 1e9)
    print(json.dumps(summ))
    if g is not None:
        print(guard.report(g))
    if a.out:
        with open(a.out, "w") as f:
            json.dump({"args": vars(a), "rows": rows, "summary": summ, "guard": g}, f, indent=1)
    return rows, summ


if __name__ == "__main__":
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import __graft_entry__
    __graft_entry__.load_package()
    from moelab_amd import sweep as _pkg
    _pkg.main()
