"""A/B timing of two variants of the expert path on one MI355X, with launch-to-launch variation in the interval.

The harness capability is the reference's (moelab/compare.py: interleaved A/B rounds in several independent
processes, a 95% interval on the ratio of medians from a two-stage bootstrap); this module is built differently:

* A launch is a fresh interpreter started by ``multiprocessing`` (spawn) that runs ``run_launch`` on a
  ``LaunchSpec`` and hands its rows back as Python objects. It builds its own weights and input windows from its
  seed, checks both arms once against the fp32 reference, captures ONE HIP graph per arm and token count (the
  variant's call chained over the windows, x <- x + run(x)), and replays the two graphs round after round. The
  order of the two arms in each round is a coin drawn from the launch's seed, so neither arm always runs first.
  Capturing once and replaying keeps capture and host launch cost out of every timed interval.
* Rows are long-format, one per replay of one arm: ``{"launch", "tokens", "round", "arm", "us_per_call"}``.
* ``Interval`` statistics work on [launch, round] arrays. ``ratio`` = median(A) / median(B) over every row of a token
  count (B is ``ratio`` x faster than A). ``interval95`` resamples launches with replacement and then, inside each
  drawn launch, its rounds (A and B of a round stay paired), all replicates drawn as one index array.
  ``interval95_rounds`` keeps every launch once and resamples rounds inside each: the spread a single launch would
  show, narrower whenever launches differ.

    python moe-lab_amd/compare.py hip_q4_moe mymod.py --shape qwen3-30b-a3b --tokens 1 8 32 --launches 5 --rounds 6
"""
import argparse
import dataclasses
import json
import multiprocessing
import os
import sys

import numpy as np


# ------------------------------------------------------------------------------------------ statistics
def paired_arrays(rows, tokens):
    """The rows of one token count as two [launch, round] arrays (A, B) of microseconds per call, launches in
    ascending id. Every launch of a run records the same number of rounds."""
    launches = sorted({r["launch"] for r in rows if r["tokens"] == tokens})
    rounds = sorted({r["round"] for r in rows if r["tokens"] == tokens})
    a = np.full((len(launches), len(rounds)), np.nan)
    b = np.full_like(a, np.nan)
    li = {L: i for i, L in enumerate(launches)}
    ri = {R: i for i, R in enumerate(rounds)}
    for r in rows:
        if r["tokens"] != tokens:
            continue
        (a if r["arm"] == "A" else b)[li[r["launch"]], ri[r["round"]]] = r["us_per_call"]
    if np.isnan(a).any() or np.isnan(b).any():
        raise ValueError(f"tokens={tokens}: every launch must record both arms in every round")
    return a, b


def ratio(a, b):
    """median(A) / median(B) over all entries."""
    return float(np.median(a) / np.median(b))


def resample(a, b, n, seed, by_launch=True):
    """n bootstrap replicates of ratio(a, b) for [launch, round] arrays. by_launch: launches drawn with
    replacement, then rounds with replacement inside each drawn launch; otherwise every launch kept once and only
    its rounds redrawn. A and B share every draw (a round's two arms stay together)."""
    L, R = a.shape
    rng = np.random.default_rng(seed)
    pick = rng.integers(0, L, size=(n, L)) if by_launch else np.broadcast_to(np.arange(L), (n, L))
    rnd = rng.integers(0, R, size=(n, L, R))
    rows = pick[:, :, None]
    sa = a[rows, rnd].reshape(n, L * R)
    sb = b[rows, rnd].reshape(n, L * R)
    return np.median(sa, axis=1) / np.median(sb, axis=1)


@dataclasses.dataclass
class Interval:
    ratio: float
    lo: float
    hi: float

    @classmethod
    def of(cls, a, b, n=4000, seed=0, by_launch=True):
        lo, hi = np.percentile(resample(a, b, n, seed, by_launch), [2.5, 97.5])
        return cls(ratio(a, b), float(lo), float(hi))


def summary_of(rows, tokens, checks=None, n=4000, seed=0):
    """One token count's record: medians, ratio, both intervals, each launch's own ratio, the arms' errors."""
    a, b = paired_arrays(rows, tokens)
    full = Interval.of(a, b, n, seed, by_launch=True)
    inner = Interval.of(a, b, n, seed + 1, by_launch=False)
    rec = {"tokens": tokens, "a_median_us": float(np.median(a)), "b_median_us": float(np.median(b)),
           "ratio": full.ratio, "interval95": [full.lo, full.hi], "interval95_rounds": [inner.lo, inner.hi],
           "launch_ratios": [ratio(a[i], b[i]) for i in range(a.shape[0])], "replays": int(a.size)}
    if checks:
        rec["max_over_rms"] = {arm: max(c[tokens][arm] for c in checks) for arm in ("A", "B")}
    return rec


# ------------------------------------------------------------------------------------------ one launch
@dataclasses.dataclass
class LaunchSpec:
    arm_a: str
    arm_b: str
    shape: tuple          # (name, d, f, E, k)
    dtype: str
    routing: str
    tokens: tuple
    rounds: int
    windows: int
    chain: int
    replays: int          # replays of a graph per round (their median is the round's value)
    seed: int
    launch: int


def variant_path(v):
    """A variant by file path, or by the name of one of this package's variants."""
    if os.path.exists(v):
        return v
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), "variants", v if v.endswith(".py") else v + ".py")


def run_launch(spec):
    """Runs in the launch's own process (spec: a LaunchSpec or its dict): returns {"rows", "checks", "probes"}."""
    import torch
    from moelab_amd import backend as be, guard
    from moelab_amd.shapes import MoEShape
    if isinstance(spec, dict):
        spec = LaunchSpec(**spec)
    shape = MoEShape(*spec.shape)
    dense = be.make_weights(shape, spec.dtype, seed=spec.seed)
    arms = {}
    for arm, path in (("A", spec.arm_a), ("B", spec.arm_b)):
        mod = be.load_variant(variant_path(path))
        arms[arm] = (mod, mod.prepare(*dense))
    torch.cuda.synchronize()
    coin = np.random.default_rng([spec.seed, 7919])
    probes = [guard.probe()]
    rows, checks = [], {}
    for T in spec.tokens:
        wins = [be.make_inputs(shape, T, spec.dtype, spec.routing, seed=[spec.seed, T, w]) for w in range(spec.windows)]
        mod_b, st_b = arms["B"]
        ref_w = mod_b.dequant(st_b) if hasattr(mod_b, "dequant") else dense
        x, idx, wts = wins[0]
        y_ref = be.reference(*ref_w, x, idx, wts)
        checks[T] = {arm: be.errors(m.run(st, x, idx, wts), y_ref)["max_over_rms"] for arm, (m, st) in arms.items()}
        graphs = {arm: be.capture(be.chain_of(lambda *z, m=m, st=st: m.run(st, *z), wins, spec.chain))[0]
                  for arm, (m, st) in arms.items()}
        for rd in range(spec.rounds):
            order = ("A", "B") if coin.random() < 0.5 else ("B", "A")
            for arm in order:
                sec = be.replay_seconds(graphs[arm], spec.replays)
                rows.append({"launch": spec.launch, "tokens": T, "round": rd, "arm": arm,
                             "us_per_call": float(np.median(sec)) / spec.chain * 1e6})
        del graphs
    probes.append(guard.probe())
    return {"rows": rows, "checks": checks, "probes": probes}


def run(arm_a, arm_b, shape, tokens, dtype="bfloat16", routing="uniform", launches=5, rounds=6, windows=3, chain=10,
        replays=5, seed=0, in_process=False):
    """Every launch's rows, checks and guard probes. in_process: run the launches in this process (tests)."""
    specs = [LaunchSpec(arm_a, arm_b, tuple(shape), dtype, routing, tuple(tokens), rounds, windows, chain, replays,
                        seed + L, L) for L in range(launches)]
    if in_process:
        outs = [run_launch(s) for s in specs]
    else:
        # a fresh interpreter per launch, one at a time (launches must not share the GPU while timing); it imports
        # __graft_entry__ by name (the repository root is on its sys.path, as on this one's) to reach the package
        import __graft_entry__
        ctx = multiprocessing.get_context("spawn")
        outs = []
        for s in specs:
            with ctx.Pool(1) as pool:
                outs.append(pool.apply(__graft_entry__.call_in_package,
                                       ("compare", "run_launch", dataclasses.asdict(s))))
    return ([r for o in outs for r in o["rows"]], [o["checks"] for o in outs],
            [p for o in outs for p in o["probes"]])


def shape_tuple(name, dims=None):
    from moelab_amd.shapes import SHAPES
    if dims:
        d, f, E, k = map(int, dims.split(","))
        return (name, d, f, E, k)
    s = SHAPES[name]
    return (s.name, s.d, s.f, s.E, s.k)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("arm_a", help="variant A: a file path or one of moe-lab_amd/variants")
    ap.add_argument("arm_b", help="variant B")
    ap.add_argument("--shape", default="qwen3-30b-a3b")
    ap.add_argument("--dims", default=None, help="d,f,E,k of a custom shape (named by --shape)")
    ap.add_argument("--dtype", default="bfloat16")
    ap.add_argument("--routing", default="uniform", choices=("uniform", "zipf", "one_hot"))
    ap.add_argument("--tokens", type=int, nargs="+", default=[1, 2, 4, 8])
    ap.add_argument("--launches", type=int, default=5)
    ap.add_argument("--rounds", type=int, default=6)
    ap.add_argument("--windows", type=int, default=3, help="(x, routing) windows each graph chains over")
    ap.add_argument("--chain", type=int, default=10, help="dependent calls per graph")
    ap.add_argument("--replays", type=int, default=5, help="replays per arm and round (their median is timed)")
    ap.add_argument("--seed", type=int, default=0, help="launch L uses seed + L")
    ap.add_argument("--in-process", action="store_true", help="run the launches in this process")
    ap.add_argument("--json", default=None, help="write rows, checks, probes and summaries here")
    a = ap.parse_args(argv)
    from moelab_amd import guard
    shape = shape_tuple(a.shape, a.dims)
    rows, checks, probes = run(a.arm_a, a.arm_b, shape, a.tokens, a.dtype, a.routing, a.launches, a.rounds, a.windows,
                               a.chain, a.replays, a.seed, a.in_process)
    summaries = [summary_of(rows, T, checks) for T in a.tokens]
    g = guard.verdict(probes) if probes else None
    width = max(len(os.path.basename(a.arm_a)), len(os.path.basename(a.arm_b)), 4)
    print(f"# {shape[0]} (d={shape[1]} f={shape[2]} E={shape[3]} k={shape[4]}) {a.dtype} {a.routing}: "
          f"{a.launches} launches, {a.rounds} rounds, {a.chain}-call graphs")
    print(f"# A = {os.path.basename(a.arm_a):{width}s}  B = {os.path.basename(a.arm_b)}")
    print(f"{'tokens':>6} {'A us':>9} {'B us':>9} {'A/B':>7}   {'95% (launches)':>15}   {'95% (rounds)':>13}"
          f"   max|err|/rms A, B")
    for s in summaries:
        e = s.get("max_over_rms", {"A": float("nan"), "B": float("nan")})
        print(f"{s['tokens']:6d} {s['a_median_us']:9.2f} {s['b_median_us']:9.2f} {s['ratio']:7.3f}   "
              f"{s['interval95'][0]:6.3f}..{s['interval95'][1]:<6.3f}   "
              f"{s['interval95_rounds'][0]:6.3f}..{s['interval95_rounds'][1]:<6.3f}   {e['A']:.1e}, {e['B']:.1e}")
    if g:
        print(guard.report(g))
    if a.json:
        with open(a.json, "w") as f:
            json.dump({"args": vars(a), "rows": rows, "checks": [{str(k): v for k, v in c.items()} for c in checks],
                       "probes": probes, "guard": g, "summaries": summaries}, f, indent=1)
    return summaries


if __name__ == "__main__":
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import __graft_entry__
    __graft_entry__.load_package()
    from moelab_amd import compare as _pkg
    _pkg.main()
