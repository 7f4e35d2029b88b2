"""Per-call device time of a variant: the slope of a chain's replay time against its length, on one MI355X.

The measurement is the reference's (moelab/slope.py: per-call time as the slope of chained timing over several chain
lengths, the chain's own residual add measured alone and subtracted, and the result against the weight-byte floor);
this module takes it its own way:

* For each length n in ``lengths`` (default 8, 16, 32, 64) ONE HIP graph holds n dependent calls x <- x + run(x)
  over the input windows; its replays are timed with HIP events on the replaying stream (``backend.replay_seconds``).
  A replayed graph has no host launch cost inside it, so the fixed part of a replay is the graph launch and the
  events alone.
* The slope is Theil-Sen's: the median of the slopes between every pair of lengths, each length represented by the
  median of its replays. One disturbed length (a clock change, a neighbour on the GPU) moves it far less than it moves
  a least-squares line, which ``least_squares`` gives beside it.
* The chain's own update (the add of a zero tensor) is measured the same way as the ``carry`` and subtracted: the
  variant's own time is ``slope - carry``. ``floor_us`` is the packed bytes of the distinct experts the windows select
  at ``hbm_gbs`` (MI355X HBM3E: 8000 GB/s).

    python moe-lab_amd/slope.py --shape qwen3-30b-a3b --tokens 1 --variants hip_q4_moe
"""
import argparse
import dataclasses
import itertools
import os
import sys

import numpy as np

LENGTHS = (8, 16, 32, 64)


def theil_sen(xs, ys):
    """(slope, intercept): the median of the pairwise slopes, and the median of y - slope * x."""
    xs, ys = np.asarray(xs, float), np.asarray(ys, float)
    pairs = [(ys[j] - ys[i]) / (xs[j] - xs[i]) for i, j in itertools.combinations(range(xs.size), 2) if xs[j] != xs[i]]
    if not pairs:
        raise ValueError("theil_sen needs two distinct x values")
    s = float(np.median(pairs))
    return s, float(np.median(ys - s * xs))


def least_squares(xs, ys):
    """(slope, intercept) of the least-squares line."""
    s, c = np.polyfit(np.asarray(xs, float), np.asarray(ys, float), 1)
    return float(s), float(c)


def replay_time(fn, windows, n, replays=7):
    """Median seconds of a replay of one HIP graph of n dependent calls x <- x + fn(x, idx, wts)."""
    from moelab_amd import backend as be
    g, _ = be.capture(be.chain_of(fn, windows, n))
    t = float(np.median(be.replay_seconds(g, replays)))
    del g
    return t


@dataclasses.dataclass
class Line:
    per_call_us: float     # Theil-Sen slope
    fixed_us: float        # its intercept: what a replay costs beyond its calls
    lsq_per_call_us: float # least-squares slope of the same points
    points: dict           # chain length -> median replay seconds


def measure(fn, windows, lengths=LENGTHS, timer=replay_time):
    """The Line of fn's chains (timer(fn, windows, n) -> seconds for one chain of n calls)."""
    pts = {int(n): timer(fn, windows, n) for n in lengths}
    s, c = theil_sen(list(pts), list(pts.values()))
    ls, _ = least_squares(list(pts), list(pts.values()))
    return Line(s * 1e6, c * 1e6, ls * 1e6, pts)


@dataclasses.dataclass
class VariantSlope:
    variant: str
    per_call_us: float   # the variant's chain slope
    own_us: float        # minus the carry (the chain's add alone)
    fixed_us: float
    floor_us: float
    frac_of_floor: float
    lsq_own_us: float


def run(shape, variants, tokens=1, dtype="bfloat16", routing="uniform", windows=None, lengths=LENGTHS,
        hbm_gbs=8000.0):
    """(carry Line, [VariantSlope]) for each variant (a path or one of moe-lab_amd/variants)."""
    import torch
    from moelab_amd import backend as be, roofline
    from moelab_amd.compare import variant_path
    nwin = windows or max(lengths)   # at least the longest chain: no expert set repeats inside a chain
    wins = [be.make_inputs(shape, tokens, dtype, routing, seed=[41, tokens, w]) for w in range(nwin)]
    carry = measure(lambda x, idx, wts: torch.zeros_like(x), wins, lengths)
    distinct = float(np.mean([w[1].unique().numel() for w in wins]))
    dense = be.make_weights(shape, dtype)
    out = []
    for v in variants:
        mod = be.load_variant(variant_path(v))
        st = mod.prepare(*dense)
        line = measure(lambda *z: mod.run(st, *z), wins, lengths)
        wbytes = roofline.bytes_moved(tokens, shape.d, shape.f, shape.E, shape.k, getattr(mod, "W_BITS", 4.5),
                                      unique=distinct)
        floor = wbytes / (hbm_gbs * 1e9) * 1e6
        own = line.per_call_us - carry.per_call_us
        out.append(VariantSlope(v, line.per_call_us, own, line.fixed_us, floor, floor / own if own > 0 else 0.0,
                                line.lsq_per_call_us - carry.lsq_per_call_us))
        del st
    return carry, out


def main(argv=None):
    from moelab_amd import compare, guard
    from moelab_amd.shapes import MoEShape
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--shape", default="qwen3-30b-a3b")
    ap.add_argument("--dims", default=None, help="d,f,E,k of a custom shape (named by --shape)")
    ap.add_argument("--dtype", default="bfloat16")
    ap.add_argument("--tokens", type=int, default=1)
    ap.add_argument("--routing", default="uniform", choices=("uniform", "zipf", "one_hot"))
    ap.add_argument("--variants", nargs="+", required=True)
    ap.add_argument("--lengths", type=int, nargs="+", default=list(LENGTHS), help="chain lengths (graph sizes)")
    ap.add_argument("--windows", type=int, default=None, help="distinct inputs (default: the longest chain)")
    ap.add_argument("--hbm-gbs", type=float, default=8000.0, help="HBM read rate of the floor (MI355X: 8000)")
    a = ap.parse_args(argv)
    shape = MoEShape(*compare.shape_tuple(a.shape, a.dims))
    probes = [guard.probe()]
    carry, res = run(shape, a.variants, a.tokens, a.dtype, a.routing, a.windows, a.lengths, a.hbm_gbs)
    probes.append(guard.probe())
    print(f"# {shape.name} T={a.tokens} {a.routing}, graphs of {'/'.join(map(str, a.lengths))} calls: "
          f"carry (x + 0 alone) {carry.per_call_us:.2f} us per call, replay overhead {carry.fixed_us:.1f} us")
    print(f"{'variant':24s} {'slope us':>9} {'own us':>8} {'(lsq)':>8} {'floor us':>9} {'of floor':>9} "
          f"{'vs first':>9}")
    for r in res:
        print(f"{r.variant:24s} {r.per_call_us:9.2f} {r.own_us:8.2f} {r.lsq_own_us:8.2f} {r.floor_us:9.2f} "
              f"{100 * r.frac_of_floor:8.1f}% {res[0].own_us / r.own_us:8.3f}x")
    print(guard.report(guard.verdict(probes)))
    return carry, res


if __name__ == "__main__":
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import __graft_entry__
    __graft_entry__.load_package()
    from moelab_amd import slope as _pkg
    _pkg.main()
