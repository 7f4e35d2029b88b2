"""Load-policy grid on MI355X: real-model shapes x T chosen by load = T*k/E (average slots per expert), the
per-slot arm (fallback.gather_moe: every slot streams its expert's rows) against the grouped arm (group,
expert tiles, combine), to set the dispatchers' thresholds (reference moelab/grid.py:1-90 fits the same
policy between mlx-lm's gather path and the custom kernels).

Each (shape, T): two packed layers with different weights alternate from call to call (so consecutive calls
do not find their weights in the 256 MB memory-side cache), 4 (x, routing) windows, 3 interleaved rounds of
5 timed runs of 10 back-to-back calls;
the medians per arm and their ratio are recorded, and per shape the smallest load from which the grouped arm
wins at every larger load measured. The run is bracketed by guard probes.

    python moe-lab_amd/grid.py --out grid.json
"""
import argparse
import json
import os
import sys

import numpy as np

GRID_SHAPES = ["qwen3-30b-a3b", "olmoe-1b-7b", "deepseek-v2-lite", "gpt-oss-20b", "mixtral-8x7b"]
LOADS = [0.0625, 0.125, 0.25, 0.5, 1, 2, 4, 8, 16, 32, 64, 128]


def t_for_load(load, E, k):
    return max(2, int(round(load * E / k)))


class Alternating:
    """fn(layer, x, idx, wts) over two layers in turn (consecutive calls read different weights)."""

    def __init__(self, layers, fn):
        self.layers, self.fn, self.i = layers, fn, 0

    def __call__(self, x, idx, wts):
        self.i ^= 1
        return self.fn(self.layers[self.i], x, idx, wts)


def time_calls(fn, inputs, reps=5, calls=10):
    """Seconds per call: `calls` back-to-back calls over the input windows between two HIP events, median of
    `reps`. The calls are independent (no residual chain), so activations keep their scale whatever the
    layer's gain; on one stream they still run one after another."""
    import torch
    for i in range(len(inputs)):
        fn(*inputs[i])
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(calls):
            fn(*inputs[i % len(inputs)])
        e1.record()
        e1.synchronize()
        ts.append(e0.elapsed_time(e1) / 1e3 / calls)
    return ts


def crossover(rows):
    """Smallest load L such that the grouped arm wins (ratio > 1) at L and at every larger load measured; None
    if it loses at the largest."""
    rows = sorted(rows, key=lambda r: r["load"])
    best = None
    for r in reversed(rows):
        if r["slots_over_grouped"] > 1.0:
            best = r["load"]
        else:
            break
    return best


def main(argv=None):
    import torch
    from moelab_amd import _lib, backend as be, guard
    from moelab_amd.experts import run_layer
    from moelab_amd.fallback import gather_moe
    from moelab_amd.problem import baseline_int4_layer, baseline_mxfp4_layer
    from moelab_amd.shapes import SHAPES
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--shapes", nargs="+", default=GRID_SHAPES)
    ap.add_argument("--loads", type=float, nargs="+", default=LOADS)
    ap.add_argument("--max-t", type=int, default=512)
    ap.add_argument("--out", default=None)
    a = ap.parse_args(argv)
    probes, rows, fits = [guard.probe()], [], {}
    for name in a.shapes:
        sh = SHAPES[name]
        fmt = "mxfp4" if name.startswith("gpt-oss") else "int4"
        mk = baseline_mxfp4_layer if fmt == "mxfp4" else baseline_int4_layer
        act = 2 if fmt == "mxfp4" else 0
        layers = [mk(sh, seed=500 + i, device="cuda") for i in range(2)]
        Ts = sorted({t_for_load(L, sh.E, sh.k) for L in a.loads} - set(range(a.max_t + 1, 1 << 30)))
        srows = []
        for T in Ts:
            inp = [be.make_inputs(sh, T, "bfloat16", "uniform", seed=900 + s) for s in range(4)]
            arms = {
                "slots": Alternating(layers, lambda s, x, idx, wts: gather_moe(s, x, idx, wts, act=act)),
                "grouped": Alternating(layers, lambda s, x, idx, wts: run_layer(s, x, idx, wts, act=act,
                                                                                path=_lib.PATH_GROUPED)),
            }
            ts = {n: [] for n in arms}
            for r in range(3):
                for n in (("slots", "grouped") if r % 2 == 0 else ("grouped", "slots")):
                    ts[n] += time_calls(arms[n], inp)
            med = {n: float(np.median(v)) * 1e6 for n, v in ts.items()}
            row = {"shape": name, "fmt": fmt, "T": T, "load": T * sh.k / sh.E, "slots_us": med["slots"],
                   "grouped_us": med["grouped"], "slots_over_grouped": med["slots"] / med["grouped"]}
            rows.append(row)
            srows.append(row)
            print(json.dumps(row), flush=True)
        fits[name] = {"grouped_from_load": crossover(srows), "E": sh.E, "k": sh.k, "d": sh.d, "f": sh.f}
        print(json.dumps({"fit": name, **fits[name]}), flush=True)
        del layers
        torch.cuda.empty_cache()
        probes.append(guard.probe())
    g = guard.verdict(probes)
    print(guard.report(g))
    if a.out:
        with open(a.out, "w") as f:
            json.dump({"rows": rows, "fits": fits, "guard": g, "probes": probes}, f, indent=1)
    return rows, fits


if __name__ == "__main__":
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import __graft_entry__
    __graft_entry__.load_package()
    from moelab_amd import grid as _pkg
    _pkg.main()
