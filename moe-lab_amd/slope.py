"""Slope timing on ROCm: per-call device time = slope of a chain's total time against its length (reference
moelab/slope.py:1-70).

A chain is `chain` dependent calls x <- x + run(x) between two HIP events; its total time is a fixed cost
(launch of the first call, the events, the final wait) plus `chain` times the per-call time, so the
least-squares slope over several chain lengths drops the fixed part. The residual add alone (run = zeros)
is fitted the same way and subtracted. The floor is the roofline's weight bytes (unique experts of the
windows) at --bw GB/s (MI355X HBM3E: 8000). --windows distinct inputs rotate through the chain, at least as
many as the longest chain, so no expert set repeats inside one chain.

Each chain is captured once into a HIP graph and the graph is replayed between the events (graph_total_time,
the default): launched eagerly from Python, a chain is bound by the host's launch rate (the residual add
alone then costs ~10 us per call on MI355X hosts, against ~2 us of device time), and the subtraction would
remove host time from device time. --eager times the chains as launched (total_time, the reference's form).

    python moe-lab_amd/slope.py --shape qwen3-30b-a3b --T 1 --variants hip_q4_moe
"""
import argparse
import os
import sys

import numpy as np

CHAINS = (10, 20, 40, 80)


def total_time(fn, inputs, chain, reps=7):
    """Median seconds of a chain of `chain` dependent calls (HIP events on the current stream)."""
    import torch

    def build():
        x = inputs[0][0]
        for i in range(chain):
            _, idx, w = inputs[i % len(inputs)]
            x = x + fn(x, idx, w).to(x.dtype)
        return x

    build()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        build()
        e1.record()
        e1.synchronize()
        ts.append(e0.elapsed_time(e1) / 1e3)
    return float(np.median(ts))


def graph_total_time(fn, inputs, chain, reps=7):
    """Median seconds of one replay of a HIP graph holding a chain of `chain` dependent calls."""
    import torch

    def build():
        x = inputs[0][0]
        for i in range(chain):
            _, idx, w = inputs[i % len(inputs)]
            x = x + fn(x, idx, w).to(x.dtype)
        return x

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        build()   # eager warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        build()
    g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        e1.synchronize()
        ts.append(e0.elapsed_time(e1) / 1e3)
    del g
    return float(np.median(ts))


def fit_line(chains, totals):
    """(slope, intercept) of the least-squares line through (chain, total)."""
    A = np.stack([np.asarray(chains, float), np.ones(len(chains))], axis=1)
    (slope, icpt), *_ = np.linalg.lstsq(A, np.asarray(totals, float), rcond=None)
    return float(slope), float(icpt)


def fit(fn, inputs, chains=CHAINS, timer=total_time):
    """Per-call and fixed time in microseconds."""
    s, c = fit_line(chains, [timer(fn, inputs, ch) for ch in chains])
    return s * 1e6, c * 1e6


def main(argv=None):
    import torch
    from moelab_amd import backend as be, guard, roofline
    from moelab_amd.shapes import SHAPES
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--shape", default="qwen3-30b-a3b")
    ap.add_argument("--dtype", default="bfloat16")
    ap.add_argument("--T", type=int, default=1)
    ap.add_argument("--routing", default="uniform")
    ap.add_argument("--variants", nargs="+", required=True)
    ap.add_argument("--windows", type=int, default=max(CHAINS))
    ap.add_argument("--bw", type=float, default=8000.0, help="read GB/s of the part (MI355X HBM3E: 8000)")
    ap.add_argument("--eager", action="store_true", help="time eagerly launched chains instead of graph replays")
    a = ap.parse_args(argv)
    timer = total_time if a.eager else graph_total_time
    sh = SHAPES[a.shape]
    w = be.make_weights(sh, a.dtype)
    inp = [be.make_inputs(sh, a.T, a.dtype, a.routing, 1000 + s) for s in range(a.windows)]
    res_us, res_icpt = fit(lambda x, i, ww: torch.zeros_like(x), inp, timer=timer)
    U = float(np.mean([i[1].unique().numel() for i in inp]))
    print(f"{a.shape} T={a.T} {a.routing} windows={a.windows} {'eager' if a.eager else 'graph'}: "
          f"residual-add-only slope {res_us:.2f}us "
          f"(fixed {res_icpt:.0f}us)")
    probes = [guard.probe()]
    base = None
    out = []
    here = os.path.dirname(os.path.abspath(__file__))
    for v in a.variants:
        path = v if os.path.exists(v) else os.path.join(here, "variants", v + ".py")
        m = be.load_variant(path)
        st = m.prepare(*w)
        floor = roofline.bytes_moved(a.T, sh.d, sh.f, sh.E, sh.k, getattr(m, "W_BITS", 4.5), unique=U) / (a.bw * 1e9) * 1e6
        s, c = fit(lambda *z: m.run(st, *z), inp, timer=timer)
        net = s - res_us
        base = base or net
        rec = {"variant": v, "per_call_us": s, "net_us": net, "fixed_us": c, "floor_us": floor,
               "frac_of_floor": floor / net, "speedup": base / net}
        out.append(rec)
        print(f"  {v:22s} per-call {s:7.2f}us  minus residual {net:7.2f}us  fixed {c:6.0f}us  floor {floor:6.2f}us  "
              f"{100 * floor / net:5.1f}% of floor@{a.bw:.0f}  speedup {base / net:.3f}x")
        del st
        probes.append(guard.probe())
    print(guard.report(guard.verdict(probes)))
    return out


if __name__ == "__main__":
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import __graft_entry__
    __graft_entry__.load_package()
    from moelab_amd import slope as _pkg
    _pkg.main()
