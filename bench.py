"""Benchmark: quantised MoE layer on one MI355X (BASELINE metric: MoE layer us/call + weight-byte GB/s
vs HBM peak at T=1 and T=32).

Workload: Qwen3-30B-A3B-shape int4 g64 SwiGLU MoE layer, d=2048, F=768, E=128, k=8,
T=1, over 48 independently seeded layers (16.3 GB of packed experts, far beyond the 256 MB Infinity
Cache). A step is one token through the 48 layers: x <- x + moe_l(x) for l = 0..47, captured once in a
HIP graph and replayed. `value` is expert weight-byte GB/s of that chain: the packed bytes of the unique
selected experts of all 48 layers divided by the step time, the reference's `run(state, x, idx, wts)`
contract (routing precomputed per layer, reference mlx_backend.py:91-117). The same chain with the
router inside each layer (moe_layer_run) is reported as `with_router`. BASELINE config 3 (T=16, 32 and 64,
uniform and Zipf(1.1) routing) reports the grouped expert path against the per-slot stock-style gather under
`batched`; configs 4, 5a and 5b under `configs`; gpt-oss-20b at T=512 (not a BASELINE config: the MXFP4 tiles
on the block-scaled MFMA) under `mxfp4_prefill`.

roofline: the dominant kernel at T=1 is the gate/up GEMV (2/3 of the weight bytes; the layer is two
launches, gate/up then down). Its average launch duration is measured with HIP events on the stream it
runs on, around replays of a graph of 48 gate/up-only launches (the same kernel the chain runs, through
moe_experts_run_stages); achieved = algorithmic bytes per launch (k experts x gate+up packed rows) /
duration.

cpu_baseline: the reference's CPU torch path (torch_loop, reference variants/cuda/torch_loop.py:11-17)
on dequantised fp32 weights of the selected experts, timed on this host for a bounded sample of layers.
cpu_points: the same path at config 3's T=16, 32 and 64 (one layer each), config 4 at T=1 and T=32 (gpt-oss MXFP4 with
biases and the clamped SwiGLU), and on 32-token samples of configs 5a and 5b.
"""
import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
import __graft_entry__  # noqa: E402

METRIC = "MoE layer µs/call + weight-byte GB/s vs HBM peak at T=1 and T=32"
HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of the T=1 gate/up kernel, from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes over
# `bench.py --layers 8 --steps 5 --warmup 2 --no-t32 --no-configs --cpu-layers 0 --copy-calibrate 256`, each
# scaled by what the counter reads for the 256 MiB device copy of the same run (FETCH_SIZE x 2.0, WRITE_SIZE x
# 1.0): 2 x 6981.0 KiB + 48.0 KiB (profiles/k_gate_up_rows_qwen3_t1_traffic.md)
GU_T1_TRAFFIC_BYTES = int(round((2.0 * 6981.0 + 48.0) * 1024))


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def graph_of(fn):
    """Capture fn() (a chain of launches on the current stream) into a HIP graph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()   # eager warm-up on the capture stream (allocations happen here, not in the graph)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def time_graph(g, steps, warmup):
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    for _ in range(steps):
        g.replay()
    b.record(st)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / 1e3 / steps   # seconds per replay


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--cpu-layers", type=int, default=4, help="layers in the CPU-baseline sample (0: skip)")
    ap.add_argument("--no-t32", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip BASELINE configs 4, 5a, 5b (reported beside)")
    ap.add_argument("--only-configs", default="", metavar="NAMES",
                    help="comma list of BASELINE config names (e.g. mixtral8x7b_int4_T512): run only those and print "
                         "their results (for profiling runs; not the bench line)")
    ap.add_argument("--routed-only", action="store_true",
                    help="with --only-configs: time only the chains with the router inside each layer call (for "
                         "kernel traces of the routed layer)")
    ap.add_argument("--copy-calibrate", type=int, default=0, metavar="MIB",
                    help="finish with 3 device copies of MIB MiB (the plain-copy reference for --pmc traffic runs)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures one MI355X: the expert path is single-GPU (expert "
                                   "parallel sharding is designed, not launched); run with --gpus 1"}))
        sys.exit(2)

    __graft_entry__.load_package()
    if args.only_configs:
        dev = torch.device("cuda:0")
        torch.cuda.set_device(dev)
        print(json.dumps(other_configs(dev, args, only=set(args.only_configs.split(",")))), flush=True)
        copy_calibrate(dev, args.copy_calibrate)
        return
    from moelab_amd import _lib, roofline, router
    from moelab_amd.experts import run_experts
    from moelab_amd.problem import baseline_int4_layer, baseline_x, zipf_bias
    from moelab_amd.shapes import SHAPES

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    sh = SHAPES["qwen3-30b-a3b"]
    L = args.layers
    per_expert = roofline.expert_bytes(sh.d, sh.f, "int4")
    log(f"library {_lib.lib().moe_version().decode()} on {torch.cuda.get_device_name(0)}; building {L} layers")
    t0 = time.time()
    layers = [baseline_int4_layer(sh, seed=1000 + l, device=dev) for l in range(L)]
    torch.cuda.synchronize()
    log(f"layers ready in {time.time() - t0:.1f}s ({L * sh.E * per_expert / 1e9:.2f} GB packed experts)")

    # one workspace for every graph below (graphs keep raw pointers into it): sized before any capture
    from moelab_amd.experts import reserve, run_routed
    reserve(layers[0], 64, sh.k)
    router.reserve(dev, 64)

    # ------------------------------------------------------------------ T = 1: experts-only chain
    x1 = baseline_x(1, sh.d, seed=0, device=dev)
    routes1 = [router.route(x1, ly["wr"], sh.k) for ly in layers]
    U1 = [int(torch.unique(r[0]).numel()) for r in routes1]
    bytes1 = sum(U1) * per_expert

    def chain_t1(path=_lib.PATH_AUTO):
        def f():
            x = x1.clone()
            for ly, (idx, wts) in zip(layers, routes1):
                x = run_experts(ly, x, idx, wts, path=path, residual=x)
            return x
        return f

    def chain_t1_router():   # router + experts per layer in one call (moe_layer_run)
        x = x1.clone()
        for ly in layers:
            x, _, _ = run_routed(ly, x, ly["wr"], sh.k, residual=x)
        return x

    def gate_up_only():
        for ly, (idx, wts) in zip(layers, routes1):
            run_experts(ly, x1, idx, wts, path=_lib.PATH_SLOTS, stages=_lib.STAGE_GATE_UP)

    def down_only():
        for ly, (idx, wts) in zip(layers, routes1):
            run_experts(ly, x1, idx, wts, path=_lib.PATH_SLOTS, stages=_lib.STAGE_DOWN)

    g1, _ = graph_of(chain_t1())
    t_step = time_graph(g1, args.steps, args.warmup)
    log(f"T=1 experts chain (default path: two per-slot launches): {t_step * 1e6 / L:.2f} us/layer, "
        f"{bytes1 / t_step / 1e9:.0f} GB/s")
    g1r, _ = graph_of(chain_t1_router)
    t_step_r = time_graph(g1r, args.steps, args.warmup)
    log(f"T=1 with router: {t_step_r * 1e6 / L:.2f} us/layer")
    ggu, _ = graph_of(gate_up_only)
    t_gu = time_graph(ggu, args.steps, args.warmup) / L
    gdn, _ = graph_of(down_only)
    t_dn = time_graph(gdn, args.steps, args.warmup) / L
    gu_bytes = sh.k * 2 * sh.f * sh.d * roofline.W_BITS["int4"] / 8
    dn_bytes = sh.k * sh.d * sh.f * roofline.W_BITS["int4"] / 8
    log(f"gate/up kernel {t_gu * 1e6:.2f} us ({gu_bytes / t_gu / 1e9:.0f} GB/s), down kernel {t_dn * 1e6:.2f} us "
        f"({dn_bytes / t_dn / 1e9:.0f} GB/s)")

    # ------------------------------------------------------------------ T = 16, 32, 64: grouped vs per-slot
    # (uniform and Zipf(1.1) routing; T=16 and T=64 locate the per-slot / grouped crossover)
    batched = {}
    routes_b = {}
    if not args.no_t32:
        batched = run_batched(dev, layers, sh, args, routes_b=routes_b)

    # ------------------------------------------------------------------ BASELINE configs 4, 5a, 5b
    configs = {}
    prefill = {}   # beside the configs: gpt-oss-20b at T=512 (block-scaled MXFP4 tiles)
    if not args.no_configs:
        del layers
        torch.cuda.empty_cache()
        configs = other_configs(dev, args, extra=prefill)

    # ------------------------------------------------------------------ CPU baseline (bounded samples)
    cpu = None
    cpu_points = {}
    if args.cpu_layers > 0:
        cpu_layers = [baseline_int4_layer(sh, seed=1000 + l, device=dev) for l in range(args.cpu_layers)]
        cpu = cpu_baseline(cpu_layers, routes1[:args.cpu_layers], x1, sh)
        log(f"CPU baseline: {cpu['value']:.1f} us/layer on {cpu['cores']} threads")
        for T in (16, 32, 64):   # config 3 (the first seeded layer of the GPU chain)
            if (T, "uniform") in routes_b:
                xT, routes = routes_b[(T, "uniform")]
                cpu_points[f"qwen3_T{T}_uniform"] = cpu_point([cpu_layers[0]], [routes[0]], xT, sh, f"T={T} uniform",
                                                             3.0)
        cpu_points.update(cpu_large_points(dev))
        for name, r in cpu_points.items():
            log(f"CPU {name}: {r['value']:.1f} {r['unit']} ({r['sample']})")

    value = bytes1 / t_step / 1e9
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_step * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "qwen3-30b-a3b int4-g64 SwiGLU MoE layer, T=1, 48 seeded layers (BASELINE config 2)",
                   "d": sh.d, "F": sh.f, "E": sh.E, "k": sh.k, "T": 1, "layers": L,
                   "weights": "int4 affine g64 (bf16 scale+bias), decoded exactly to bf16 operands",
                   "accumulation": "fp32", "parallelism": "single GPU"},
        "us_per_layer": round(t_step * 1e6 / L, 3),
        "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        "weight_bytes_per_step": bytes1,
        "with_router": {"us_per_layer": round(t_step_r * 1e6 / L, 3),
                        "weight_GBps": round(bytes1 / t_step_r / 1e9, 2)},
        "kernels_t1": {"gate_up_us": round(t_gu * 1e6, 3), "down_us": round(t_dn * 1e6, 3)},
        "batched": batched,
        "configs": configs,
        "mxfp4_prefill": prefill,
        "roofline": {"bound": "hbm", "kernel": "k_gate_up_rows<FmtInt4, 3, 1, 1> (T=1 gate/up GEMV + GLU)",
                     "achieved": round(gu_bytes / t_gu / 1e9, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_bytes / t_gu / 1e9 / HBM_PEAK_GBS, 4), "traffic": GU_T1_TRAFFIC_BYTES,
                     "launch_us": round(t_gu * 1e6, 3), "algorithmic_bytes_per_launch": gu_bytes},
        "cpu_baseline": cpu,
        "cpu_points": cpu_points,
    }
    print(json.dumps(out), flush=True)
    copy_calibrate(dev, args.copy_calibrate)


def run_batched(dev, layers, sh, args, points=None, routes_b=None):
    """BASELINE config 3 over the seeded Qwen3 layers: T = 16, 32, 64 with uniform and Zipf(1.1) routing (the Zipf
    skew is a per-expert router bias); `points` limits it to some (T, dist) pairs."""
    from moelab_amd import router
    from moelab_amd.problem import baseline_x, zipf_bias
    out = {}
    for T in (16, 32, 64):
        for dist in ("uniform", "zipf"):
            if points is not None and (T, dist) not in points:
                continue
            xT = baseline_x(T, sh.d, seed=T, device=dev)
            bias = torch.from_numpy(zipf_bias(sh.E, 1.1, seed=3)).to(dev) if dist == "zipf" else None
            routes = [router.route(xT, ly["wr"], sh.k, bias=bias) for ly in layers]
            if routes_b is not None:
                routes_b[(T, dist)] = (xT, routes)
            out.setdefault(f"T{T}", {})[dist] = r = time_batched(layers, xT, routes, T, sh, args, bias=bias)
            log(f"T={T} {dist}: grouped {r['us_per_layer_grouped']:.1f} us/layer "
                f"({r['weight_GBps_grouped']:.0f} GB/s), per-slot {r['us_per_layer_per_slot']:.1f} us/layer, "
                f"speedup {r['speedup_per_token']:.2f}x, U={r['unique_experts_mean']:.1f}; with router "
                f"{r['with_router']['us_per_layer']:.1f} us/layer (router then experts as two calls "
                f"{r['with_router']['route_then_experts_us']:.1f})")
    return out


def routed_times(layers, x, k, args, bias=None, norm=True, scale=1.0, act=0):
    """The residual chain with the router inside each layer call (moe_layer_run: the router's launches, which also
    group the slots, then the expert launches), and the same layers as two calls each (router.route, then the experts
    call on its ids, which groups the slots itself): seconds per layer of each. Every layer routes and computes from
    the fixed x and adds to the running sum (y <- y + moe_l(x)), so the routing is the one the expert-only chains use
    and the layers stay dependent."""
    from moelab_amd import router
    from moelab_amd.experts import run_layer, run_routed
    steps, warm = max(5, args.steps // 5), max(2, args.warmup // 5)

    def one_call():
        y = x.clone()
        for ly in layers:
            y, _, _ = run_routed(ly, x, ly["wr"], k, bias=bias, norm=norm, scale=scale, act=act, residual=y)
        return y

    def two_calls():
        y = x.clone()
        for ly in layers:
            idx, wts = router.route(x, ly["wr"], k, bias=bias, norm=norm, scale=scale)
            y = run_layer(ly, x, idx, wts, act=act, residual=y)
        return y
    res = []
    for fn in (one_call, two_calls):
        if fn is two_calls and getattr(args, "routed_only", False):
            res.append(float("nan"))
            continue
        g, _ = graph_of(fn)
        res.append(time_graph(g, steps, warm) / len(layers))
        del g
    return res


def time_batched(layers, x, routes, T, sh, args, bias=None):
    """One BASELINE config 3 point: the 48-layer residual chain on the grouped path and on the per-slot path
    (graph replays), plus the grouped path's two stages timed alone (x fixed: timing only), and the chain with the
    router inside each layer call."""
    from moelab_amd import _lib, roofline
    from moelab_amd.experts import run_experts
    L = len(layers)
    per_expert = roofline.expert_bytes(sh.d, sh.f, "int4")
    U = [int(torch.unique(r[0]).numel()) for r in routes]
    steps, warm = max(5, args.steps // 5), max(2, args.warmup // 5)

    def chain(path):
        def f():
            y = x.clone()
            for ly, (idx, wts) in zip(layers, routes):
                y = run_experts(ly, y, idx, wts, path=path, residual=y)
            return y
        return f

    def stage(st):
        def f():
            for ly, (idx, wts) in zip(layers, routes):
                run_experts(ly, x, idx, wts, path=_lib.PATH_GROUPED, stages=st)
        return f
    res = {}
    for name, fn in (("grouped", chain(_lib.PATH_GROUPED)), ("per_slot", chain(_lib.PATH_SLOTS)),
                     ("gate_up", stage(_lib.STAGE_GATE_UP)), ("down", stage(_lib.STAGE_DOWN))):
        if getattr(args, "routed_only", False):
            res[name] = float("nan")
            continue
        g, _ = graph_of(fn)
        res[name] = time_graph(g, steps, warm)
        del g
    t_one, t_two = routed_times(layers, x, sh.k, args, bias=bias)
    ub = sum(U) * per_expert
    return {
        "T": T,
        "us_per_layer_grouped": round(res["grouped"] * 1e6 / L, 2),
        "us_per_layer_per_slot": round(res["per_slot"] * 1e6 / L, 2),
        "speedup_per_token": round(res["per_slot"] / res["grouped"], 3),
        "tokens_per_s_grouped": round(T * L / res["grouped"], 1),
        "unique_experts_mean": round(float(np.mean(U)), 2),
        "weight_GBps_grouped": round(ub / res["grouped"] / 1e9, 1),
        "slot_weight_GBps_per_slot": round(L * T * sh.k * per_expert / res["per_slot"] / 1e9, 1),
        # stage split of the grouped path: gate/up (2/3 of the bytes), then down + combine (1/3)
        "gate_up_stage_us": round(res["gate_up"] * 1e6 / L, 2),
        "down_stage_us": round(res["down"] * 1e6 / L, 2),
        "gate_up_stage_GBps": round(ub * 2 / 3 / res["gate_up"] / 1e9, 1),
        "down_stage_GBps": round(ub / 3 / res["down"] / 1e9, 1),
        # router inside the layer call: one router launch (logits, tail, grouping), then the expert launches
        "with_router": {"us_per_layer": round(t_one * 1e6, 2), "weight_GBps": round(ub / L / t_one / 1e9, 1),
                        "route_then_experts_us": round(t_two * 1e6, 2)},
    }


def copy_calibrate(dev, mib):
    """3 plain device copies of `mib` MiB: the reference dispatch for FETCH_SIZE / WRITE_SIZE scaling."""
    if mib <= 0:
        return
    n = mib << 20
    a = torch.empty(n, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    log(f"copy calibration: 3 device copies of {n} bytes")


def other_configs(dev, args, only=None, extra=None):
    """BASELINE configs 4 (gpt-oss-20b MXFP4 + biases, clamped SwiGLU, T=1 and T=32), 5a (Mixtral-8x7B int4,
    T=512, MFMA-bound) and 5b (DeepSeek-V2-Lite int4, T=256, 2 shared experts): dependent residual chains of
    seeded layers (enough of them to exceed the 256 MB Infinity Cache), uniform router logits, timed like the
    headline. Reported beside `value`."""
    from moelab_amd import _lib, roofline, router
    from moelab_amd.experts import make_state, merge_shared, run_layer
    from moelab_amd import formats
    from moelab_amd.problem import baseline_int4_layer, baseline_mxfp4_layer, baseline_x
    from moelab_amd.shapes import SHAPES
    out = {}

    def chain_time(layers, x, routes, act):
        def f():
            y = x.clone()
            for ly, (idx, wts) in zip(layers, routes):
                y = run_layer(ly, y, idx, wts, act=act, residual=y)
            return y
        g, _ = graph_of(f)
        t = time_graph(g, max(5, args.steps // 5), max(2, args.warmup // 5))
        del g
        return t

    def report(name, sh, fmt, layers, T, act, shared_f=0, bias_bytes=0.0, into=None, with_router=True):
        x = baseline_x(T, sh.d, seed=T, device=dev)
        routes = [router.route(x, ly["wr"], sh.k) for ly in layers]
        U = [int(torch.unique(r[0]).numel()) for r in routes]
        t = float("nan") if args.routed_only else chain_time(layers, x, routes, act) / len(layers)
        t_one = t_two = None
        if with_router:
            t_one, t_two = routed_times(layers, x, sh.k, args, act=act)
        per_e = roofline.expert_bytes(sh.d, sh.f, fmt) + bias_bytes
        wb = np.mean(U) * per_e + (roofline.expert_bytes(sh.d, shared_f, fmt) if shared_f else 0.0)
        fl = 6.0 * sh.d * sh.f * T * sh.k + 6.0 * sh.d * shared_f * T
        hbm_floor = wb / (HBM_PEAK_GBS * 1e9)
        mfma_floor = fl / 2.5e15
        r = {"T": T, "us_per_layer": round(t * 1e6, 2), "tokens_per_s": round(T / t, 1),
             "unique_experts_mean": round(float(np.mean(U)), 2), "weight_MB_per_layer": round(wb / 1e6, 2),
             "weight_GBps": round(wb / t / 1e9, 1), "TFLOPs": round(fl / t / 1e12, 2),
             "bound": "mfma" if mfma_floor > hbm_floor else "hbm",
             "frac_of_roofline": round(max(hbm_floor, mfma_floor) / t, 4), "layers": len(layers)}
        if with_router:   # one router launch (logits, tail, grouping) then the expert launches
            r["with_router"] = {"us_per_layer": round(t_one * 1e6, 2), "route_then_experts_us": round(t_two * 1e6, 2)}
        (out if into is None else into)[name] = r
        log(f"{name}: {r}")

    def want(*names):
        return only is None or any(n in only for n in names)

    # config 3 points by name, for profiling runs (`--only-configs qwen3_int4_T32_zipf`); the bench line runs them all
    pts = {(T, dist) for T in (16, 32, 64) for dist in ("uniform", "zipf")
           if only is not None and f"qwen3_int4_T{T}_{dist}" in only}
    if pts:
        sh = SHAPES["qwen3-30b-a3b"]
        layers = [baseline_int4_layer(sh, seed=1000 + l, device=dev) for l in range(args.layers)]
        from moelab_amd.experts import reserve
        reserve(layers[0], 64, sh.k)
        router.reserve(dev, 64)
        out["batched"] = run_batched(dev, layers, sh, args, points=pts)
        del layers
        torch.cuda.empty_cache()

    # config 4: gpt-oss-20b MXFP4, biases, clamped SwiGLU (act 2), softmax over the top-4
    if want("gptoss20b_mxfp4_T1", "gptoss20b_mxfp4_T32"):
        sh = SHAPES["gpt-oss-20b"]
        layers = [baseline_mxfp4_layer(sh, seed=2000 + l, device=dev) for l in range(8)]
        bias_b = 2 * (2 * sh.f + sh.d)   # bf16 gate/up/down biases per expert
        for T in (1, 32):
            if want(f"gptoss20b_mxfp4_T{T}"):
                report(f"gptoss20b_mxfp4_T{T}", sh, "mxfp4", layers, T, 2, bias_bytes=bias_b)
        # beside the configs (not a BASELINE config): the same layers at a prefill size, where the MXFP4 tiles
        # run on the block-scaled MFMA (64 slots per expert: the dense tiles)
        if extra is not None:
            report("gptoss20b_mxfp4_T512", sh, "mxfp4", layers, 512, 2, bias_bytes=bias_b, into=extra,
                   with_router=False)
        del layers
        torch.cuda.empty_cache()
    # config 5a: Mixtral-8x7B int4 T=512
    if want("mixtral8x7b_int4_T512"):
        sh = SHAPES["mixtral-8x7b"]
        layers = [baseline_int4_layer(sh, seed=3000 + l, device=dev) for l in range(2)]
        report("mixtral8x7b_int4_T512", sh, "int4", layers, 512, 0)
        del layers
        torch.cuda.empty_cache()
    # config 5b: DeepSeek-V2-Lite int4 T=256, routed top-6 of 64 plus 2 shared experts (F=1408 each)
    if not want("dsv2lite_int4_T256_shared2"):
        return out
    sh = SHAPES["deepseek-v2-lite"]
    layers = []
    for l in range(8):
        ly = baseline_int4_layer(sh, seed=4000 + l, device=dev)
        g = torch.Generator(device=dev).manual_seed(4100 + l)
        ly["shared"] = make_state("int4", *(formats.random_int4(sh.shared, n, k, generator=g, device=dev)
                                            for n, k in ((sh.f, sh.d), (sh.f, sh.d), (sh.d, sh.f))))
        layers.append(merge_shared(ly))   # shared experts as experts 64, 65: one call per layer
        del ly
    report("dsv2lite_int4_T256_shared2", sh, "int4", layers, 256, 0, shared_f=sh.shared * sh.f)
    del layers
    torch.cuda.empty_cache()
    return out


def cpu_baseline(layers, routes, x, sh):
    """torch_loop (the reference's CPU torch path) on fp32 dense weights of the selected experts only: the
    bench line's cpu_baseline, at T=1 on the first layers of the GPU chain."""
    r = cpu_point(layers, routes, x, sh, "T=1", 10.0)
    dt = r["value"] * 1e-6
    r["unit"] = "us/layer (T=1, expert path)"
    r["weight_GBps_equiv"] = round(sh.k * roofline_bytes(sh) / dt / 1e9, 2)
    return r


def cpu_point(layers, routes, x, sh, what, budget_s, fmt="int4", act=0):
    """torch_loop (the reference's CPU torch path) on fp32 dense copies of the selected experts (int4 or MXFP4, with
    the state's additive biases when it has them; act 2: gpt-oss's clamped SwiGLU): a residual chain over `layers`,
    repeated for about budget_s seconds; microseconds per layer-call."""
    from moelab_amd import formats
    from moelab_amd.experts import unpack
    orc = __graft_entry__.load_oracle()
    xs = x.float().cpu()
    dense = []
    for ly, (idx, wts) in zip(layers, routes):
        sel = sorted(set(idx.flatten().tolist()))
        w = {}
        for n in ("g", "u", "d"):
            p = unpack(ly, n)
            deq = (lambda e: formats.dequant_int4(p[0][e], p[1][e], p[2][e])) if fmt == "int4" else \
                (lambda e: formats.dequant_mxfp4(p[0][e], p[1][e]))
            w[n] = {e: deq(e).float().cpu() for e in sel}
        b = {n: {e: ly[n][e].float().cpu() for e in sel} for n in ("bg", "bu", "bd") if n in ly}
        dense.append((w, b, idx.cpu().long(), wts.cpu()))

    def once():
        y = xs
        for w, b, idx, wts in dense:
            y = y + orc.torch_loop(w["g"], w["u"], w["d"], y, idx, wts, act=act, bg=b.get("bg"), bu=b.get("bu"),
                                   bd=b.get("bd"))
        return y
    once()
    t0 = time.perf_counter()
    reps = 0
    while time.perf_counter() - t0 < budget_s and reps < 2000:
        once()
        reps += 1
    dt = (time.perf_counter() - t0) / reps / len(dense)
    T = x.shape[0]
    return {"value": round(dt * 1e6, 1), "unit": "us/layer", "tokens_per_s": round(T / dt, 1),
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{len(dense)} {sh.name} {fmt} layer(s) at {what} (T={T}, k={sh.k}, selected experts "
                      f"dequantised to fp32{', biases, clamped SwiGLU' if act == 2 else ''}), {reps} reps, "
                      f"~{budget_s:.0f} s"}


def cpu_large_points(dev):
    """BASELINE configs 4, 5a and 5b on the CPU torch path, on bounded samples: config 4 (gpt-oss-20b MXFP4, biases,
    clamped SwiGLU) at T=1 and T=32 through one seeded layer; 5a and 5b on the first 32 tokens of the T=512 / T=256
    batch (uniform router logits) through one seeded layer, 5b's routed experts only (the shared experts are two
    dense SwiGLU MLPs on every token, left out of this sample). Reported per layer-call and tokens/s."""
    from moelab_amd import router
    from moelab_amd.problem import baseline_int4_layer, baseline_mxfp4_layer, baseline_x
    from moelab_amd.shapes import SHAPES
    out = {}
    sh = SHAPES["gpt-oss-20b"]
    ly = baseline_mxfp4_layer(sh, seed=2000, device=dev)
    for T in (1, 32):
        x = baseline_x(T, sh.d, seed=T, device=dev)
        out[f"gptoss20b_mxfp4_T{T}"] = cpu_point([ly], [router.route(x, ly["wr"], sh.k)], x, sh, f"T={T}", 3.0,
                                                 fmt="mxfp4", act=2)
    del ly
    torch.cuda.empty_cache()
    for key, name, T in (("mixtral8x7b_int4_T512_32tok", "mixtral-8x7b", 512),
                         ("dsv2lite_int4_T256_32tok_routed", "deepseek-v2-lite", 256)):
        sh = SHAPES[name]
        ly = baseline_int4_layer(sh, seed=3000, device=dev)
        x = baseline_x(T, sh.d, seed=T, device=dev)[:32].contiguous()
        out[key] = cpu_point([ly], [router.route(x, ly["wr"], sh.k)], x, sh, f"a 32-token sample of T={T}", 3.0)
        del ly
        torch.cuda.empty_cache()
    return out


def roofline_bytes(sh):
    from moelab_amd import roofline
    return roofline.expert_bytes(sh.d, sh.f, "int4")


if __name__ == "__main__":
    main()
