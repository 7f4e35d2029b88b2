"""torch-ROCm harness the gfx950 variants drop under.

The reference's harness names are kept so a variant and its callers move over unchanged (reference
moelab/torch_backend.py:1-126, moelab/mlx_backend.py:21-163): ``load_variant``, ``make_weights``,
``make_inputs``, ``reference``, ``errors``, ``TOL``, ``time_chained``, ``bench_variant``. The bodies are this
build's own:
  * inputs are drawn on the device (weights) or from one numpy stream (activations, routing through
    ``problem.make_routing``);
  * ``reference`` sorts the slots by expert once and walks contiguous segments, with the GLU kind and the
    gpt-oss biases built in;
  * ``errors`` reports the north-star gate (max |y - y_ref| / RMS(y_ref)) beside the relative Frobenius error;
  * timing captures the whole dependent chain x <- x + run(x) in one HIP graph and times its replays with HIP
    events on the replaying stream (an eagerly launched chain is host-bound on ROCm).
"""
import importlib
import importlib.util
import os
import platform

import numpy as np
import torch

from . import roofline
from .problem import make_routing

DEVICE = "cuda" if torch.cuda.is_available() else "cpu"
DTYPES = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}
# rel-Fro pass thresholds by activation dtype (the reference harness's table, mlx_backend.py:163)
TOL = {"float32": 1e-4, "float16": 5e-3, "bfloat16": 1e-2}
NORTH_STAR_GATE = 1e-2   # max |y - y_ref| <= 1e-2 RMS(y_ref)


def env_info():
    info = {"device": DEVICE, "torch": torch.__version__, "python": platform.python_version()}
    if DEVICE == "cuda":
        p = torch.cuda.get_device_properties(0)
        info.update(gpu=p.name, arch=getattr(p, "gcnArchName", ""), hip=torch.version.hip)
    return info


def load_variant(path):
    """A variant module by file path (the reference loads variants by path, mlx_backend.py:21-25). This
    package's own variants (variants/*.py, relative imports) load as package modules; any other file loads on
    its own."""
    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "variants")
    if os.path.dirname(os.path.abspath(path)) == here:
        return importlib.import_module(f"{__package__}.variants.{os.path.splitext(os.path.basename(path))[0]}")
    spec = importlib.util.spec_from_file_location(f"variant_{abs(hash(path))}", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


# ------------------------------------------------------------------------------------------ inputs
def make_weights(shape, dtype="bfloat16", seed=0):
    """Dense expert weights drawn on the device, N(0, 1 / fan_in) per projection: gate and up [E, F, d]
    (fan-in d), down [E, d, F] (fan-in F), cast to `dtype` (what a variant's prepare() quantises)."""
    gen = torch.Generator(device=DEVICE).manual_seed(int(seed))
    out = []
    for rows, fan_in in ((shape.f, shape.d), (shape.f, shape.d), (shape.d, shape.f)):
        w = torch.empty((shape.E, rows, fan_in), device=DEVICE, dtype=torch.float32)
        out.append(w.normal_(0.0, fan_in ** -0.5, generator=gen).to(DTYPES[dtype]))
    return tuple(out)


def make_inputs(shape, T, dtype="bfloat16", routing="uniform", seed=0):
    """(x [T, d], idx [T, k] int32, wts [T, k] fp32) on the device from one numpy stream: x ~ N(0, 1), then
    the routing of problem.make_routing (uniform, zipf, one_hot) from the same stream. seed: an int or a sequence
    of ints (numpy's seed sequence)."""
    rng = np.random.default_rng(seed if isinstance(seed, (list, tuple)) else int(seed))
    x = rng.standard_normal((T, shape.d), dtype=np.float32)
    idx, wts = make_routing(T, shape.E, shape.k, routing, rng)
    dev = lambda a: torch.as_tensor(a).to(DEVICE)  # noqa: E731
    return dev(x).to(DTYPES[dtype]), dev(np.ascontiguousarray(idx, np.int32)), dev(np.ascontiguousarray(wts, np.float32))


# --------------------------------------------------------------------------------------- reference
_ACTS = {
    0: lambda g, u: torch.nn.functional.silu(g) * u,
    1: lambda g, u: torch.nn.functional.gelu(g, approximate="tanh") * u,
    2: lambda g, u: (lambda gc: gc * torch.sigmoid(1.702 * gc))(g.clamp(max=7.0)) * (u.clamp(-7.0, 7.0) + 1.0),
}


@torch.no_grad()
def reference(wg, wu, wd, x, idx, wts, act=0, bg=None, bu=None, bd=None):
    """fp32 layer on dense (dequantised) weights, the check every variant is held to (reference
    torch_backend.py:58-67; the gpt-oss biases and clamped SwiGLU of metal_mxfp4_gptoss.py:110-126).
    The T*k slots are sorted by expert once (stable), then each expert's contiguous segment of slots is
    gathered, projected and scattered back with its routing weight. Slots with ids outside [0, E) contribute
    nothing, as in the library."""
    x32 = x.float()
    T, k = idx.shape
    E = wg.shape[0]
    flat = idx.reshape(-1).long()
    # slots with ids outside [0, E) add nothing (the library's contract): they sort after every expert's segment
    key = torch.where((flat >= 0) & (flat < E), flat, torch.full_like(flat, E))
    order = torch.argsort(key, stable=True)
    counts = torch.bincount(key, minlength=E + 1)[:E].tolist()
    w_slot = wts.reshape(-1).float()[order]
    tok = order // k
    y = torch.zeros_like(x32)
    glu = _ACTS[int(act)]
    start = 0
    for e, c in enumerate(counts):
        if c == 0:
            continue
        seg = slice(start, start + c)
        start += c
        xe = x32.index_select(0, tok[seg])
        g = torch.mm(xe, wg[e].float().t())
        u = torch.mm(xe, wu[e].float().t())
        if bg is not None:
            g = g + bg[e].float()
            u = u + bu[e].float()
        o = torch.mm(glu(g, u), wd[e].float().t())
        if bd is not None:
            o = o + bd[e].float()
        y.index_add_(0, tok[seg], o * w_slot[seg].unsqueeze(1))
    return y


@torch.no_grad()
def errors(y, y_ref):
    """Deviation of y from y_ref, in fp64: the north-star ratio max |y - y_ref| / RMS(y_ref) (`max_over_rms`),
    its two parts, the relative Frobenius error the reference's harness gates on, and whether y is finite."""
    a = y.double()
    r = y_ref.double().to(a.device)
    diff = (a - r).abs()
    rms = float(r.square().mean().sqrt()) if r.numel() else 0.0
    mx = float(diff.max()) if diff.numel() else 0.0
    return {"max_abs": mx, "rms_ref": rms, "max_over_rms": mx / rms if rms > 0 else float("inf") * (mx > 0),
            "rel_fro": float(torch.linalg.vector_norm(a - r) / (torch.linalg.vector_norm(r) + 1e-30)),
            "finite": bool(torch.isfinite(a).all())}


# ------------------------------------------------------------------------------------------ timing
def capture(fn):
    """fn() captured in a HIP graph. fn runs once eagerly on the capture stream first, so any allocation or
    workspace growth happens outside the graph. Returns (graph, the captured call's output)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def replay_seconds(graph, reps, warmup=1):
    """Seconds of each of `reps` replays of a captured graph: HIP events recorded on the current stream just before
    and just after the replay (a replay is stream-ordered: every node of the graph, including work captured from
    other streams, which capture joins back to this one, ends before the second event)."""
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    out = np.empty(reps)
    st = torch.cuda.current_stream()
    for i in range(reps):
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(st)
        graph.replay()
        t1.record(st)
        t1.synchronize()
        out[i] = t0.elapsed_time(t1) * 1e-3
    return out


def chain_of(fn, inputs, chain):
    """A function running `chain` dependent calls x <- x + fn(x, idx, wts) over the (x, idx, wts) windows
    `inputs` (window i % len(inputs) for call i), returning the last x."""
    def run():
        x = inputs[0][0]
        for i in range(chain):
            _, idx, wts = inputs[i % len(inputs)]
            x = x + fn(x, idx, wts).to(x.dtype)
        return x
    return run


def time_chained(fn, inputs, reps, chain=10, eager=False):
    """Seconds per call of fn(x, idx, wts) in a chain of `chain` dependent calls x <- x + fn(x, idx, wts) over the
    (x, idx, wts) windows `inputs`, one value per repetition. The chain is one HIP graph replayed `reps` times
    (eager=True launches it from the host each time instead; on a CPU device always)."""
    run = chain_of(fn, inputs, chain)
    if DEVICE == "cuda" and not eager:
        g, _ = capture(run)
        per = replay_seconds(g, reps) / chain
        del g
        return per
    import time
    run()
    if DEVICE == "cuda":
        torch.cuda.synchronize()
    per = np.empty(reps)
    for i in range(reps):
        t0 = time.perf_counter()
        run()
        if DEVICE == "cuda":
            torch.cuda.synchronize()
        per[i] = (time.perf_counter() - t0) / chain
    return per


@torch.no_grad()
def bench_variant(mod, shape, tokens, dtype="bfloat16", routing="uniform", hw="mi355x", iters=30, n_rot=3,
                  check=True, weights=None, emit=print):
    """Check and time a variant at each T in `tokens`; emits one record per T:
    {"variant", "shape", "T", "dtype", "routing", "time_us": {"p20", "median", "p80"}, "unique_experts",
     "weight_GBps", "TFLOPs", "floor_us", "frac_of_floor", "check": errors(...) + {"pass"}}.
    Weights are quantised once by mod.prepare; the reference runs on mod.dequant(state) when the variant has
    it (the quantised weights the kernels see), else on the dense weights."""
    dense = weights if weights is not None else make_weights(shape, dtype)
    state = mod.prepare(*dense)
    ref_w = mod.dequant(state) if hasattr(mod, "dequant") else dense
    w_bits = getattr(mod, "W_BITS", 16)
    for T in tokens:
        windows = [make_inputs(shape, T, dtype, routing, seed=1000 * T + s) for s in range(n_rot)]
        rec = {"variant": mod.META["name"], "shape": getattr(shape, "name", ""), "T": T, "dtype": dtype,
               "routing": routing}
        if check:
            x, idx, wts = windows[0]
            err = errors(mod.run(state, x, idx, wts), reference(*ref_w, x, idx, wts))
            err["pass"] = err["finite"] and err["rel_fro"] < TOL[dtype]
            rec["check"] = err
        per = time_chained(lambda *z: mod.run(state, *z), windows, reps=max(5, iters // 3))
        med = float(np.median(per))
        U = float(np.mean([float(w[1].unique().numel()) for w in windows]))
        floor = roofline.floor_time_s(T, shape.d, shape.f, shape.E, shape.k, hw, w_bits, unique=U)
        rec.update({"time_us": {"p20": float(np.percentile(per, 20)) * 1e6, "median": med * 1e6,
                                "p80": float(np.percentile(per, 80)) * 1e6},
                    "unique_experts": U,
                    "weight_GBps": roofline.bytes_moved(T, shape.d, shape.f, shape.E, shape.k, w_bits,
                                                        unique=U) / med / 1e9,
                    "TFLOPs": roofline.flops(T, shape.d, shape.f, shape.k) / med / 1e12,
                    "floor_us": floor * 1e6, "frac_of_floor": floor / med})
        emit(rec)
