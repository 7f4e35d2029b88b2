"""torch-ROCm harness the gfx950 variants drop under: fp32 reference, errors, chained timing.

Same contract and outputs as the reference's backends (reference moelab/torch_backend.py:1-126,
moelab/mlx_backend.py:21-163):
    META, prepare(w_gate, w_up, w_down) -> state, run(state, x, idx, wts) -> y, dequant(state)
Timing uses HIP events on the current stream around a chain of dependent calls with a residual
(x_{i+1} = x_i + run(x_i), reference mlx_backend.py:91-117), so host launch cost is excluded the same
way the reference excludes its eval round-trip.
"""
import importlib
import importlib.util
import platform

import numpy as np
import torch

from . import roofline
from .problem import make_routing

DEVICE = "cuda" if torch.cuda.is_available() else "cpu"
DTYPES = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}
TOL = {"float32": 1e-4, "float16": 5e-3, "bfloat16": 1e-2}   # rel-Fro gate (reference mlx_backend.py:163)


def env_info():
    info = {"device": DEVICE, "torch": torch.__version__, "python": platform.python_version()}
    if DEVICE == "cuda":
        p = torch.cuda.get_device_properties(0)
        info.update(gpu=p.name, arch=getattr(p, "gcnArchName", ""), hip=torch.version.hip)
    return info


def load_variant(path):
    """A variant module by file path (reference mlx_backend.py:21-25). This package's own variants
    (variants/*.py, relative imports) load as package modules; any other file loads on its own."""
    import os
    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "variants")
    if os.path.dirname(os.path.abspath(path)) == here:
        return importlib.import_module(f"{__package__}.variants.{os.path.splitext(os.path.basename(path))[0]}")
    spec = importlib.util.spec_from_file_location(f"variant_{abs(hash(path))}", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def make_weights(shape, dtype, seed=0):
    g = torch.Generator(device=DEVICE).manual_seed(seed)
    d, f, E = shape.d, shape.f, shape.E
    mk = lambda *s, sc: (torch.randn(*s, generator=g, device=DEVICE) * sc).to(DTYPES[dtype])  # noqa: E731
    return mk(E, f, d, sc=d ** -0.5), mk(E, f, d, sc=d ** -0.5), mk(E, d, f, sc=f ** -0.5)


def make_inputs(shape, T, dtype, routing, seed):
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.standard_normal((T, shape.d)).astype(np.float32)).to(DEVICE, DTYPES[dtype])
    idx, wts = make_routing(T, shape.E, shape.k, routing, rng)
    return x, torch.from_numpy(idx).to(DEVICE), torch.from_numpy(wts).to(DEVICE)


def glu(g, u, act=0):
    if act == 0:
        return torch.nn.functional.silu(g) * u
    if act == 1:
        return 0.5 * g * (1 + torch.tanh(0.7978845608028654 * (g + 0.044715 * g ** 3))) * u
    g = torch.clamp(g, max=7.0)
    u = torch.clamp(u, -7.0, 7.0)
    return g * torch.sigmoid(1.702 * g) * (u + 1)


@torch.no_grad()
def reference(wg, wu, wd, x, idx, wts, act=0, bg=None, bu=None, bd=None):
    """fp32 per-expert loop on dequantised weights (reference torch_backend.py:58-67, plus the gpt-oss
    biases and activation of metal_mxfp4_gptoss.py:110-126)."""
    x32 = x.float()
    y = torch.zeros_like(x32)
    for e in idx.unique().tolist():
        t, j = (idx == e).nonzero(as_tuple=True)
        xe = x32[t]
        g, u = xe @ wg[e].float().T, xe @ wu[e].float().T
        if bg is not None:
            g, u = g + bg[e].float(), u + bu[e].float()
        o = glu(g, u, act) @ wd[e].float().T
        if bd is not None:
            o = o + bd[e].float()
        y.index_add_(0, t, o * wts[t, j, None].float())
    return y


def errors(y, y_ref):
    diff = y.float() - y_ref
    rms = float(y_ref.pow(2).mean().sqrt().item()) if y_ref.numel() else 0.0
    return {"rel_fro": (diff.norm() / (y_ref.norm() + 1e-30)).item(), "max_abs": diff.abs().max().item(),
            "rms_ref": rms, "finite": bool(torch.isfinite(y).all().item())}


def _sync():
    if DEVICE == "cuda":
        torch.cuda.synchronize()


def time_chained(fn, inputs, reps, chain=10):
    """Chain of `chain` dependent calls x <- x + fn(x) per rep; HIP events on the current stream around
    each chain; returns seconds per call, one value per rep."""
    def once():
        x = inputs[0][0]
        for i in range(chain):
            _, idx, wts = inputs[i % len(inputs)]
            x = x + fn(x, idx, wts).to(x.dtype)
        return x
    once()
    _sync()
    ts = []
    for _ in range(reps):
        if DEVICE == "cuda":
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            once()
            b.record()
            b.synchronize()
            ts.append(a.elapsed_time(b) / 1e3 / chain)
        else:
            import time
            t0 = time.perf_counter()
            once()
            ts.append((time.perf_counter() - t0) / chain)
    return np.array(ts)


@torch.no_grad()
def bench_variant(mod, shape, tokens, dtype="bfloat16", routing="uniform", hw="mi355x", iters=30, n_rot=3,
                  check=True, weights=None, emit=print):
    wg, wu, wd = weights if weights is not None else make_weights(shape, dtype)
    state = mod.prepare(wg, wu, wd)
    rwg, rwu, rwd = mod.dequant(state) if hasattr(mod, "dequant") else (wg, wu, wd)
    w_bits = getattr(mod, "W_BITS", 16)
    for T in tokens:
        inputs = [make_inputs(shape, T, dtype, routing, seed=s) for s in range(n_rot)]
        res = {"type": "result", "variant": mod.META["name"], "T": T}
        if check:
            x, idx, wts = inputs[0]
            res.update(errors(mod.run(state, x, idx, wts), reference(rwg, rwu, rwd, x, idx, wts)))
            res["ok"] = res["finite"] and res["rel_fro"] < TOL[dtype]
        ts = time_chained(lambda *a: mod.run(state, *a), inputs, reps=max(5, iters // 3))
        med = float(np.median(ts))
        U = float(np.mean([i[1].unique().numel() for i in inputs]))
        nbytes = roofline.bytes_moved(T, shape.d, shape.f, shape.E, shape.k, w_bits, unique=U)
        floor = roofline.floor_time_s(T, shape.d, shape.f, shape.E, shape.k, hw, w_bits, unique=U)
        res.update({"median_us": med * 1e6, "p20_us": float(np.percentile(ts, 20)) * 1e6,
                    "p80_us": float(np.percentile(ts, 80)) * 1e6, "unique_experts": U,
                    "gbs": nbytes / med / 1e9, "tflops": roofline.flops(T, shape.d, shape.f, shape.k) / med / 1e12,
                    "floor_us": floor * 1e6, "frac_of_floor": floor / med})
        emit(res)
