"""GPU contention guard for timing runs on ROCm (reference moelab/guard.py:1-80).

Every timing run brackets itself with a read-bandwidth probe; the lowest probe of the run is compared with
this machine's history:
    reference = 90th percentile of the last N_HISTORY probes recorded under the same device key,
    status    = "contended" if min(probes) < THRESH * reference, else "ok";
    fewer than MIN_HISTORY probes in the history -> "calibrating" (no verdict yet).
The probe reads a 512 MiB fp16 buffer (twice the MI355X's 256 MB memory-side cache, so it measures HBM and
not the cache) with a sum reduction, median of 9 calls timed by HIP events. The device key is the GPU's
name, gfx target and compute-unit count plus the host name (reference guard.py keys by chip and power source).
The history is JSON at $MOELAB_AMD_PROBE_HISTORY, else ~/.cache/moelab_amd/hw_probe.json.
"""
import json
import os
import socket

import numpy as np

THRESH, N_HISTORY, MIN_HISTORY = 0.92, 40, 5


def history_path():
    return os.environ.get("MOELAB_AMD_PROBE_HISTORY") or os.path.join(
        os.path.expanduser("~"), ".cache", "moelab_amd", "hw_probe.json")


def key():
    import torch
    if not torch.cuda.is_available():
        return f"cpu|{socket.gethostname()}"
    p = torch.cuda.get_device_properties(0)
    return f"{p.name}|{getattr(p, 'gcnArchName', '')}|{p.multi_processor_count}cu|{socket.gethostname()}"


def probe(n_bytes=1 << 29, reps=9):
    """GB/s of a read-bound fp16 sum over n_bytes on cuda:0 (median of `reps` timed calls)."""
    import torch
    a = torch.rand(n_bytes // 2, device="cuda", dtype=torch.float16)
    a.sum()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        a.sum()
        e1.record()
        e1.synchronize()
        ts.append(e0.elapsed_time(e1) / 1e3)
    del a
    return float(n_bytes / np.median(ts) / 1e9)


def verdict(probes, update=True, path=None, device_key=None):
    path = path or history_path()
    k = device_key or key()
    rec = {}
    if os.path.exists(path):
        with open(path) as f:
            rec = json.load(f)
    hist = rec.get(k, [])
    hist = hist if isinstance(hist, list) else []
    lo = float(min(probes))
    if len(hist) >= MIN_HISTORY:
        ref = float(np.percentile(hist, 90))
        status = "contended" if lo < THRESH * ref else "ok"
    else:
        ref, status = float(max(probes)), "calibrating"
    if update:
        rec[k] = (hist + [float(p) for p in probes])[-N_HISTORY:]
        os.makedirs(os.path.dirname(path) or ".", exist_ok=True)
        with open(path, "w") as f:
            json.dump(rec, f, indent=1)
    return {"key": k, "probe_ref_gbs": ref, "probe_min_gbs": lo, "probe_ratio": lo / ref, "status": status,
            "contended": status == "contended", "history": len(hist)}


def report(v):
    tag = {"ok": "ok",
           "calibrating": f"calibrating ({v['history']} probes in history): verdict not yet meaningful",
           "contended": "CONTENDED: absolute numbers unreliable, re-run without other GPU work"}[v["status"]]
    return (f"guard: probe min {v['probe_min_gbs']:.0f} GB/s vs p90 {v['probe_ref_gbs']:.0f} for {v['key']} "
            f"({100 * v['probe_ratio']:.0f}%) -> {tag}")
