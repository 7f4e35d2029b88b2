"""GPU contention guard for timing runs on ROCm (reference moelab/guard.py:1-80).

Every timing run brackets itself with a read-bandwidth probe; the lowest probe of the run is compared with
this machine's history:
    reference = 90th percentile of the last N_HISTORY probes recorded under the same device key,
    status    = "contended" if min(probes) < THRESH * reference, else "ok";
    fewer than MIN_HISTORY probes in the history -> "calibrating" (no verdict yet).
The probe streams a 512 MiB buffer (twice the MI355X's 256 MB memory-side cache, so it measures HBM and not the
cache) with this library's read kernel (moe_probe_read: 16-byte loads, nothing else), median of 9 launches timed by
HIP events. The device key is the GPU's
name, gfx target and compute-unit count plus the host name (reference guard.py keys by chip and power source).
The history is JSON at $MOELAB_AMD_PROBE_HISTORY, else ~/.cache/moelab_amd/hw_probe.json.
"""
import ctypes
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
    """GB/s of this library's streaming-read probe (moe_probe_read: 16-byte loads, the expert kernels' weight-load
    pattern) over n_bytes on cuda:0, median of `reps` launches timed by HIP events on the current stream."""
    import torch
    from . import _lib
    L = _lib.lib()
    buf = torch.full((n_bytes,), 0x5A, dtype=torch.uint8, device="cuda")
    sink = torch.empty(_lib.PROBE_SINK, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream()

    def launch():
        _lib.check("moe_probe_read", L.moe_probe_read(_lib.ptr(buf), n_bytes, _lib.ptr(sink),
                                                      ctypes.c_void_p(st.cuda_stream)))
    launch()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        launch()
        e1.record(st)
        e1.synchronize()
        ts.append(e0.elapsed_time(e1) / 1e3)
    del buf, sink
    return float(n_bytes / np.median(ts) / 1e9)


class ProbeHistory:
    """Probe readings per device key, kept as JSON {key: [GB/s, ...]} (newest last, at most N_HISTORY each)."""

    def __init__(self, path=None):
        self.path = path or history_path()
        try:
            with open(self.path) as f:
                data = json.load(f)
        except (OSError, ValueError):
            data = {}
        # a key holding anything but a list of numbers (an older single-value format) starts afresh
        self.data = {k: [float(x) for x in v] for k, v in data.items()
                     if isinstance(v, list) and all(isinstance(x, (int, float)) for x in v)}

    def readings(self, device_key):
        return self.data.get(device_key, [])

    def record(self, device_key, probes):
        self.data[device_key] = (self.readings(device_key) + [float(p) for p in probes])[-N_HISTORY:]
        os.makedirs(os.path.dirname(os.path.abspath(self.path)), exist_ok=True)
        tmp = self.path + ".tmp"
        with open(tmp, "w") as f:
            json.dump(self.data, f, indent=1)
        os.replace(tmp, self.path)


def verdict(probes, update=True, path=None, device_key=None):
    """Judge this run's probes against the device's history (read before this run's probes are added):
    the run's weakest probe against the 90th percentile of the stored readings. Returns
    {"key", "probe_ref_gbs", "probe_min_gbs", "probe_ratio", "status", "contended", "history"}."""
    dk = device_key or key()
    store = ProbeHistory(path)
    past = store.readings(dk)
    weakest = min(float(p) for p in probes)
    calibrating = len(past) < MIN_HISTORY
    ref = max(float(p) for p in probes) if calibrating else float(np.percentile(np.asarray(past), 90))
    status = "calibrating" if calibrating else ("contended" if weakest < THRESH * ref else "ok")
    if update:
        store.record(dk, probes)
    return {"key": dk, "probe_ref_gbs": ref, "probe_min_gbs": weakest, "probe_ratio": weakest / ref,
            "status": status, "contended": status == "contended", "history": len(past)}


_STATUS_TEXT = {
    "ok": "no contention seen",
    "calibrating": "history too short ({history} of {need} probes): no verdict yet",
    "contended": "contended: another job shared the GPU, absolute timings are not trustworthy; rerun on an idle GPU",
}


def report(v):
    """One line for a verdict."""
    note = _STATUS_TEXT[v["status"]].format(history=v["history"], need=MIN_HISTORY)
    return (f"[guard {v['status']}] weakest probe {v['probe_min_gbs']:.0f} GB/s = {100 * v['probe_ratio']:.0f}% of "
            f"the reference {v['probe_ref_gbs']:.0f} GB/s on {v['key']}: {note}")
