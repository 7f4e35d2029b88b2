"""Seeded inputs: the reference's problem generator and the BASELINE layer configurations.

Kernel contract (reference moelab/problem.py:3-10):
    y = moe(x, w_gate, w_up, w_down, idx, wts)
    x [T, d]; w_gate, w_up [E, f, d]; w_down [E, d, f] (out, in); idx [T, k] int32; wts [T, k] float
    y [T, d] = sum_j wts[t, j] * down_e(act(gate_e x_t) * up_e x_t),  e = idx[t, j]

``make_routing`` / ``make_problem`` restate reference problem.py:15-64 with the same numpy Generator
calls in the same order, so a seed gives the same problem as the reference harness. The recorded
routing traces (reference runs/*.npz) are not part of this repository; mode="trace" takes a path.

The BASELINE generators build packed layers directly on the device (no dense weights):
int4 g64: uniform codes, bf16 scales ~U(0.005, 0.02), biases = -8 * scale;
MXFP4: uniform E2M1 codes, E8M0 byte = 127 + U{-8..-4}, bf16 biases ~N(0, 0.01) (gpt-oss);
router weight bf16 ~N(0, 0.02); x bf16 ~N(0, 1); Zipf(s) popularity as a per-expert router bias.
"""
import numpy as np
import torch

from . import formats


def make_routing(T, E, k, mode="uniform", rng=None, zipf_a=1.2, trace_path=None):
    rng = rng or np.random.default_rng(0)
    if mode == "uniform":
        logits = rng.standard_normal((T, E))
    elif mode == "zipf":  # skewed popularity: a per-expert logit offset over a random permutation
        pop = 1.0 / np.arange(1, E + 1) ** zipf_a
        logits = rng.standard_normal((T, E)) + np.log(pop)[rng.permutation(E)] * 2.0
    elif mode == "one_hot":  # every token to the same k experts (worst imbalance)
        logits = np.tile(np.arange(E, 0, -1, dtype=np.float64), (T, 1))
    elif mode == "trace":
        return _trace_routing(T, E, k, rng, trace_path)
    else:
        raise ValueError(mode)
    idx = np.argsort(-logits, axis=1)[:, :k].astype(np.int32)
    top = np.take_along_axis(logits, idx, axis=1)
    w = np.exp(top - top.max(1, keepdims=True))
    w = (w / w.sum(1, keepdims=True)).astype(np.float32)
    return idx, w


def _trace_routing(T, E, k, rng, path):
    """Windows of T consecutive tokens from a recorded trace npz (arrays [layers, tokens, k] + 'E')."""
    if path is None:
        raise ValueError("routing='trace' needs trace_path (recorded traces are not shipped)")
    z = np.load(path)
    tr = [z[n] for n in z.files if n != "E"]
    assert int(z["E"]) == E and tr[0].shape[2] == k, "trace recorded for another E/k"
    t = tr[rng.integers(len(tr))]
    layer, start = rng.integers(t.shape[0]), rng.integers(t.shape[1] - T)
    idx = t[layer, start:start + T].astype(np.int32)
    w = rng.random((T, k)).astype(np.float32)
    return idx, w / w.sum(1, keepdims=True)


def make_problem(shape, T, routing="uniform", seed=0):
    rng = np.random.default_rng(seed)
    d, f, E, k = shape.d, shape.f, shape.E, shape.k
    s_in, s_hid = 1.0 / np.sqrt(d), 1.0 / np.sqrt(f)
    p = {
        "x": rng.standard_normal((T, d)).astype(np.float32),
        "w_gate": (rng.standard_normal((E, f, d)) * s_in).astype(np.float32),
        "w_up": (rng.standard_normal((E, f, d)) * s_in).astype(np.float32),
        "w_down": (rng.standard_normal((E, d, f)) * s_hid).astype(np.float32),
    }
    p["idx"], p["wts"] = make_routing(T, E, k, routing, rng)
    return p


# ------------------------------------------------------------------------------- BASELINE layers
def zipf_bias(E, s=1.1, seed=0):
    """Per-expert router logit offset 2*log(r^-s) over a random permutation (Zipf(s) popularity)."""
    rng = np.random.default_rng(seed)
    pop = 1.0 / np.arange(1, E + 1) ** s
    return (np.log(pop)[rng.permutation(E)] * 2.0).astype(np.float32)


def baseline_int4_layer(shape, seed, device, router=True):
    """One BASELINE int4 g64 SwiGLU layer (an expert state plus "wr"), generated packed on the device."""
    from .experts import make_state
    g = torch.Generator(device=device).manual_seed(int(seed))
    E, d, F = shape.E, shape.d, shape.f
    layer = make_state("int4", formats.random_int4(E, F, d, generator=g, device=device),
                       formats.random_int4(E, F, d, generator=g, device=device),
                       formats.random_int4(E, d, F, generator=g, device=device))
    if router:
        layer["wr"] = (torch.randn((E, d), generator=g, device=device) * 0.02).to(torch.bfloat16)
    return layer


def baseline_mxfp4_layer(shape, seed, device, biases=True, router=True):
    """One BASELINE MXFP4 layer (gpt-oss: per-expert bf16 biases ~N(0, 0.01), kept as fp32 in the state
    like reference metal_mxfp4_gptoss.py:105)."""
    from .experts import make_state
    g = torch.Generator(device=device).manual_seed(int(seed))
    E, d, F = shape.E, shape.d, shape.f
    layer = make_state("mxfp4", formats.random_mxfp4(E, F, d, generator=g, device=device),
                       formats.random_mxfp4(E, F, d, generator=g, device=device),
                       formats.random_mxfp4(E, d, F, generator=g, device=device))
    if biases:
        for n, rows in (("bg", F), ("bu", F), ("bd", d)):
            b = (torch.randn((E, rows), generator=g, device=device) * 0.01).to(torch.bfloat16)
            layer[n] = b.to(torch.float32)
    if router:
        layer["wr"] = (torch.randn((E, d), generator=g, device=device) * 0.02).to(torch.bfloat16)
    return layer


def baseline_x(T, d, seed, device):
    g = torch.Generator(device=device).manual_seed(int(seed) + 7919)
    return torch.randn((T, d), generator=g, device=device).to(torch.bfloat16)
