"""CPU oracle for the quantised MoE-layer hot path (numpy fp64 + the C router in moe_oracle.c).

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
may import this module, and only as the checker (or the timed CPU baseline). The product package
never imports it; its GPU path fails loudly when the HIP library is missing.

What each function restates (reference file:line) and what pins it (tests/test_oracle.py):
  bf16 helpers          IEEE round-to-nearest-even truncation of fp32      pinned: torch's bf16 cast
  unpack_int4           reference metal_q4_decode_v4.py:57-64 (low nibble first)
                                                                            pinned: hand-packed words
  dequant_int4          w = s*q + b per 64-group (metal_q4_decode_v4.py:36-65)
                                                                            pinned: known answers
  dequant_mxfp4         e2m1 * 2^(s-127) (metal_mxfp4_moe.py:1-41)      pinned: OCP E2M1 table,
                                                                            powers of two
  router_logits (C)     gate GEMV, fixed fp32 order                         pinned: fp64 dot bound
  topk (C)              router.py:15-66                                     pinned: stable argsort,
                                                                            known answers, brute force
  topk_closed_form      stable argsort(-v) + softmax over the top-k (router.py:5-6)
  group                 stable sort by expert (triton_fused_moe.py:56-70; tiles_v2.py:362-373)
                                                                            pinned: brute-force ranks
  moe_reference         fp64 per-expert loop (problem.py:73-85, mlx_backend.py:48-65,
                        metal_mxfp4_gptoss.py:110-126)                     pinned: per-token loop,
                                                                            linearity, zero rows
  torch_loop            the reference's CPU torch path (variants/cuda/torch_loop.py:11-17); timed
                        as the CPU baseline
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def lib():
    """The compiled C half of the oracle (oracle/libmoe_oracle.so, built by oracle/Makefile)."""
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "libmoe_oracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library missing: {path} (run `make -C oracle`)")
        L = ctypes.CDLL(path)
        L.oracle_router_logits.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int] * 3 + [ctypes.c_void_p]
        L.oracle_router_logits.restype = ctypes.c_int
        L.oracle_topk.argtypes = [ctypes.c_void_p] + [ctypes.c_int] * 4 + [ctypes.c_float] + [ctypes.c_void_p] * 2
        L.oracle_topk.restype = ctypes.c_int
        _LIB = L
    return _LIB


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


# ------------------------------------------------------------------------------------------ bf16
def f32_to_bf16_bits(a):
    """fp32 -> bf16 bit patterns (uint16), round to nearest even; NaN stays NaN."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = np.isnan(np.asarray(a, dtype=np.float32))
    out = np.where(nan, (u >> 16) | 0x40, rounded)
    return out.astype(np.uint16)


def bf16_bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(a):
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


# --------------------------------------------------------------------------------------- formats
def unpack_int4(words):
    """uint32/int32 words [..., K/8] -> codes [..., K] (uint8); nibble i of word j is element 8j+i."""
    w = np.asarray(words).astype(np.int64) & 0xFFFFFFFF
    q = np.empty(w.shape + (8,), dtype=np.uint8)
    for i in range(8):
        q[..., i] = (w >> (4 * i)) & 0xF
    return q.reshape(*w.shape[:-1], w.shape[-1] * 8)


def dequant_int4(words, scales_bits, biases_bits, group=64):
    """Affine int4: w = scale * q + bias, scale/bias per `group` elements (bf16 bit patterns)."""
    q = unpack_int4(words).astype(np.float64)
    *lead, K = q.shape
    s = bf16_bits_to_f32(scales_bits).astype(np.float64)
    b = bf16_bits_to_f32(biases_bits).astype(np.float64)
    q = q.reshape(*lead, K // group, group)
    return (q * s[..., None] + b[..., None]).reshape(*lead, K)


E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])


def e8m0_scale(s):
    """E8M0 byte -> the fp32 whose bits are s << 23: 2^(s-127) for s in 1..254, 0 for s = 0."""
    return (np.asarray(s, dtype=np.uint32) << 23).view(np.float32)


def dequant_mxfp4(words, scale_bytes, group=32):
    q = unpack_int4(words)
    v = E2M1[q]
    *lead, K = v.shape
    s = e8m0_scale(scale_bytes).astype(np.float64)
    return (v.reshape(*lead, K // group, group) * s[..., None]).reshape(*lead, K)


# ---------------------------------------------------------------------------------------- router
def router_logits(x_bits, wr_bits, bias=None):
    """x_bits [T, d] uint16 (bf16), wr_bits [E, d] uint16 -> fp32 logits [T, E] in the GPU's order."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    wr_bits = np.ascontiguousarray(wr_bits, dtype=np.uint16)
    T, d = x_bits.shape
    E = wr_bits.shape[0]
    out = np.empty((T, E), dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    rc = lib().oracle_router_logits(_ptr(x_bits), _ptr(wr_bits), None if b is None else _ptr(b), T, d, E, _ptr(out))
    if rc != 0:
        raise ValueError(f"oracle_router_logits: rc={rc}")
    return out


def topk(logits, k, norm=True, scale=1.0):
    """Router tail on fp32 logits [T, E] -> (idx [T, k] int32, wts [T, k] fp32)."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = lg.shape
    idx = np.empty((T, k), dtype=np.int32)
    wts = np.empty((T, k), dtype=np.float32)
    rc = lib().oracle_topk(_ptr(lg), T, E, k, int(bool(norm)), float(scale), _ptr(idx), _ptr(wts))
    if rc != 0:
        raise ValueError(f"oracle_topk: rc={rc}")
    return idx, wts


def topk_closed_form(logits, k, norm=True):
    """Same contract in closed form: ids = stable argsort of -v (v = logits with NaN -> -inf);
    weights = softmax over the chosen logits (norm) or the full-softmax probabilities (not norm)."""
    v = np.where(np.isnan(logits), -np.inf, logits).astype(np.float64)
    idx = np.argsort(-v, axis=1, kind="stable")[:, :k].astype(np.int32)
    top = np.take_along_axis(v, idx, axis=1)
    with np.errstate(invalid="ignore", divide="ignore"):
        if norm:
            w = np.exp(top - top[:, :1])
            w = w / w.sum(1, keepdims=True)
        else:
            m = v.max(1, keepdims=True)
            w = np.exp(top - m) / np.where(np.isfinite(v), np.exp(v - m), 0.0).sum(1, keepdims=True)
    return idx, w


# -------------------------------------------------------------------------------------- grouping
def group(idx, E):
    """Slot -> expert grouping. Slots are flat ids p = t*k + j. Returns
    counts [E], offsets [E+1] (exclusive scan), sorted_slots [T*k] (ascending p within each expert),
    active [U] (experts with count > 0, ascending)."""
    flat = np.asarray(idx, dtype=np.int64).reshape(-1)
    order = np.argsort(flat, kind="stable").astype(np.int32)
    counts = np.bincount(flat, minlength=E).astype(np.int32)
    offsets = np.zeros(E + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    active = np.nonzero(counts)[0].astype(np.int32)
    return counts, offsets, order, active


# ------------------------------------------------------------------------------- expert compute
def act_fn(g, u, act):
    """act 0: silu(g)*u (SwiGLU); 1: tanh-GELU(g)*u (GeGLU, reference mlx_backend.py:61);
    2: gpt-oss clamped SwiGLU g=min(g,7), u=clip(u,-7,7), g*sigmoid(1.702 g)*(u+1)
    (reference metal_mxfp4_gptoss.py:36-43, 119-121)."""
    if act == 0:
        return g / (1.0 + np.exp(-g)) * u
    if act == 1:
        return 0.5 * g * (1.0 + np.tanh(0.7978845608028654 * (g + 0.044715 * g ** 3))) * u
    if act == 2:
        g = np.minimum(g, 7.0)
        u = np.clip(u, -7.0, 7.0)
        return g / (1.0 + np.exp(-1.702 * g)) * (u + 1.0)
    raise ValueError(act)


def moe_reference(x, wg, wu, wd, idx, wts, act=0, bg=None, bu=None, bd=None, shared=None, shared_gate=None):
    """fp64 per-expert loop. x [T, d]; wg/wu: callables e -> [F, d] (or arrays [E, F, d]); wd: e -> [d, F].
    bg/bu [E, F], bd [E, d]: optional additive biases (gpt-oss), bd inside the routing weight.
    shared: optional list of (wg_s [Fs, d], wu_s, wd_s) always-on SwiGLU experts, added with weight 1, or with
    weight sigmoid(x_t . shared_gate) per token when shared_gate [d] is given (Qwen-style gated shared expert,
    reference e2e.py:66-68; DeepSeek adds them ungated, e2e.py:146-147).
    Returns y [T, d] float64."""
    get = lambda w, e: w(e) if callable(w) else w[e]  # noqa: E731
    x = np.asarray(x, dtype=np.float64)
    idx = np.asarray(idx)
    T, d = x.shape
    y = np.zeros((T, d))
    for e in np.unique(idx):
        t, j = np.nonzero(idx == e)
        xe = x[t]
        g = xe @ np.asarray(get(wg, e), dtype=np.float64).T
        u = xe @ np.asarray(get(wu, e), dtype=np.float64).T
        if bg is not None:
            g = g + np.asarray(bg[e], dtype=np.float64)
            u = u + np.asarray(bu[e], dtype=np.float64)
        h = act_fn(g, u, act)
        o = h @ np.asarray(get(wd, e), dtype=np.float64).T
        if bd is not None:
            o = o + np.asarray(bd[e], dtype=np.float64)
        np.add.at(y, t, o * np.asarray(wts, dtype=np.float64)[t, j][:, None])
    gs = np.ones((T, 1)) if shared_gate is None else \
        1.0 / (1.0 + np.exp(-(x @ np.asarray(shared_gate, dtype=np.float64))))[:, None]
    for (sg, su, sd) in (shared or []):
        g = x @ np.asarray(sg, dtype=np.float64).T
        u = x @ np.asarray(su, dtype=np.float64).T
        y += gs * ((g / (1.0 + np.exp(-g)) * u) @ np.asarray(sd, dtype=np.float64).T)
    return y


def moe_reference_per_token(x, wg, wu, wd, idx, wts, act=0):
    """The same layer token by token (the form of reference fp32_truth_q4.py:8-20): an independent
    formulation used to pin moe_reference."""
    x = np.asarray(x, dtype=np.float64)
    T, d = x.shape
    y = np.zeros((T, d))
    for t in range(T):
        for j, e in enumerate(np.asarray(idx)[t]):
            h = act_fn(np.asarray(wg[e], np.float64) @ x[t], np.asarray(wu[e], np.float64) @ x[t], act)
            y[t] += float(wts[t][j]) * (np.asarray(wd[e], np.float64) @ h)
    return y


def error_metrics(y, y_ref):
    """rel-Fro, max-abs, cos, finite (reference problem.py:88-98) plus RMS of the reference."""
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(y_ref, dtype=np.float64)
    diff = y - r
    nr = np.linalg.norm(r) + 1e-30
    return {
        "rel_fro": float(np.linalg.norm(diff) / nr),
        "max_abs": float(np.abs(diff).max()) if diff.size else 0.0,
        "rms_ref": float(np.sqrt(np.mean(r * r))) if r.size else 0.0,
        "cos": float((y * r).sum() / (np.linalg.norm(y) * nr + 1e-30)),
        "finite": bool(np.isfinite(y).all()),
    }


def torch_loop(wg, wu, wd, x, idx, wts, act=0, bg=None, bu=None, bd=None):
    """The reference's eager CPU torch path (variants/cuda/torch_loop.py:11-17) on dense weights:
    per unique expert, gather its (token, slot) pairs, two matmuls, the GLU, down matmul, index_add.
    act 0 is the reference's SiLU GLU; act 2 with the optional biases bg, bu [E, F], bd [E, d] is the gpt-oss
    expert of the reference's fp32 truth (metal_mxfp4_gptoss.py:110-126: biases added to the gate/up products,
    g = min(g, 7), u = clip(u, -7, 7), g sigmoid(1.702 g) (u + 1), the down bias inside the routing weight);
    act 1 is the tanh-GELU GLU. wg, wu, wd, bg, bu, bd may be dicts {expert: tensor}."""
    import torch
    y = torch.zeros_like(x)
    for e in idx.unique().tolist():
        t, j = (idx == e).nonzero(as_tuple=True)
        xe = x[t]
        g, u = xe @ wg[e].T, xe @ wu[e].T
        if bg is not None:
            g, u = g + bg[e], u + bu[e]
        if act == 0:
            h = torch.nn.functional.silu(g) * u
        elif act == 1:
            h = torch.nn.functional.gelu(g, approximate="tanh") * u
        else:
            g, u = g.clamp(max=7.0), u.clamp(-7.0, 7.0)
            h = g * torch.sigmoid(1.702 * g) * (u + 1.0)
        o = h @ wd[e].T
        if bd is not None:
            o = o + bd[e]
        y.index_add_(0, t, o * wts[t, j, None].to(x.dtype))
    return y
