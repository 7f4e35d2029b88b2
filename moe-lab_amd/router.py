"""Fused router on gfx950: logits [T, E] -> top-k ids [T, k] int32 + weights [T, k] fp32.

Mirrors reference moelab/router.py (semantics :1-12, ``topk_norm`` :71-80):
  * norm=True: weights = softmax over the top-k logits (= the renormalised full softmax);
    norm=False: the full-softmax probabilities of the chosen experts (DeepSeek-V2 greedy);
  * ties: the lowest expert id wins; NaN logits count as -inf; with fewer than k finite logits the
    remaining slots take the lowest unused ids with weight 0;
  * E <= 1024, k <= min(E, 32).
``route`` adds what the reference leaves to the stock gate GEMV (reference e2e.py:57-59): the logits
x . Wr^T (+ bias) are computed in the same kernel, in fp32, in one fixed reduction order, so a CPU
restatement reproduces them bit for bit and the chosen ids are exact.
"""
import torch

from . import _lib


def topk_norm(logits, k, norm=True, scale=1.0):
    """logits [..., E] (fp32, bf16 or fp16, on the GPU) -> (idx [T, k] int32, wts [T, k] fp32)."""
    E = logits.shape[-1]
    assert E <= 1024 and k <= min(E, 32), (E, k)
    _lib.require_device(logits, "logits")
    lg = logits.reshape(-1, E).contiguous()
    T = lg.shape[0]
    if lg.dtype not in _lib.DTYPE:
        lg = lg.float()
    idx = torch.empty((T, k), dtype=torch.int32, device=lg.device)
    wts = torch.empty((T, k), dtype=torch.float32, device=lg.device)
    rc = _lib.lib().moe_topk(_lib.ptr(lg), _lib.DTYPE[lg.dtype], T, E, k, int(bool(norm)), float(scale),
                             _lib.ptr(idx), _lib.ptr(wts), _lib.stream_of(lg.device))
    _lib.check("moe_topk", rc)
    return idx, wts


def reserve(device, T):
    """Nothing to size: the router's launches need no scratch of their own (kept for callers that size every buffer
    before capturing a HIP graph)."""
    return None


def route(x, wr, k, bias=None, norm=True, scale=1.0, return_logits=False):
    """Gate GEMV, then the router tails (two launches). x [T, d] bf16, wr [E, d] bf16, bias [E] (any float) or None.
    Returns (idx [T, k] int32, wts [T, k] fp32[, logits [T, E] fp32])."""
    _lib.require_device(x, "x")
    assert x.dtype == torch.bfloat16 and wr.dtype == torch.bfloat16, "router takes bf16 x and Wr"
    T, d = x.shape
    E = wr.shape[0]
    assert wr.shape[1] == d and E <= 1024 and 1 <= k <= min(E, 32), (x.shape, wr.shape, k)
    x = x.contiguous()
    wr = wr.contiguous()
    b = None if bias is None else bias.to(torch.float32).contiguous()
    logits = torch.empty((T, E), dtype=torch.float32, device=x.device)
    idx = torch.empty((T, k), dtype=torch.int32, device=x.device)
    wts = torch.empty((T, k), dtype=torch.float32, device=x.device)
    rc = _lib.lib().moe_router(_lib.ptr(x), _lib.ptr(wr), _lib.ptr(b), T, d, E, k, int(bool(norm)), float(scale),
                               _lib.ptr(logits), _lib.ptr(idx), _lib.ptr(wts), None, _lib.stream_of(x.device))
    _lib.check("moe_router", rc)
    return (idx, wts, logits) if return_logits else (idx, wts)


def route_group(x, wr, k, bias=None, norm=True, scale=1.0):
    """route() plus the stable slot grouping, built by the router's own launches (moe_router_group: after the logits
    launch, the launch that runs the tails sorts the T*k slots by expert with a wave prefix sum of the counts).
    Returns (idx, wts, logits, (counts [E], offsets [E+1], sorted [T*k], active [E], meta [2])), the grouping as
    group(idx, E) returns it."""
    _lib.require_device(x, "x")
    assert x.dtype == torch.bfloat16 and wr.dtype == torch.bfloat16, "router takes bf16 x and Wr"
    T, d = x.shape
    E = wr.shape[0]
    assert wr.shape[1] == d and E <= 1024 and 1 <= k <= min(E, 32), (x.shape, wr.shape, k)
    L = _lib.lib()
    x = x.contiguous()
    wr = wr.contiguous()
    b = None if bias is None else bias.to(torch.float32).contiguous()
    dev = x.device
    logits = torch.empty((T, E), dtype=torch.float32, device=dev)
    idx = torch.empty((T, k), dtype=torch.int32, device=dev)
    wts = torch.empty((T, k), dtype=torch.float32, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    srt = torch.empty(max(T * k, 1), dtype=torch.int32, device=dev)
    active = torch.empty(E, dtype=torch.int32, device=dev)
    meta = torch.empty(2, dtype=torch.int32, device=dev)
    rc = L.moe_router_group(_lib.ptr(x), _lib.ptr(wr), _lib.ptr(b), T, d, E, k, int(bool(norm)), float(scale),
                            _lib.ptr(logits), _lib.ptr(idx), _lib.ptr(wts), _lib.ptr(counts), _lib.ptr(offsets),
                            _lib.ptr(srt), _lib.ptr(active), _lib.ptr(meta), _lib.stream_of(dev))
    _lib.check("moe_router_group", rc)
    return idx, wts, logits, (counts, offsets, srt[:T * k], active, meta)


def group(idx, E):
    """Stable slot grouping on the GPU: returns (counts [E], offsets [E+1], sorted [T*k], active [E], meta [2])."""
    _lib.require_device(idx, "idx")
    flat = idx.reshape(-1).to(torch.int32).contiguous()
    n = flat.numel()
    dev = flat.device
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    srt = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    active = torch.empty(E, dtype=torch.int32, device=dev)
    meta = torch.empty(2, dtype=torch.int32, device=dev)
    rc = _lib.lib().moe_group(_lib.ptr(flat), n, E, _lib.ptr(counts), _lib.ptr(offsets), _lib.ptr(srt),
                              _lib.ptr(active), _lib.ptr(meta), _lib.stream_of(dev))
    _lib.check("moe_group", rc)
    return counts, offsets, srt[:n], active, meta
