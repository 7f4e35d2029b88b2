"""Host side of the expert path: packed-weight state, the C-ABI call, workspace handling.

A state is a plain dict, as in the reference variants (reference metal_q4_moe.py:32-35,
metal_mxfp4_gptoss.py:100-107), holding the packed row records the library reads:
    "fmt": "int4" | "mxfp4";  "shape": (E, d, F)
    "g", "u": uint8 records [E, F, row_bytes(fmt, d)];  "d": uint8 records [E, d, row_bytes(fmt, F)]
    "bg", "bu", "bd": optional fp32 additive biases [E, F], [E, F], [E, d] (gpt-oss)
    "gt", "ut", "dt": optional uint8 tile-major copies of g, u, d (moe_tiles_pack, built on the device by
                      add_tiles); the grouped T > 1 path streams them when all three are present
"""
import torch

from . import _lib, formats

FMT = {"int4": _lib.FMT_INT4_G64, "mxfp4": _lib.FMT_MXFP4}


def dims(s):
    E, d, F = s["shape"]
    return E, d, F


def make_state(fmt, g, u, d, bg=None, bu=None, bd=None, tiles=True):
    """State from (codes, scales[, biases]) triples in the reference's layout (packed into row records).
    tiles: also build the tile-major copies the grouped path streams (GPU states only; twice the weight
    memory, in exchange for full-bandwidth weight loads at T > 1)."""
    E, F, W = g[0].shape
    s = {"fmt": fmt, "shape": (E, W * 8, F)}
    for n, p in (("g", g), ("u", u), ("d", d)):
        s[n] = formats.pack_rows(fmt, *p)
    for n, b in (("bg", bg), ("bu", bu), ("bd", bd)):
        if b is not None:
            s[n] = b.to(torch.float32).contiguous()
    if tiles and s["g"].is_cuda:
        add_tiles(s)
    return s


def tile_bytes(fmt, N, K):
    """Bytes of one expert's N x K projection in the tile-major layout (include/moe_mi355x.h)."""
    return int(_lib.lib().moe_tile_bytes(FMT[fmt], N, K))


def add_tiles(s):
    """Build s["gt"], s["ut"], s["dt"] from the row records on the device (moe_tiles_pack)."""
    E, d, F = dims(s)
    L = _lib.lib()
    for n, K, N in (("g", d, F), ("u", d, F), ("d", F, d)):
        rows = s[n]
        _lib.require_device(rows, "expert weights")
        nb = tile_bytes(s["fmt"], N, K)
        if nb == 0:
            raise ValueError(f"no tile layout for N={N}, K={K}")
        t = torch.empty(E * nb, dtype=torch.uint8, device=rows.device)
        _lib.check("moe_tiles_pack", L.moe_tiles_pack(FMT[s["fmt"]], E, N, K, _lib.ptr(rows.contiguous()),
                                                      _lib.ptr(t), _lib.stream_of(rows.device)))
        s[n + "t"] = t
    s["_tiles_of"] = tuple(s[n].data_ptr() for n in ("g", "u", "d"))
    return s


def drop_tiles(s):
    """The same state without tile-major copies (the grouped path then reads the row records)."""
    return {k: v for k, v in s.items() if k not in ("gt", "ut", "dt", "_c", "_tiles_of")}


def unpack(s, n):
    """The reference-layout (codes, scales[, biases]) of projection n of a state."""
    E, d, F = dims(s)
    return formats.unpack_rows(s["fmt"], s[n], F if n == "d" else d)


def _desc(s):
    """ctypes moe_experts_t for a state (cached; rebuilt if any tensor changed)."""
    tensors = (s["g"], s["u"], s["d"]) + tuple(s.get(b) for b in ("bg", "bu", "bd", "gt", "ut", "dt"))
    key = tuple(0 if t is None else t.data_ptr() for t in tensors)
    c = s.get("_c")
    if c is not None and c[0] == key:
        return c[1]
    E, d, F = dims(s)
    for n, K, N in (("g", d, F), ("u", d, F), ("d", F, d)):
        assert s[n].dtype == torch.uint8 and tuple(s[n].shape) == (E, N, formats.row_bytes(s["fmt"], K)), n
    if any(n in s for n in ("gt", "ut", "dt")):
        assert s.get("_tiles_of") == tuple(s[n].data_ptr() for n in ("g", "u", "d")), \
            "tile-major copies were built from other row records: call add_tiles(s) again"

    def proj(n, bias):
        rows, tiles = s[n], s.get(n + "t")
        for t in (rows, bias, tiles):
            if t is not None:
                _lib.require_device(t, "expert weights")
                assert t.is_contiguous(), "expert weights must be contiguous"
        if tiles is not None:
            K, N = (F, d) if n == "d" else (d, F)
            assert tiles.dtype == torch.uint8 and tiles.numel() == E * tile_bytes(s["fmt"], N, K), n + "t"
        return _lib.Proj(rows.data_ptr(), None if bias is None else bias.data_ptr(),
                         None if tiles is None else tiles.data_ptr())

    desc = _lib.Experts(FMT[s.get("fmt", "int4")], E, d, F, proj("g", s.get("bg")), proj("u", s.get("bu")),
                        proj("d", s.get("bd")))
    s["_c"] = (key, desc)
    return desc


def run_experts(s, x, idx, wts, act=0, path=_lib.PATH_AUTO, nored=False, residual=None, out=None, out_dtype=None,
                stages=_lib.STAGE_ALL):
    """y [T, d] (or [T*k, d] unweighted per slot when nored) on the GPU through moe_experts_run.
    x: bf16, fp16 or fp32 (fp16 and fp32 reach the gate/up kernels exactly, as 2 or 3 bf16 planes).
    out_dtype: x.dtype (default, as the reference) or another of the three (fp32: the unrounded result);
    residual, if given, is added inside the last kernel and has out_dtype.
    stages: STAGE_ALL, or STAGE_GATE_UP then STAGE_DOWN as two calls sharing the per-device workspace."""
    _lib.require_device(x, "x")
    if x.dtype not in _lib.DTYPE:
        raise TypeError(f"activation dtype {x.dtype}: the expert kernels take bf16, fp16 or fp32")
    T, d = x.shape
    k = idx.shape[1]
    x = x.contiguous()
    idx = idx.to(torch.int32).contiguous()
    wts = wts.to(torch.float32).contiguous()
    desc = _desc(s)
    L = _lib.lib()
    nbytes = L.moe_experts_workspace_bytes(desc, T, k, path)
    ws = _lib.workspace(x.device, nbytes)
    out_dtype = x.dtype if out_dtype is None else out_dtype
    if out is None:
        out = torch.empty((T * k if nored else T, d), dtype=out_dtype, device=x.device)
    assert out.dtype == out_dtype and out.dtype in _lib.DTYPE
    res = None if residual is None else residual.to(out_dtype).contiguous()
    rc = L.moe_experts_run_stages(desc, _lib.ptr(x), _lib.DTYPE[x.dtype], _lib.ptr(idx), _lib.ptr(wts), T, k,
                                  int(act), int(path), int(bool(nored)), _lib.ptr(out), _lib.DTYPE[out.dtype],
                                  _lib.ptr(res), _lib.ptr(ws), ws.numel(), int(stages), _lib.stream_of(x.device))
    _lib.check("moe_experts_run_stages", rc)
    return out


def reserve(s, T, k, device=None):
    """Size the per-device workspace for calls on state s of up to T tokens with k slots each, on either path
    (and the state's shared experts): call it before capturing such calls in a HIP graph. A graph keeps the
    workspace pointer it was captured with; the workspace never moves while it is large enough, and a buffer it
    outgrows is kept alive, but growing it during capture raises."""
    device = torch.device(device or s["g"].device)
    desc = _desc(s)
    L = _lib.lib()
    need = max([int(L.moe_experts_workspace_bytes(desc, t, k, p)) for t in {1, int(T)}
                for p in (_lib.PATH_SLOTS, _lib.PATH_GROUPED)] +
               [int(L.moe_layer_workspace_bytes(desc, t, k)) for t in {1, int(T)}])
    if "shared" in s:
        need = max(need, int(L.moe_shared_experts_workspace_bytes(_desc(s["shared"]), int(T))))
    if "n_shared" in s:
        S = int(s["n_shared"])
        need = max([need] + [int(L.moe_experts_shared_workspace_bytes(desc, S, t, k, p))
                             for t in {1, int(T)} for p in (_lib.PATH_AUTO, _lib.PATH_SLOTS, _lib.PATH_GROUPED)] +
                   [int(L.moe_layer_shared_workspace_bytes(desc, S, t, k)) for t in {1, int(T)}])
    return _lib.workspace(device, need)


def run_routed(s, x, wr, k, bias=None, norm=True, scale=1.0, act=0, residual=None, out=None, out_dtype=None):
    """Router + experts in one call (moe_layer_run): the fused router's logits x . wr^T (+ bias) and tail (the same
    ids as router.route), then the experts on the default path. At T > 1 no launch of its own groups the slots: the
    gate/up wave tiles group them in-kernel (and write the down stage's pass lists) where they run, else the
    router's last workgroup builds the grouping. x [T, d] bf16, wr [E, d] bf16 (E the routed experts).
    A merge_shared state (s["n_shared"]) runs moe_layer_run_shared: its shared experts join every token, weighted by
    sigmoid(x . s["shared_gate"]) or 1. A state with separate shared experts (s["shared"]) adds them by a second call.
    Returns (y [T, d], idx [T, k] int32, wts [T, k] fp32), idx / wts the routed slots."""
    _lib.require_device(x, "x")
    if x.dtype != torch.bfloat16 or wr.dtype != torch.bfloat16:
        raise TypeError("run_routed takes bf16 x and router weights (the gate GEMV reads bf16)")
    T, d = x.shape
    x = x.contiguous()
    wr = wr.contiguous()
    b = None if bias is None else bias.to(torch.float32).contiguous()
    desc = _desc(s)
    L = _lib.lib()
    S = int(s.get("n_shared", 0))
    nbytes = L.moe_layer_shared_workspace_bytes(desc, S, T, k) if S else L.moe_layer_workspace_bytes(desc, T, k)
    ws = _lib.workspace(x.device, nbytes)
    final_dtype = x.dtype if out_dtype is None else out_dtype
    separate_shared = "shared" in s and not S
    user_out = out
    out_dtype = torch.float32 if separate_shared else final_dtype
    if out is None or separate_shared:
        out = torch.empty((T, d), dtype=out_dtype, device=x.device)
    assert out.dtype == out_dtype and out.dtype in _lib.DTYPE
    idx = torch.empty((T, k), dtype=torch.int32, device=x.device)
    wts = torch.empty((T, k), dtype=torch.float32, device=x.device)
    res = None if residual is None else residual.to(out_dtype).contiguous()
    if S:
        g = s.get("shared_gate")
        g = None if g is None else g.to(torch.bfloat16).contiguous()
        rc = L.moe_layer_run_shared(desc, S, _lib.ptr(x), _lib.DTYPE[x.dtype], _lib.ptr(wr), _lib.ptr(b), _lib.ptr(g),
                                    T, k, int(bool(norm)), float(scale), int(act), _lib.ptr(idx), _lib.ptr(wts),
                                    _lib.ptr(out), _lib.DTYPE[out.dtype], _lib.ptr(res), _lib.ptr(ws), ws.numel(),
                                    _lib.stream_of(x.device))
        _lib.check("moe_layer_run_shared", rc)
    else:
        rc = L.moe_layer_run(desc, _lib.ptr(x), _lib.DTYPE[x.dtype], _lib.ptr(wr), _lib.ptr(b), T, k,
                             int(bool(norm)), float(scale), int(act), _lib.ptr(idx), _lib.ptr(wts), _lib.ptr(out),
                             _lib.DTYPE[out.dtype], _lib.ptr(res), _lib.ptr(ws), ws.numel(), _lib.stream_of(x.device))
        _lib.check("moe_layer_run", rc)
    if separate_shared:
        out = run_shared(s["shared"], x, gate=s.get("shared_gate"), act=act, residual=out, out=user_out,
                         out_dtype=final_dtype)
    return out, idx, wts


def run_shared(s, x, gate=None, act=0, residual=None, out=None, out_dtype=None):
    """Shared experts (always on) through moe_shared_experts_run: y = residual + g_t * sum_s expert_s(x_t),
    g_t = sigmoid(x_t . gate) for a bf16 gate vector [d] (Qwen-style gated shared expert, reference
    e2e.py:66-68) or 1 (DeepSeek, e2e.py:146-147). s: an expert state whose E experts are the shared ones."""
    _lib.require_device(x, "x")
    if x.dtype not in _lib.DTYPE:
        raise TypeError(f"activation dtype {x.dtype}: the expert kernels take bf16, fp16 or fp32")
    T, d = x.shape
    x = x.contiguous()
    desc = _desc(s)
    L = _lib.lib()
    ws = _lib.workspace(x.device, L.moe_shared_experts_workspace_bytes(desc, T))
    out_dtype = x.dtype if out_dtype is None else out_dtype
    if out is None:
        out = torch.empty((T, d), dtype=out_dtype, device=x.device)
    assert out.dtype == out_dtype and out.dtype in _lib.DTYPE
    res = None if residual is None else residual.to(out_dtype).contiguous()
    g = None if gate is None else gate.to(torch.bfloat16).contiguous()
    rc = L.moe_shared_experts_run(desc, _lib.ptr(x), _lib.DTYPE[x.dtype], T, int(act), _lib.ptr(g), _lib.ptr(out),
                                  _lib.DTYPE[out.dtype], _lib.ptr(res), _lib.ptr(ws), ws.numel(),
                                  _lib.stream_of(x.device))
    _lib.check("moe_shared_experts_run", rc)
    return out


def merge_shared(s):
    """The state with its shared experts (s["shared"]) appended to the routed ones as experts E .. E + S - 1, for
    one call per layer (moe_experts_run_shared: one grouping, one combine, the shared experts' work inside the
    routed launches). Needs the same format, d and F in both sets; additive biases are concatenated (zeros where a
    set has none). Routed ids keep their meaning. Returns a new state (its weights a copy; s is left as it is)."""
    sh = s["shared"]
    E, d, F = dims(s)
    S, d2, F2 = dims(sh)
    if sh["fmt"] != s["fmt"] or (d2, F2) != (d, F):
        raise ValueError(f"shared experts ({sh['fmt']}, d={d2}, F={F2}) do not match the routed ones "
                         f"({s['fmt']}, d={d}, F={F}): run them with run_shared")
    if S + 1 > 64:
        raise ValueError("at most 63 shared experts")
    m = {k: v for k, v in s.items()
         if k not in ("g", "u", "d", "bg", "bu", "bd", "gt", "ut", "dt", "_c", "_tiles_of", "shared", "shape")}
    m["shape"] = (E + S, d, F)
    for n in ("g", "u", "d"):
        m[n] = torch.cat([s[n], sh[n]], 0).contiguous()
    for b, N in (("bg", F), ("bu", F), ("bd", d)):
        if b in s or b in sh:
            parts = [t[b] if b in t else torch.zeros((n, N), dtype=torch.float32, device=s["g"].device)
                     for t, n in ((s, E), (sh, S))]
            m[b] = torch.cat(parts, 0).contiguous()
    m["n_shared"] = S
    if "gt" in s:
        add_tiles(m)
    return m


def run_experts_shared(s, x, idx, wts, act=0, path=_lib.PATH_AUTO, residual=None, out=None, out_dtype=None):
    """Routed and shared experts of a merge_shared state in one call (moe_experts_run_shared): idx, wts [T, k]
    the routed slots (ids < E - S); every token also takes the S shared experts with weight
    sigmoid(x . s["shared_gate"]) or 1."""
    _lib.require_device(x, "x")
    if x.dtype not in _lib.DTYPE:
        raise TypeError(f"activation dtype {x.dtype}: the expert kernels take bf16, fp16 or fp32")
    T, d = x.shape
    k = int(idx.shape[1])
    S = int(s["n_shared"])
    x = x.contiguous()
    idx = idx.to(torch.int32).contiguous()
    wts = wts.to(torch.float32).contiguous()
    desc = _desc(s)
    L = _lib.lib()
    ws = _lib.workspace(x.device, L.moe_experts_shared_workspace_bytes(desc, S, T, k, int(path)))
    out_dtype = x.dtype if out_dtype is None else out_dtype
    if out is None:
        out = torch.empty((T, d), dtype=out_dtype, device=x.device)
    assert out.dtype == out_dtype and out.dtype in _lib.DTYPE
    res = None if residual is None else residual.to(out_dtype).contiguous()
    g = s.get("shared_gate")
    g = None if g is None else g.to(torch.bfloat16).contiguous()
    rc = L.moe_experts_run_shared(desc, S, _lib.ptr(x), _lib.DTYPE[x.dtype], _lib.ptr(idx), _lib.ptr(wts), T, k,
                                  int(act), int(path), _lib.ptr(g), _lib.ptr(out), _lib.DTYPE[out.dtype],
                                  _lib.ptr(res), _lib.ptr(ws), ws.numel(), _lib.stream_of(x.device))
    _lib.check("moe_experts_run_shared", rc)
    return out


def run_layer(s, x, idx, wts, act=0, path=_lib.PATH_AUTO, residual=None, out_dtype=None):
    """Routed experts, then the state's shared experts if it has them (s["shared"], optional
    s["shared_gate"]): the routed sum stays fp32 until the shared call adds to it. A merge_shared state runs
    both in one call."""
    if "n_shared" in s:
        return run_experts_shared(s, x, idx, wts, act=act, path=path, residual=residual, out_dtype=out_dtype)
    if "shared" not in s:
        return run_experts(s, x, idx, wts, act=act, path=path, residual=residual, out_dtype=out_dtype)
    y = run_experts(s, x, idx, wts, act=act, path=path, residual=residual, out_dtype=torch.float32)
    return run_shared(s["shared"], x, gate=s.get("shared_gate"), act=act, residual=y,
                      out_dtype=x.dtype if out_dtype is None else out_dtype)

