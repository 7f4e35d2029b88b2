"""Host side of the expert path: packed-weight state, the C-ABI call, workspace handling.

A state is a plain dict, as in the reference variants (reference metal_q4_moe.py:32-35,
metal_mxfp4_gptoss.py:100-107):
    "g", "u", "d": (codes, scales, biases) for int4 g64, (codes, scales) for MXFP4
                   gate/up codes [E, F, d/8], down codes [E, d, F/8] (int32 words)
    "bg", "bu", "bd": optional fp32 additive biases [E, F], [E, F], [E, d] (gpt-oss)
    "fmt": "int4" | "mxfp4"
"""
import torch

from . import _lib

FMT = {"int4": _lib.FMT_INT4_G64, "mxfp4": _lib.FMT_MXFP4}


def dims(s):
    codes_g = s["g"][0]
    E, F = codes_g.shape[0], codes_g.shape[1]
    d = s["d"][0].shape[1]
    return E, d, F


def _desc(s):
    """ctypes moe_experts_t for a state (cached; rebuilt if any tensor changed)."""
    tensors = tuple(s["g"]) + tuple(s["u"]) + tuple(s["d"]) + tuple(s.get(b) for b in ("bg", "bu", "bd"))
    key = tuple(0 if t is None else t.data_ptr() for t in tensors)
    c = s.get("_c")
    if c is not None and c[0] == key:
        return c[1]
    E, d, F = dims(s)

    def proj(p, bias):
        codes, scales = p[0], p[1]
        biases = p[2] if len(p) > 2 else None
        for t in (codes, scales, biases, bias):
            if t is not None:
                _lib.require_device(t, "expert weights")
                assert t.is_contiguous(), "expert weights must be contiguous"
        return _lib.Proj(codes.data_ptr(), scales.data_ptr(), None if biases is None else biases.data_ptr(),
                         None if bias is None else bias.data_ptr())

    desc = _lib.Experts(FMT[s.get("fmt", "int4")], E, d, F, proj(s["g"], s.get("bg")), proj(s["u"], s.get("bu")),
                        proj(s["d"], s.get("bd")))
    s["_c"] = (key, desc)
    return desc


def run_experts(s, x, idx, wts, act=0, path=_lib.PATH_AUTO, nored=False, residual=None, out=None, out_dtype=None,
                stages=_lib.STAGE_ALL):
    """y [T, d] (or [T*k, d] unweighted per slot when nored) on the GPU through moe_experts_run.
    out_dtype: x.dtype (default, as the reference) or torch.float32 for the unrounded result;
    residual, if given, is added inside the last kernel and has out_dtype.
    stages: STAGE_ALL, or STAGE_GATE_UP then STAGE_DOWN as two calls sharing the per-device workspace."""
    _lib.require_device(x, "x")
    if x.dtype not in (torch.bfloat16,):
        raise NotImplementedError(f"activation dtype {x.dtype}: the gfx950 expert kernels take bf16")
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
    assert out.dtype == out_dtype and out.dtype in (torch.bfloat16, torch.float32)
    res = None if residual is None else residual.to(out_dtype).contiguous()
    rc = L.moe_experts_run_stages(desc, _lib.ptr(x), _lib.DTYPE[x.dtype], _lib.ptr(idx), _lib.ptr(wts), T, k,
                                  int(act), int(path), int(bool(nored)), _lib.ptr(out), _lib.DTYPE[out.dtype],
                                  _lib.ptr(res), _lib.ptr(ws), ws.numel(), int(stages), _lib.stream_of(x.device))
    _lib.check("moe_experts_run_stages", rc)
    return out
