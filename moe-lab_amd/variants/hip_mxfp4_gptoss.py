"""gpt-oss MXFP4 experts on MI355X: per-expert biases and the clamped SwiGLU.

Same kernels and dispatch as hip_mxfp4_moe, with the differences of reference
moelab/variants/mlx/metal_mxfp4_gptoss.py:1-17:
  * per-expert biases: gate/up bias added before the activation, down bias added before the routing
    weight, y = sum_k w_k * (W_down h + b_down) (reference :8, :110-126);
  * activation: act 1 (the state's "act", default) = gpt-oss clamped SwiGLU, g = min(g, 7),
    u = clip(u, -7, 7), g * sigmoid(1.702 g) * (u + 1) (reference :33-43); act 0 = plain SwiGLU.
    In this library's ABI the clamped form is MOE_ACT_GPTOSS (2) and tanh-GELU is 1.
"""
import torch

from .. import _lib, backend
from . import hip_mxfp4_moe as _b
from ..experts import reserve  # noqa: F401  (workspace sizing before graph capture)

META = {"name": "hip_mxfp4_gptoss",
        "description": "gfx950 HIP MXFP4 + per-expert biases + gpt-oss clamped SwiGLU"}
MODE, GS, BITS, W_BITS = _b.MODE, _b.GS, _b.BITS, _b.W_BITS
ALPHA, LIMIT = 1.702, 7.0
_ACT = {0: _lib.ACT_SWIGLU, 1: _lib.ACT_GPTOSS}


def prepare(w_gate, w_up, w_down):
    s = _b.prepare(w_gate, w_up, w_down)
    E, d, F = s["shape"]
    dev = w_gate.device
    s["bg"] = torch.zeros((E, F), dtype=torch.float32, device=dev)
    s["bu"] = torch.zeros((E, F), dtype=torch.float32, device=dev)
    s["bd"] = torch.zeros((E, d), dtype=torch.float32, device=dev)
    s["act"] = 0   # the lab contract runs plain SwiGLU on prepare()d weights (reference :10)
    return s


def dequant(s):
    return _b.dequant(s)


def state(g, u, d, bg, bu, bd, act=1):
    """run() state from packed gpt-oss projections: (codes, e8m0) pairs and bf16/fp32 biases, kept as fp32
    (reference metal_mxfp4_gptoss.py:100-107)."""
    s = _b.state_from_packed(g, u, d, bg, bu, bd)
    s["act"] = act
    return s


def reference(s, x, idx, wts):
    """fp32 truth on the dequantised weights (reference metal_mxfp4_gptoss.py:110-126)."""
    wg, wu, wd = dequant(s)
    y = backend.reference(wg, wu, wd, x, idx.long(), wts, act=_ACT[s["act"]], bg=s["bg"], bu=s["bu"], bd=s["bd"])
    return y.to(x.dtype)


def run(s, x, idx, wts, residual=None, out_dtype=None):
    return _b.run(s, x, idx, wts, act=_ACT[s.get("act", 1)], residual=residual, out_dtype=out_dtype)
