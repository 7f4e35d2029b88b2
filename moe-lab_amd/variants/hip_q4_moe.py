"""Production dispatcher, int4 affine g64 MoE experts on MI355X (gfx950 HIP kernels).

Same variant contract and dispatch shape as the reference's production int4 dispatcher
(reference moelab/variants/mlx/metal_q4_moe.py:1-64):
    T == 1                  -> per-slot GEMV, two launches: gate+up+GLU for the k slots, then down +
                               k-reduction
    T > 1, custom_wins(...) -> grouped expert tiles: each selected expert's rows are read once and
                               applied to all of its slots (group, gate/up, down, combine)
    otherwise               -> gather_moe (module attribute, monkeypatchable like the reference's); on
                               MI355X the small loads (fallback.grouped_from_load)
prepare / dequant keep the reference's state layout (mx.quantize affine, group 64), so `dequant(state)`
gives the weights the fp32 reference uses. reserve(state, T, k) sizes the per-device workspace before a caller
captures calls in a HIP graph (graphs keep the workspace pointer they were captured with).
"""
import torch

from .. import _lib, formats
from ..experts import dims, make_state, reserve, run_experts, run_layer, unpack  # noqa: F401
from ..fallback import gather_moe, grouped_from_load, grouped_wins  # noqa: F401  (gather_moe: tests patch the attribute)

META = {"name": "hip_q4_moe", "description": "gfx950 HIP: per-slot GEMV at T=1, grouped expert tiles at T>1"}
BITS, GS = 4, 64
MODE = "affine"
W_BITS = BITS + 32 / GS


def prepare(w_gate, w_up, w_down):
    """Dense weights gate/up [E, F, d], down [E, d, F] (any float dtype, on the GPU) -> packed state."""
    E, f, d = w_gate.shape
    assert d % 64 == 0 and f % 64 == 0, "d, f must be multiples of 64"
    q = {n: formats.quantize_int4(w.contiguous()) for n, w in (("g", w_gate), ("u", w_up), ("d", w_down))}
    return make_state("int4", q["g"], q["u"], q["d"])


def state_from_packed(g, u, d, bg=None, bu=None, bd=None):
    """State from (codes, scales, biases) triples in the reference's layout, e.g. a checkpoint."""
    return make_state("int4", g, u, d, bg, bu, bd)


def dequant(s):
    return tuple(formats.dequant_int4(*unpack(s, n), group_size=GS) for n in ("g", "u", "d"))


def custom_wins(T, k, E, D, F):
    """Load policy, refitted on MI355X (fallback.grouped_wins; the reference's name and meaning,
    metal_q4_moe.py:42-46: True runs the grouped expert tiles, False the fallback): grouped from a load
    T*k/E of 1.0 (experts below 2.5 Mi weights per projection) or 0.27, the per-slot GEMV below, and near that
    threshold only with enough live gate/up wave tiles to fill the chip."""
    return grouped_wins(T, k, E, D, F)


def run_slots(s, x, idx, act=0):
    """T = 1 per-slot expert outputs [k, D], unweighted (reference metal_q4_moe.py:49-51)."""
    ones = torch.ones(idx.shape, dtype=torch.float32, device=x.device)
    return run_experts(s, x, idx, ones, act=act, path=_lib.PATH_SLOTS, nored=True)


def run(s, x, idx, wts, act=0, residual=None, out_dtype=None):
    """act: 0 = SwiGLU, 1 = GeGLU (tanh-GELU), 2 = gpt-oss clamped SwiGLU. residual: optional [T, D]
    added to the output inside the last kernel (y = residual + moe(x)). out_dtype: x.dtype (default,
    as the reference) or torch.float32 for the unrounded result."""
    T, k = idx.shape
    kw = dict(act=act, residual=residual, out_dtype=out_dtype)
    if T == 1:
        return run_layer(s, x, idx, wts, path=_lib.PATH_AUTO, **kw)
    E, D, F = dims(s)
    if not custom_wins(T, k, E, D, F):
        return gather_moe(s, x, idx, wts, GS, BITS, **kw)
    return run_layer(s, x, idx, wts, path=_lib.PATH_GROUPED, **kw)
