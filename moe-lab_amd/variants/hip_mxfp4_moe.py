"""MXFP4 MoE experts on MI355X (gfx950 HIP kernels).

Variant contract and dispatch shape of the reference's MXFP4 dispatcher (reference
moelab/variants/mlx/metal_mxfp4_moe.py:440-512): E2M1 codes with one E8M0 scale per 32 inputs,
the scale applied in fp32 per group (exact for every byte 1..254; reference metal_mxfp4_moe.py:33-41);
    T == 1          -> per-slot GEMV, two launches (gate/up/GLU for the k slots, then down + k-reduction)
    T > 1, grouped(...)  -> grouped expert tiles (each selected expert read once)
    otherwise       -> gather_moe (per-slot path), the reference's load-policy fallback (:474-477); on MI355X
                       it takes the small loads (fallback.grouped_from_load), not the large ones
"""
import torch

from .. import _lib, formats
from ..experts import dims, make_state, reserve, run_experts, run_layer, unpack  # noqa: F401
from ..fallback import gather_moe, grouped_from_load, grouped_wins  # noqa: F401  (gather_moe: tests patch the attribute)

META = {"name": "hip_mxfp4_moe", "description": "gfx950 HIP MXFP4: per-slot GEMV at T=1, grouped expert tiles at T>1"}
MODE, GS, BITS = "mxfp4", 32, 4
W_BITS = 4 + 8 / 32

LOAD_MAX = None  # tests set a number to override the policy below (reference metal_mxfp4_moe.py:465)


def load_max(D, F):
    """Grouped tiles up to this load (T*k/E) (reference metal_mxfp4_moe.py:465-471). On MI355X the grouped
    path wins at every high load measured, so there is no upper cut unless LOAD_MAX sets one."""
    return LOAD_MAX if LOAD_MAX is not None else float("inf")


def grouped(T, k, E, D, F):
    """True: grouped tiles; False: the per-slot fallback. With LOAD_MAX set (tests, A/B runs) the reference's
    rule, grouped up to LOAD_MAX; otherwise the MI355X fit (fallback.grouped_wins): grouped from
    fallback.grouped_from_load, near it only with enough live gate/up wave tiles."""
    load = T * k / E
    if LOAD_MAX is not None:
        return load <= LOAD_MAX
    return grouped_wins(T, k, E, D, F)


def prepare(w_gate, w_up, w_down):
    E, f, d = w_gate.shape
    assert d % 64 == 0 and f % 64 == 0, "shape constraints"
    q = {n: formats.quantize_mxfp4(w.contiguous()) for n, w in (("g", w_gate), ("u", w_up), ("d", w_down))}
    return make_state("mxfp4", q["g"], q["u"], q["d"])


def state_from_packed(g, u, d, bg=None, bu=None, bd=None):
    """State from (codes, e8m0 scales) pairs in the reference's layout, optional fp32 biases."""
    return make_state("mxfp4", g, u, d, bg, bu, bd)


def dequant(s):
    return tuple(formats.dequant_mxfp4(*unpack(s, n), group_size=GS) for n in ("g", "u", "d"))


def run(s, x, idx, wts, act=0, residual=None, out_dtype=None):
    T, k = idx.shape
    kw = dict(act=act, residual=residual, out_dtype=out_dtype)
    if T == 1:
        return run_layer(s, x, idx, wts, path=_lib.PATH_AUTO, **kw)
    E, D, F = dims(s)
    if not grouped(T, k, E, D, F):
        return gather_moe(s, x, idx, wts, GS, BITS, MODE, **kw)
    return run_layer(s, x, idx, wts, path=_lib.PATH_GROUPED, **kw)


def run_slots(s, x, idx, act=0):
    ones = torch.ones(idx.shape, dtype=torch.float32, device=x.device)
    return run_experts(s, x, idx, ones, act=act, path=_lib.PATH_SLOTS, nored=True)
