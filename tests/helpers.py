"""Shared test helpers: move packed GPU states to the CPU oracle, run the oracle reference."""
import numpy as np
import torch

import __graft_entry__

orc = __graft_entry__.load_oracle()

TOL_MAXABS_RMS = 1e-2   # max |y - y_ref| <= 1e-2 * RMS(y_ref)  (fp32 accumulation; h kept at ~16 bits)
BF16_HALF_ULP = 2.0 ** -8   # round-to-nearest into bf16 moves a value by at most 2^-8 of its magnitude
F16_HALF_ULP = 2.0 ** -11   # fp16: 2^-11 (normal range)


def np_u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def np_words(t):
    return t.detach().cpu().contiguous().numpy().view(np.uint32)


def deq(state, name, experts=None):
    """Oracle dequantisation (fp64) of projection `name` of a packed state, optionally only `experts`.
    The records are split back into the reference's (codes, scales[, biases]) layout first."""
    from moelab_amd.experts import unpack
    p = unpack(state, name)
    sel = (lambda t: t) if experts is None else (lambda t: t[experts])  # noqa: E731
    if state["fmt"] == "int4":
        return orc.dequant_int4(np_words(sel(p[0])), np_u16(sel(p[1])), np_u16(sel(p[2])))
    return orc.dequant_mxfp4(np_words(sel(p[0])), sel(p[1]).cpu().numpy())


class LazyExperts:
    """e -> dequantised [N, K] weights of one expert (keeps the oracle's memory bounded at full sizes)."""

    def __init__(self, state, name):
        self.state, self.name = state, name

    def __call__(self, e):
        return deq(self.state, self.name, experts=[int(e)])[0]


def oracle_y(state, x, idx, wts, act=0):
    """The oracle's layer for a packed state; the state's shared experts (state["shared"], optional
    state["shared_gate"]) are added as the oracle's shared list."""
    xs = orc.bf16_bits_to_f32(np_u16(x)) if x.dtype == torch.bfloat16 else x.float().cpu().numpy()
    b = {n: state[n].cpu().numpy().astype(np.float64) for n in ("bg", "bu", "bd") if n in state}
    shared, sgate = None, None
    if "shared" in state:
        sh = state["shared"]
        wg, wu, wd = (deq(sh, n) for n in ("g", "u", "d"))
        shared = [(wg[s], wu[s], wd[s]) for s in range(wg.shape[0])]
        if state.get("shared_gate") is not None:
            sgate = orc.bf16_bits_to_f32(np_u16(state["shared_gate"]))
    return orc.moe_reference(xs, LazyExperts(state, "g"), LazyExperts(state, "u"), LazyExperts(state, "d"),
                             idx.cpu().numpy(), wts.cpu().numpy(), act, b.get("bg"), b.get("bu"), b.get("bd"),
                             shared=shared, shared_gate=sgate)


def assert_close(y, y_ref, tol=TOL_MAXABS_RMS, what=""):
    """fp32 outputs: max |y - y_ref| <= tol * RMS(y_ref) (the north-star gate).
    bf16 / fp16 outputs: the same plus the storage rounding of each element, |y - y_ref| <= tol * RMS + 2^-8 |y_ref|
    (fp16: 2^-11 |y_ref|)
    (a bf16 result cannot be closer to y_ref than its own rounding; for outputs beyond ~4 RMS that rounding
    alone exceeds 1e-2 RMS). The gate on the unrounded fp32 result is tested separately."""
    yv = y.float().cpu().numpy()
    err = orc.error_metrics(yv, y_ref)
    assert err["finite"], (what, err)
    if y.dtype == torch.float32:
        assert err["max_abs"] <= tol * err["rms_ref"] + 1e-30, (what, err)
    else:
        half_ulp = F16_HALF_ULP if y.dtype == torch.float16 else BF16_HALF_ULP
        excess = np.abs(yv - y_ref) - (tol * err["rms_ref"] + half_ulp * np.abs(y_ref))
        assert (excess <= 1e-30).all(), (what, err, float(excess.max()))
    return err
