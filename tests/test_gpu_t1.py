"""The T=1 decode path (MOE_PATH_AUTO at T=1: the per-slot gate/up GEMV, then the down GEMV with the k-reduction)
against the oracle, across shapes with k = 1, 2, 3, 4, 6, 8, 16, both formats, biases and the clamped GLU, output
dtypes and a residual; repeated calls and HIP graph replays of a dependent chain must give the same bits (every
reduction runs in a fixed order)."""
import numpy as np
import pytest
import torch

from helpers import assert_close, oracle_y

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

CASES = [
    # (name, fmt, d, F, E, k, act, biases)
    ("qwen3", "int4", 2048, 768, 128, 8, 0, False),
    ("k16", "int4", 1024, 512, 32, 16, 0, False),
    ("gptoss-mxfp4", "mxfp4", 2880, 2880, 32, 4, 2, True),
    ("dsv2", "int4", 2048, 1408, 64, 6, 0, False),
    ("k2-geglu", "int4", 1024, 2048, 8, 2, 1, False),
    ("k1", "int4", 512, 256, 8, 1, 0, False),
    ("k3", "int4", 320, 768, 8, 3, 0, False),
    ("mxfp4-k8", "mxfp4", 512, 512, 16, 8, 0, False),
]


def build(case, seed=1):
    from moelab_amd.problem import baseline_int4_layer, baseline_mxfp4_layer
    from moelab_amd.shapes import MoEShape
    name, fmt, d, F, E, k, act, biases = case
    sh = MoEShape(name, d=d, f=F, E=E, k=k)
    if fmt == "int4":
        s = baseline_int4_layer(sh, seed, DEV, router=False)
    else:
        s = baseline_mxfp4_layer(sh, seed, DEV, biases=biases, router=False)
    return sh, s


def route(sh, seed):
    from moelab_amd.problem import make_routing
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.standard_normal((1, sh.d)).astype(np.float32)).to(DEV, torch.bfloat16)
    idx, wts = make_routing(1, sh.E, sh.k, "uniform", rng)
    return x, torch.from_numpy(idx).to(DEV), torch.from_numpy(wts).to(DEV)


@pytest.mark.parametrize("case", CASES, ids=lambda c: c[0])
def test_t1_matches_oracle_deterministically(case):
    from moelab_amd import _lib
    from moelab_amd.experts import run_experts
    sh, s = build(case)
    act = case[6]
    x, idx, wts = route(sh, seed=7)
    print(f"case t1 {case[0]}", flush=True)
    ref = oracle_y(s, x, idx, wts, act)
    first = None
    for rep in range(3):
        y = run_experts(s, x, idx, wts, act=act, path=_lib.PATH_AUTO, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert_close(y, ref, what=(case[0], rep))
        if first is None:
            first = y.clone()
        assert torch.equal(y, first), (case[0], rep)   # deterministic
    assert torch.equal(run_experts(s, x, idx, wts, act=act, path=_lib.PATH_SLOTS, out_dtype=torch.float32), first)
    for od in (torch.bfloat16, torch.float16):
        yo = run_experts(s, x, idx, wts, act=act, path=_lib.PATH_AUTO, out_dtype=od)
        assert yo.dtype == od
        assert_close(yo, ref, what=(case[0], od))
    res = torch.randn((1, sh.d), device=DEV).to(torch.bfloat16)
    yr = run_experts(s, x, idx, wts, act=act, path=_lib.PATH_AUTO, residual=res)
    assert_close(yr, ref + res.float().cpu().numpy(), what=(case[0], "residual"))


def test_t1_invalid_ids_add_nothing():
    """Slots whose expert id is outside [0, E) contribute nothing (the grouped combine's rule)."""
    from moelab_amd import _lib
    from moelab_amd.experts import run_experts
    sh, s = build(CASES[0])
    x, idx, wts = route(sh, seed=3)
    bad = idx.clone()
    bad[0, 2] = -1
    bad[0, 5] = sh.E + 4
    keep = torch.ones_like(wts)
    keep[0, 2] = keep[0, 5] = 0
    y = run_experts(s, x, bad, wts, path=_lib.PATH_AUTO, out_dtype=torch.float32)
    y_ref = run_experts(s, x, idx, wts * keep, path=_lib.PATH_AUTO, out_dtype=torch.float32)
    torch.cuda.synchronize()
    rms = float(y_ref.pow(2).mean().sqrt())
    assert float((y - y_ref).abs().max()) <= 1e-5 * rms


def test_t1_graph_replays():
    """A chain of 6 dependent layers (x <- x + moe(x)) captured once and replayed 4 times, with eager work and
    fresh allocations between replays: every replay equals the eager chain bit for bit."""
    from moelab_amd import _lib
    from moelab_amd.experts import reserve, run_experts
    from moelab_amd.problem import baseline_int4_layer, baseline_x
    from moelab_amd.shapes import SHAPES
    from moelab_amd.experts import make_state, unpack
    sh = SHAPES["qwen3-30b-a3b"]

    def small(seed):   # scales x0.1: a residual chain of BASELINE-scale layers overflows (h is quadratic in x)
        base = baseline_int4_layer(sh, seed=seed, device=DEV, router=False)
        parts = {n: list(unpack(base, n)) for n in ("g", "u", "d")}
        for n in parts:
            parts[n][1] = (parts[n][1].float() * 0.1).to(torch.bfloat16)
            parts[n][2] = (parts[n][1].float() * -8.0).to(torch.bfloat16)
        return make_state("int4", parts["g"], parts["u"], parts["d"])
    layers = [small(100 + i) for i in range(6)]
    rng = np.random.default_rng(5)
    routes = []
    for _ in layers:
        from moelab_amd.problem import make_routing
        i, w = make_routing(1, sh.E, sh.k, "uniform", rng)
        routes.append((torch.from_numpy(i).to(DEV), torch.from_numpy(w).to(DEV)))
    x0 = baseline_x(1, sh.d, seed=5, device=DEV)
    reserve(layers[0], 1, sh.k)

    def chain():
        x = x0.clone()
        for ly, (i, w) in zip(layers, routes):
            x = run_experts(ly, x, i, w, path=_lib.PATH_AUTO, residual=x)
        return x
    eager = chain()
    torch.cuda.synchronize()
    assert bool(torch.isfinite(eager).all()) and float(eager.float().abs().max()) > 0
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        chain()
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = chain()
    for rep in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep
        junk = torch.randn(1 << 20, device=DEV) * 2   # eager work and an allocation between replays
        del junk
