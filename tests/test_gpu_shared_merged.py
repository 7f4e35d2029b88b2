"""Routed and shared experts in one call (moe_experts_run_shared, experts.merge_shared): the shared experts become
experts E .. E + S - 1 of the routed state and every token takes them with weight sigmoid(x . gate) or 1
(reference e2e.py:66-68 Qwen-style gated shared expert, e2e.py:146-147 DeepSeek). Checked against the oracle's
routed + shared sum (computed on the unmerged state) at the north-star gate, against the two-call form
(moe_experts_run then moe_shared_experts_run), at T = 1 (per-slot GEMV over k + S slots) and on the grouped
tiles, both formats, biases on the routed set only, routed ids that fall on a shared expert's id
(they join no group, as in a routed-only call), and the argument checks.
"""
import numpy as np
import pytest
import torch

from helpers import assert_close, oracle_y

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def layer(fmt, d, F, E, k, S, seed, gated=False, biases=False):
    from moelab_amd import formats
    from moelab_amd.experts import make_state
    from moelab_amd.problem import baseline_int4_layer, baseline_mxfp4_layer
    from moelab_amd.shapes import MoEShape
    sh = MoEShape("m", d=d, f=F, E=E, k=k)
    if fmt == "int4":
        s = baseline_int4_layer(sh, seed, DEV, router=False)
    else:
        s = baseline_mxfp4_layer(sh, seed, DEV, biases=biases, router=False)
    g = torch.Generator(device=DEV).manual_seed(seed + 1)
    rnd = formats.random_int4 if fmt == "int4" else formats.random_mxfp4
    s["shared"] = make_state(fmt, rnd(S, F, d, generator=g, device=DEV), rnd(S, F, d, generator=g, device=DEV),
                             rnd(S, d, F, generator=g, device=DEV))
    if gated:
        s["shared_gate"] = (torch.randn(d, generator=g, device=DEV) * 0.05).to(torch.bfloat16)
    return sh, s


def inputs(sh, T, seed, routing="uniform"):
    from moelab_amd.problem import make_routing
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.standard_normal((T, sh.d)).astype(np.float32)).to(DEV, torch.bfloat16)
    idx, wts = make_routing(T, sh.E, sh.k, routing, rng)
    return x, torch.from_numpy(idx).to(DEV), torch.from_numpy(wts).to(DEV)


CASES = [
    # (fmt, d, F, E, k, S, T, routing, gated, biases)
    ("int4", 256, 384, 16, 4, 2, 1, "uniform", False, False),      # T = 1: per-slot GEMV over k + S slots
    ("int4", 256, 384, 16, 4, 2, 7, "uniform", True, False),       # gated shared experts
    ("int4", 512, 384, 32, 6, 2, 64, "zipf", False, False),        # wave tiles, in-kernel grouping
    ("int4", 256, 384, 16, 4, 1, 200, "uniform", True, False),     # 200 tokens on the shared expert
    ("mxfp4", 512, 512, 8, 2, 2, 40, "uniform", False, True),      # routed biases, none on the shared set
    ("mxfp4", 256, 256, 8, 4, 2, 300, "uniform", True, True),      # block-scaled tiles, 32-token passes
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-k{c[4]}S{c[5]}-T{c[6]}-{'g' if c[8] else 'u'}")
def test_merged_shared_against_oracle_and_two_calls(case):
    from moelab_amd.experts import merge_shared, run_layer
    fmt, d, F, E, k, S, T, routing, gated, biases = case
    sh, s = layer(fmt, d, F, E, k, S, seed=600 + T, gated=gated, biases=biases)
    m = merge_shared(s)
    assert m["shape"][0] == E + S and m["n_shared"] == S
    x, idx, wts = inputs(sh, T, seed=T, routing=routing)
    print(f"case merged-shared {case}", flush=True)
    y1 = run_layer(m, x, idx, wts, out_dtype=torch.float32)
    y2 = run_layer(s, x, idx, wts, out_dtype=torch.float32)
    yb = run_layer(m, x, idx, wts)
    torch.cuda.synchronize()
    ref = oracle_y(s, x, idx, wts)
    assert_close(y1, ref, what=("merged", case))
    assert_close(y2, ref, what=("two calls", case))
    assert_close(yb, ref, what=("merged bf16", case))
    assert yb.dtype == torch.bfloat16


def test_merged_routed_ids_on_shared_ids_join_no_group():
    """A routed id equal to a shared expert's id (E) or past it is outside the routed set: it contributes
    nothing, as in a routed-only call, instead of reaching the shared expert."""
    from moelab_amd.experts import merge_shared, run_layer
    sh, s = layer("int4", 256, 384, 16, 4, 2, seed=61)
    m = merge_shared(s)
    x, idx, wts = inputs(sh, 24, seed=61)
    bad = idx.clone()
    bad[2, 1] = sh.E
    bad[9, 3] = sh.E + 1
    bad[20, 0] = -1
    y = run_layer(m, x, bad, wts, out_dtype=torch.float32)
    keep = (bad >= 0) & (bad < sh.E)
    ref = oracle_y(s, x, idx, wts * keep)
    assert_close(y, ref, what="ids on shared ids")


def test_merged_shared_argument_errors():
    from moelab_amd import _lib
    from moelab_amd.experts import _desc, merge_shared
    sh, s = layer("int4", 256, 384, 8, 2, 2, seed=62)
    m = merge_shared(s)
    L = _lib.lib()
    desc = _desc(m)
    x, idx, wts = inputs(sh, 4, seed=62)
    y = torch.empty_like(x)
    ws = _lib.workspace(x.device, L.moe_experts_shared_workspace_bytes(desc, 2, 4, 2, 0))

    def call(S, k, nbytes, path=0):
        return L.moe_experts_run_shared(desc, S, _lib.ptr(x), 0, _lib.ptr(idx), _lib.ptr(wts), 4, k, 0, path, None,
                                        _lib.ptr(y), 0, None, _lib.ptr(ws), nbytes, None)
    assert call(2, 2, ws.numel()) == 0
    assert call(10, 2, ws.numel()) == _lib.MOE_ERR_ARG     # S >= E
    assert call(0, 2, ws.numel()) == _lib.MOE_ERR_ARG
    assert call(2, 63, ws.numel()) == _lib.MOE_ERR_ARG     # k + S > 64
    assert call(2, 2, ws.numel(), path=7) == _lib.MOE_ERR_ARG
    assert call(2, 2, 1024) == _lib.MOE_ERR_WORKSPACE
    assert L.moe_experts_shared_workspace_bytes(desc, 0, 4, 2, 0) == 0
    torch.cuda.synchronize()


def test_merge_shared_rejects_other_shapes():
    from moelab_amd.experts import make_state, merge_shared
    from moelab_amd import formats
    sh, s = layer("int4", 256, 384, 8, 2, 2, seed=63)
    g = torch.Generator(device=DEV).manual_seed(64)
    s["shared"] = make_state("int4", *(formats.random_int4(2, n, kk, generator=g, device=DEV)
                                       for n, kk in ((320, 256), (320, 256), (256, 320))))
    with pytest.raises(ValueError):
        merge_shared(s)
