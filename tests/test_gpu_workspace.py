"""Workspace lifetime under HIP graph capture (moe-lab_amd/_lib.py: workspace / grow; experts.reserve).

A captured graph keeps the raw workspace pointer of its capture. When a later, larger call grows the per-device
workspace, the old buffer must stay valid: the graph's replays are checked against the oracle and against the
first replay bit for bit, with eager work and fresh allocations (which would reuse a freed buffer) in between."""
import numpy as np
import pytest
import torch

from helpers import assert_close, oracle_y

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_graph_replays_stay_valid_after_the_workspace_grows():
    from moelab_amd import _lib
    from moelab_amd.experts import reserve, run_experts
    from moelab_amd.problem import baseline_int4_layer, make_routing
    from moelab_amd.shapes import MoEShape
    sh = MoEShape("ws", d=256, f=384, E=8, k=2)
    s = baseline_int4_layer(sh, seed=3, device=DEV, router=False)
    rng = np.random.default_rng(3)
    T = 6
    x = torch.from_numpy(rng.standard_normal((T, sh.d)).astype(np.float32)).to(DEV, torch.bfloat16)
    i0, w0 = make_routing(T, sh.E, sh.k, "uniform", rng)
    idx, wts = torch.from_numpy(i0).to(DEV), torch.from_numpy(w0).to(DEV)
    reserve(s, T, sh.k)
    out = torch.empty((T, sh.d), dtype=torch.float32, device=DEV)
    run_experts(s, x, idx, wts, path=_lib.PATH_GROUPED, out=out, out_dtype=torch.float32)   # warm-up, eager
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run_experts(s, x, idx, wts, path=_lib.PATH_GROUPED, out=out, out_dtype=torch.float32)
    ws_before = _lib.workspace(DEV, 0)
    g.replay()
    torch.cuda.synchronize()
    first = out.clone()
    assert_close(first, oracle_y(s, x, idx, wts), what="first replay")
    # a call needing more than the current workspace grows it (earlier tests may have grown it already: ask for
    # one byte more than it has); memory allocated afterwards would land on a freed buffer
    _lib.workspace(DEV, ws_before.numel() + 1)
    assert _lib.workspace(DEV, 0).data_ptr() != ws_before.data_ptr()
    T2 = 300
    x2 = torch.randn((T2, sh.d), device=DEV).to(torch.bfloat16)
    i2, w2 = make_routing(T2, sh.E, sh.k, "uniform", rng)
    y2 = run_experts(s, x2, torch.from_numpy(i2).to(DEV), torch.from_numpy(w2).to(DEV), path=_lib.PATH_GROUPED)
    junk = [torch.full((ws_before.numel(),), 0x7F, dtype=torch.uint8, device=DEV) for _ in range(4)]
    for rep in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, first), rep
        y2 = y2 + 0   # eager work between replays
    del junk
