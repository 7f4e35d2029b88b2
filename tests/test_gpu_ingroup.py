"""In-kernel grouping of the wave tiles (both stages on the wave tiles, at most 1024 slots): every workgroup finds
its pass from the raw ids (LDS histogram, wave scan of the per-expert pass counts, ballot-ranked slot list) instead of
reading the pass list of the grouping launch (group_slots). The passes and their slot order are the grouping
launch's, so the outputs must be bit-identical to the same call with the grouping launch (MOE_INGROUP=0), and
within the north-star gate of the oracle; covered: uniform / zipf / one-hot loads, ids outside [0, E) (they join no
pass), experts with several passes, 16- and 32-token passes, both pass lists (expert-major and compact), the
1024-slot limit and the first size past it, fp32 x on 3 planes, MXFP4, and the stages run as two calls."""
import numpy as np
import pytest
import torch

from helpers import assert_close, oracle_y

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def state(fmt, d, F, E, k, seed):
    from moelab_amd.problem import baseline_int4_layer, baseline_mxfp4_layer
    from moelab_amd.shapes import MoEShape
    sh = MoEShape("g", d=d, f=F, E=E, k=k)
    if fmt == "int4":
        return sh, baseline_int4_layer(sh, seed, DEV, router=False)
    return sh, baseline_mxfp4_layer(sh, seed, DEV, biases=True, router=False)


def inputs(sh, T, routing, seed, dtype=torch.bfloat16):
    from moelab_amd.problem import make_routing
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.standard_normal((T, sh.d)).astype(np.float32)).to(DEV, dtype)
    idx, wts = make_routing(T, sh.E, sh.k, routing, rng)
    return x, torch.from_numpy(idx).to(DEV), torch.from_numpy(wts).to(DEV)


def both(monkeypatch, s, x, idx, wts, act=0, **kw):
    """The call with the grouping launch, then in-kernel grouped with the default pass list, the compact one
    (every pass found by the scan) and the expert-major one (first passes by expert id, the rest by the scan):
    all four must agree bit for bit. Returns (grouping launch, default in-kernel)."""
    from moelab_amd import _lib
    from moelab_amd.experts import run_experts
    kw.setdefault("path", _lib.PATH_GROUPED)
    monkeypatch.setenv("MOE_INGROUP", "0")
    y0 = run_experts(s, x, idx, wts, act=act, out_dtype=torch.float32, **kw)
    monkeypatch.setenv("MOE_INGROUP", "1")
    y1 = run_experts(s, x, idx, wts, act=act, out_dtype=torch.float32, **kw)
    for first in ("0", "1"):
        monkeypatch.setenv("MOE_INGROUP_FIRST", first)
        yf = run_experts(s, x, idx, wts, act=act, out_dtype=torch.float32, **kw)
        torch.cuda.synchronize()
        assert torch.equal(yf, y0), ("pass list", first, float((yf - y0).abs().max()))
    monkeypatch.delenv("MOE_INGROUP_FIRST")
    torch.cuda.synchronize()
    return y0, y1


CASES = [
    # (fmt, d, F, E, k, T, routing, act)
    ("int4", 2048, 768, 128, 8, 32, "uniform", 0),     # Qwen3 decode batch: 16-token passes, mostly 1-3 slots
    ("int4", 2048, 768, 128, 8, 64, "zipf", 0),        # skewed: hot experts over several passes
    ("int4", 1024, 512, 8, 2, 100, "uniform", 0),      # 25 slots per expert: 32-token passes (nt = 2)
    ("int4", 512, 384, 64, 6, 7, "one_hot", 0),        # every token on the same 6 experts
    ("int4", 1024, 512, 128, 8, 4, "uniform", 0),      # 32 slots on 128 experts: the compact pass list
    ("int4", 512, 256, 256, 4, 256, "uniform", 1),     # 1024 slots: the in-kernel limit
    ("int4", 512, 256, 256, 4, 257, "uniform", 1),     # 1028 slots: the grouping launch again
    ("mxfp4", 512, 512, 32, 4, 24, "zipf", 2),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-E{c[3]}k{c[4]}-T{c[5]}-{c[6]}")
def test_ingroup_equals_grouping_launch(case, monkeypatch):
    fmt, d, F, E, k, T, routing, act = case
    sh, s = state(fmt, d, F, E, k, seed=T)
    x, idx, wts = inputs(sh, T, routing, seed=T)
    print(f"case ingroup {case}", flush=True)
    y0, y1 = both(monkeypatch, s, x, idx, wts, act=act)
    assert torch.equal(y0, y1), float((y0 - y1).abs().max())
    assert_close(y1, oracle_y(s, x, idx, wts, act), what=case)


def test_ingroup_invalid_ids_and_ragged(monkeypatch):
    """Ids -1 and E + 3 scattered over the slots (they contribute nothing), ragged per-expert counts."""
    sh, s = state("int4", 1024, 512, 64, 8, seed=3)
    x, idx, wts = inputs(sh, 40, "zipf", seed=5)
    bad = idx.clone()
    bad[3, 1] = -1
    bad[17, 7] = sh.E + 3
    bad[39, 0] = -1
    y0, y1 = both(monkeypatch, s, x, bad, wts)
    assert torch.equal(y0, y1)
    keep = (bad >= 0) & (bad < sh.E)
    assert_close(y1, oracle_y(s, x, idx, wts * keep), what="invalid ids")


def test_ingroup_fp32_planes_and_stages(monkeypatch):
    """fp32 x (three bf16 planes per token) and the two stages as separate calls: both decide the grouping from
    (T, k, E, d, F) alone, so the split call equals the whole one bit for bit."""
    from moelab_amd import _lib
    from moelab_amd.experts import run_experts
    sh, s = state("int4", 512, 384, 16, 4, seed=9)
    x, idx, wts = inputs(sh, 48, "uniform", seed=9, dtype=torch.float32)
    y0, y1 = both(monkeypatch, s, x, idx, wts)
    assert torch.equal(y0, y1)
    assert_close(y1, oracle_y(s, x, idx, wts), what="fp32 x")
    g = _lib.PATH_GROUPED
    run_experts(s, x, idx, wts, path=g, out_dtype=torch.float32, stages=_lib.STAGE_GATE_UP)
    y2 = run_experts(s, x, idx, wts, path=g, out_dtype=torch.float32, stages=_lib.STAGE_DOWN)
    torch.cuda.synchronize()
    assert torch.equal(y2, y1)


@pytest.mark.parametrize("fmt,T,routing", [("int4", 32, "uniform"), ("int4", 64, "zipf"), ("mxfp4", 32, "uniform")])
def test_down_ring_depth_bit_identical(monkeypatch, fmt, T, routing):
    """The down wave tiles keep one slice in flight instead of two when the launch has many live waves (a choice
    made on the device from the pass count; MOE_WAVE_DN_SHALLOW is its threshold). Both walks fold the same slices
    in the same order, so forcing either one (threshold 1: always one slice; 0: always the ring) gives the same
    outputs bit for bit, and the default call (uniform T=32 takes one slice, Zipf T=64 the ring) equals both."""
    from moelab_amd import _lib
    from moelab_amd.experts import run_experts
    sh, s = state(fmt, 2048, 768, 128, 8, seed=11)
    x, idx, wts = inputs(sh, T, routing, seed=T)
    print(f"case ring depth {fmt} T={T} {routing}", flush=True)
    ys = {}
    for v in ("1", "0", None):
        if v is None:
            monkeypatch.delenv("MOE_WAVE_DN_SHALLOW", raising=False)
        else:
            monkeypatch.setenv("MOE_WAVE_DN_SHALLOW", v)
        ys[v] = run_experts(s, x, idx, wts, out_dtype=torch.float32, path=_lib.PATH_GROUPED)
    torch.cuda.synchronize()
    assert torch.equal(ys["1"], ys["0"]), float((ys["1"] - ys["0"]).abs().max())
    assert torch.equal(ys[None], ys["0"])
    assert_close(ys[None], oracle_y(s, x, idx, wts), what=f"down ring depth {fmt} T={T} {routing}")
