"""moe_layer_run (router + experts in one call) against the oracle router and against the separate calls.

At T=1 the router launch computes the logits only and every gate/up wave runs the router tail itself
(reference moelab/router.py:15-66 semantics: lowest id on ties, softmax over the top-k or full-softmax
probabilities times a scale); at T>1 the tail runs as its own launch. Either way the ids must equal the CPU
oracle's (logits in the documented fixed order, bit for bit), the weights must match it to float rounding, and the
layer output must be bit-identical to router.route followed by the experts call on the same ids (the same
kernels run) and within the north-star gate of the oracle."""
import numpy as np
import pytest
import torch

from helpers import assert_close, np_u16, oracle_y, orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def check_layer(s, x, wr, k, bias=None, norm=True, scale=1.0, act=0, what=""):
    from moelab_amd import router
    from moelab_amd.experts import run_experts, run_routed
    y, idx, wts = run_routed(s, x, wr, k, bias=bias, norm=norm, scale=scale, act=act, out_dtype=torch.float32)
    i2, w2 = router.route(x, wr, k, bias=bias, norm=norm, scale=scale)
    y2 = run_experts(s, x, i2, w2, act=act, out_dtype=torch.float32)
    torch.cuda.synchronize()
    b = None if bias is None else bias.float().cpu().numpy()
    idx_ref, wts_ref = orc.topk(orc.router_logits(np_u16(x), np_u16(wr), b), k, norm=norm, scale=scale)
    assert np.array_equal(idx.cpu().numpy(), idx_ref), what
    np.testing.assert_allclose(wts.cpu().numpy(), wts_ref, rtol=2e-6, atol=1e-7)
    assert torch.equal(idx, i2) and torch.equal(wts, w2), what
    assert torch.equal(y, y2), (what, float((y - y2).abs().max()))
    assert_close(y, oracle_y(s, x, idx, wts, act), what=what)
    yb, _, _ = run_routed(s, x, wr, k, bias=bias, norm=norm, scale=scale, act=act)
    assert yb.dtype == torch.bfloat16
    return idx


@pytest.mark.parametrize("T", [1, 2, 32])
def test_layer_qwen3_shape(T):
    from moelab_amd.problem import baseline_int4_layer, baseline_x
    from moelab_amd.shapes import SHAPES
    sh = SHAPES["qwen3-30b-a3b"]
    s = baseline_int4_layer(sh, seed=60 + T, device=DEV)
    x = baseline_x(T, sh.d, seed=T, device=DEV)
    print(f"case layer qwen3 T={T}", flush=True)
    check_layer(s, x, s["wr"], sh.k, what=("qwen3", T))


@pytest.mark.parametrize("T", [1, 5])
def test_layer_bias_full_softmax_and_scale(T):
    """Zipf-skewed router bias, DeepSeek-V2-style full-softmax probabilities (norm=False) times a scale."""
    from moelab_amd.problem import baseline_int4_layer, baseline_x, zipf_bias
    from moelab_amd.shapes import SHAPES
    sh = SHAPES["deepseek-v2-lite"]
    s = baseline_int4_layer(sh, seed=70 + T, device=DEV)
    x = baseline_x(T, sh.d, seed=T, device=DEV)
    bias = torch.from_numpy(zipf_bias(sh.E, 1.1, seed=4)).to(DEV)
    print(f"case layer bias/full-softmax T={T}", flush=True)
    check_layer(s, x, s["wr"], sh.k, bias=bias, norm=False, scale=2.5, what=("dsv2", T))


@pytest.mark.parametrize("T", [1, 8])
def test_layer_gptoss_mxfp4(T):
    """gpt-oss: MXFP4 experts with biases, the clamped SwiGLU (act 2), softmax over the top-4."""
    from moelab_amd.problem import baseline_mxfp4_layer, baseline_x
    from moelab_amd.shapes import SHAPES
    sh = SHAPES["gpt-oss-20b"]
    s = baseline_mxfp4_layer(sh, seed=80 + T, device=DEV)
    x = baseline_x(T, sh.d, seed=T, device=DEV)
    print(f"case layer gptoss T={T}", flush=True)
    check_layer(s, x, s["wr"], sh.k, act=2, what=("gptoss", T))


def test_layer_ties_pick_lowest_ids():
    """All-equal router rows (every logit ties): the tail in the gate/up waves picks ids 0..k-1 with equal weights,
    as the reference's known answer (reference tests/test_router.py:36-41)."""
    from moelab_amd.problem import baseline_int4_layer, baseline_x
    from moelab_amd.shapes import MoEShape
    sh = MoEShape("ties", d=256, f=256, E=16, k=4)
    s = baseline_int4_layer(sh, seed=9, device=DEV)
    wr = torch.full((sh.E, sh.d), 0.01, device=DEV).to(torch.bfloat16)
    x = baseline_x(1, sh.d, seed=9, device=DEV)
    idx = check_layer(s, x, wr, sh.k, what="ties")
    assert idx.cpu().numpy().tolist() == [[0, 1, 2, 3]]


@pytest.mark.parametrize("E", [200, 1000])
def test_layer_ties_across_logit_groups(E):
    """The router tail in the gate/up waves with E > 128 (4 and 16 logits per lane): three router rows set equal so
    that experts 9, 67 and E - 50 (lanes 9, 3 and (E - 50) % 64 of logit groups 0, 1 and (E - 50) // 64) tie for
    the top; the rounds must take them lowest id first, as the oracle does, and the rest of the layer must match."""
    from moelab_amd.problem import baseline_int4_layer, baseline_x
    from moelab_amd.shapes import MoEShape
    sh = MoEShape("tiesJ", d=256, f=256, E=E, k=4)
    s = baseline_int4_layer(sh, seed=11, device=DEV)
    x = baseline_x(1, sh.d, seed=11, device=DEV)
    wr = s["wr"].clone()
    top = (torch.sign(x[0].float()) * 0.05).to(torch.bfloat16)   # logit 0.05 sum |x|: above every random row's
    for e in (9, 67, E - 50):
        wr[e] = top
    print(f"case layer ties across groups E={E}", flush=True)
    idx = check_layer(s, x, wr, sh.k, what=("tiesJ", E))
    assert idx.cpu().numpy()[0, :3].tolist() == [9, 67, E - 50]


@pytest.mark.parametrize("T,dist", [(32, "uniform"), (32, "zipf"), (64, "zipf"), (16, "uniform")])
def test_layer_batched_router_builds_grouping(T, dist, monkeypatch):
    """BASELINE config 3 through moe_layer_run: the router's launches (logits, tails), the gate/up wave tiles grouping
    the slots in-kernel and writing the lists the down stage reads; bit-identical to route + the experts call, and the
    same again with MOE_LAYER_INGROUP=0 (the router's last workgroup builds the grouping and pass lists)."""
    from moelab_amd.experts import run_routed
    from moelab_amd.problem import baseline_int4_layer, baseline_x, zipf_bias
    from moelab_amd.shapes import SHAPES
    sh = SHAPES["qwen3-30b-a3b"]
    s = baseline_int4_layer(sh, seed=90 + T, device=DEV)
    x = baseline_x(T, sh.d, seed=T, device=DEV)
    bias = torch.from_numpy(zipf_bias(sh.E, 1.1, seed=3)).to(DEV) if dist == "zipf" else None
    print(f"case layer batched T={T} {dist}", flush=True)
    check_layer(s, x, s["wr"], sh.k, bias=bias, what=("qwen3", T, dist))
    y, _, _ = run_routed(s, x, s["wr"], sh.k, bias=bias, out_dtype=torch.float32)
    monkeypatch.setenv("MOE_LAYER_INGROUP", "0")
    y2, _, _ = run_routed(s, x, s["wr"], sh.k, bias=bias, out_dtype=torch.float32)
    assert torch.equal(y, y2)


def _shared_layer(fmt, d, F, E, k, S, seed, gated):
    from moelab_amd import formats
    from moelab_amd.experts import make_state, merge_shared
    from moelab_amd.problem import baseline_int4_layer, baseline_mxfp4_layer
    from moelab_amd.shapes import MoEShape
    sh = MoEShape("m", d=d, f=F, E=E, k=k)
    s = baseline_int4_layer(sh, seed, DEV) if fmt == "int4" else baseline_mxfp4_layer(sh, seed, DEV)
    g = torch.Generator(device=DEV).manual_seed(seed + 1)
    rnd = formats.random_int4 if fmt == "int4" else formats.random_mxfp4
    s["shared"] = make_state(fmt, rnd(S, F, d, generator=g, device=DEV), rnd(S, F, d, generator=g, device=DEV),
                             rnd(S, d, F, generator=g, device=DEV))
    if gated:
        s["shared_gate"] = (torch.randn(d, generator=g, device=DEV) * 0.05).to(torch.bfloat16)
    return sh, s, merge_shared(s)


SHARED_CASES = [
    # (fmt, d, F, E, k, S, T, gated, norm, scale)
    ("int4", 512, 256, 16, 4, 2, 1, False, True, 1.0),      # T = 1: per-slot GEMV over k + S slots
    ("int4", 512, 256, 16, 4, 2, 7, True, True, 1.0),       # gated (Qwen-style), wave tiles
    ("int4", 512, 384, 64, 6, 2, 256, False, False, 1.0),   # DeepSeek-V2 greedy: full softmax, dense down
    ("int4", 256, 256, 16, 4, 1, 300, True, False, 2.5),    # 1500 slots, 300 on the shared expert: dense tiles
    ("mxfp4", 512, 512, 8, 2, 2, 40, True, True, 1.0),      # MXFP4, block-scaled wave tiles
]


@pytest.mark.parametrize("case", SHARED_CASES, ids=lambda c: f"{c[0]}-E{c[3]}k{c[4]}S{c[5]}-T{c[6]}-{'g' if c[7] else 'u'}")
def test_layer_shared_router_builds_grouping(case):
    """moe_layer_run_shared: the router launch also computes the shared gate (one more logit row in the same fixed
    order), writes the merged [T, k + S] slot lists and groups them; the experts follow as moe_experts_run_shared.
    Bit-identical to route + run_experts_shared on the same ids, and within the gate of the oracle's routed +
    shared sum."""
    from moelab_amd import router
    from moelab_amd.experts import run_experts_shared, run_routed
    from moelab_amd.problem import baseline_x
    fmt, d, F, E, k, S, T, gated, norm, scale = case
    sh, s, m = _shared_layer(fmt, d, F, E, k, S, seed=100 + T, gated=gated)
    x = baseline_x(T, d, seed=T + 5, device=DEV)
    act = 0   # SwiGLU: the oracle's shared experts are SwiGLU MLPs (no model pairs gpt-oss's act with them)
    print(f"case layer shared {case}", flush=True)
    y, idx, wts = run_routed(m, x, s["wr"], k, norm=norm, scale=scale, act=act, out_dtype=torch.float32)
    i2, w2 = router.route(x, s["wr"], k, norm=norm, scale=scale)
    y2 = run_experts_shared(m, x, i2, w2, act=act, out_dtype=torch.float32)
    torch.cuda.synchronize()
    idx_ref, wts_ref = orc.topk(orc.router_logits(np_u16(x), np_u16(s["wr"])), k, norm=norm, scale=scale)
    assert np.array_equal(idx.cpu().numpy(), idx_ref)
    assert torch.equal(idx, i2) and torch.equal(wts, w2)
    assert torch.equal(y, y2), float((y - y2).abs().max())
    assert_close(y, oracle_y(s, x, idx, wts, act), what=case)
    # the state with separate shared experts: router + routed experts in one call, the shared ones in a second
    y3, _, _ = run_routed(s, x, s["wr"], k, norm=norm, scale=scale, act=act, out_dtype=torch.float32)
    assert_close(y3, oracle_y(s, x, idx, wts, act), what=case)


def test_layer_grouping_beyond_one_workgroup():
    """2048 tokens exceed what the router's one finishing workgroup takes: the tails run one wave per token and the
    grouping runs as a launch of its own; results as the separate calls."""
    from moelab_amd.problem import baseline_int4_layer, baseline_x
    from moelab_amd.shapes import MoEShape
    sh = MoEShape("big", d=128, f=128, E=8, k=2)
    s = baseline_int4_layer(sh, seed=12, device=DEV)
    x = baseline_x(2048, sh.d, seed=12, device=DEV)
    print("case layer 4096 slots", flush=True)
    check_layer(s, x, s["wr"], sh.k, what="big")
