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
