"""BASELINE configurations at their full sizes against the CPU oracle.

The reference runs Zipf-skewed and dispatch-boundary cases through every production path
(reference tests/test_edge_cases.py:55-74). Here each BASELINE config runs at its real shape and token count
on the GPU, built exactly as bench.py builds it (same generators and seeds): config 3 (Qwen3-30B-A3B int4 at
T = 16, 32, 64, uniform and Zipf(1.1) routing), 5a (Mixtral-8x7B int4, T = 512, the dense fp16 tiles) and
5b (DeepSeek-V2-Lite int4, T = 256, routed top-6 of 64 plus 2 always-on shared experts). Router ids and the
slot grouping are compared bit for bit with the oracle. Token outputs are independent of each other, so the
fp64 oracle runs on a seeded sample of 64 token rows of the full call (every row when T <= 64), at the
north-star gate max|y - y_ref| <= 1e-2 RMS(y_ref) (fp32 output; bf16 output: plus its own rounding).
"""
import numpy as np
import pytest
import torch

from helpers import assert_close, np_u16, oracle_y, orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def sample_rows(T, n=64, seed=0):
    if T <= n:
        return np.arange(T)
    return np.sort(np.random.default_rng(seed).choice(T, size=n, replace=False))


def route_checked(x, wr, k, bias=None):
    """Fused router on the GPU; logits, ids and weights against the oracle (ids and logits bit for bit)."""
    from moelab_amd import router
    idx, wts, logits = router.route(x, wr, k, bias=bias, return_logits=True)
    b = None if bias is None else bias.float().cpu().numpy()
    lg_ref = orc.router_logits(np_u16(x), np_u16(wr), b)
    idx_ref, wts_ref = orc.topk(lg_ref, k)
    torch.cuda.synchronize()
    assert np.array_equal(logits.cpu().numpy().view(np.uint32), lg_ref.view(np.uint32)), "logits differ"
    assert np.array_equal(idx.cpu().numpy(), idx_ref), "router ids differ"
    np.testing.assert_allclose(wts.cpu().numpy(), wts_ref, rtol=1e-6, atol=1e-7)
    return idx, wts


def grouping_checked(idx, E):
    """moe_group (the grouped path's slot grouping) against the oracle's stable sort, bit for bit."""
    from moelab_amd import router
    counts, offsets, srt, active, meta = router.group(idx, E)
    c_ref, o_ref, s_ref, a_ref = orc.group(idx.cpu().numpy(), E)
    torch.cuda.synchronize()
    assert np.array_equal(counts.cpu().numpy(), c_ref)
    assert np.array_equal(offsets.cpu().numpy(), o_ref)
    assert np.array_equal(srt.cpu().numpy(), s_ref)
    assert int(meta[0]) == a_ref.size and np.array_equal(active[:a_ref.size].cpu().numpy(), a_ref)
    return int(a_ref.size)


def check_rows(y, state, x, idx, wts, rows, what, act=0):
    sel = torch.as_tensor(rows, device=DEV)
    ref = oracle_y(state, x[sel], idx[sel], wts[sel], act)
    return assert_close(y[sel], ref, what=what)


@pytest.mark.parametrize("norm", [True, False])
def test_config1_tiny_routed_layer(norm):
    """BASELINE config 1 as stated: d=512, F=256, E=8, top-1, T=4 tokens of bf16 x ~N(0,1), router weights
    ~N(0,0.02), SwiGLU int4 g64 experts (uniform codes, scales U(0.005,0.02), biases -8 scale). The fused router runs
    inside the layer call (moe_layer_run): softmax then top-1, with the one weight renormalised to 1 (norm) or the
    full softmax probability. Ids and weights against the oracle's router (ids bit for bit), y at the gate."""
    from moelab_amd.experts import run_routed
    from moelab_amd.problem import baseline_int4_layer, baseline_x
    from moelab_amd.shapes import MoEShape
    print(f"case config1 norm={norm}", flush=True)
    sh = MoEShape("config1", d=512, f=256, E=8, k=1)
    ly = baseline_int4_layer(sh, seed=1, device=DEV)
    x = baseline_x(4, sh.d, seed=1, device=DEV)
    y, idx, wts = run_routed(ly, x, ly["wr"], 1, norm=norm, out_dtype=torch.float32)
    lg_ref = orc.router_logits(np_u16(x), np_u16(ly["wr"]), None)
    idx_ref, wts_ref = orc.topk(lg_ref, 1, norm=norm)
    torch.cuda.synchronize()
    assert np.array_equal(idx.cpu().numpy(), idx_ref), "router ids differ"
    np.testing.assert_allclose(wts.cpu().numpy(), wts_ref, rtol=1e-6, atol=1e-7)
    if norm:
        assert np.all(wts.cpu().numpy() == 1.0)
    check_rows(y, ly, x, idx, wts, np.arange(4), ("config1", norm))


@pytest.mark.parametrize("routing", ["uniform", "zipf"])
@pytest.mark.parametrize("T", [16, 32, 64])
def test_config3_qwen3_full_size(T, routing):
    """Config 3: Qwen3-30B-A3B int4 g64 (d=2048, F=768, E=128, k=8) at T = 16, 32, 64, uniform router logits or
    Zipf(1.1) popularity through the router bias (zipf_bias(E, 1.1, seed=3), as bench.py). Both arms the bench
    times: the variant's dispatch (grouped expert tiles at these loads) and the per-slot GEMV over all slots."""
    from moelab_amd import _lib
    from moelab_amd.experts import run_experts
    from moelab_amd.problem import baseline_int4_layer, baseline_x, zipf_bias
    from moelab_amd.shapes import SHAPES
    from moelab_amd.variants import hip_q4_moe as q4
    sh = SHAPES["qwen3-30b-a3b"]
    layer = baseline_int4_layer(sh, seed=5000 + T, device=DEV)
    x = baseline_x(T, sh.d, seed=T, device=DEV)
    bias = torch.from_numpy(zipf_bias(sh.E, 1.1, seed=3)).to(DEV) if routing == "zipf" else None
    print(f"case config3 T={T} routing={routing}", flush=True)
    idx, wts = route_checked(x, layer["wr"], sh.k, bias)
    U = grouping_checked(idx, sh.E)
    if routing == "zipf":
        assert U < 0.6 * sh.E, U   # the skew concentrates the slots on few experts
    assert q4.custom_wins(T, sh.k, sh.E, sh.d, sh.f)   # the grouped tiles take these loads
    rows = sample_rows(T)
    y = q4.run(layer, x, idx, wts)
    y32 = q4.run(layer, x, idx, wts, out_dtype=torch.float32)
    ys = run_experts(layer, x, idx, wts, path=_lib.PATH_SLOTS, out_dtype=torch.float32)
    torch.cuda.synchronize()
    check_rows(y32, layer, x, idx, wts, rows, ("config3", T, routing, "grouped fp32"))
    check_rows(y, layer, x, idx, wts, rows, ("config3", T, routing, "grouped bf16"))
    check_rows(ys, layer, x, idx, wts, rows, ("config3", T, routing, "per-slot fp32"))


def test_config5a_mixtral_full_size():
    """Config 5a: Mixtral-8x7B int4 g64 (d=4096, F=14336, E=8, k=2) at T=512 (128 slots per expert: the dense
    fp16 tiles on both projections, the down split over K), uniform router; 64 sampled token rows."""
    from moelab_amd.problem import baseline_int4_layer, baseline_x
    from moelab_amd.shapes import SHAPES
    from moelab_amd.variants import hip_q4_moe as q4
    sh = SHAPES["mixtral-8x7b"]
    T = 512
    layer = baseline_int4_layer(sh, seed=3000, device=DEV)
    x = baseline_x(T, sh.d, seed=T, device=DEV)
    print("case config5a mixtral T=512", flush=True)
    idx, wts = route_checked(x, layer["wr"], sh.k)
    grouping_checked(idx, sh.E)
    y32 = q4.run(layer, x, idx, wts, out_dtype=torch.float32)
    y = q4.run(layer, x, idx, wts)
    torch.cuda.synchronize()
    rows = sample_rows(T, seed=51)
    check_rows(y32, layer, x, idx, wts, rows, ("config5a", "fp32"))
    check_rows(y, layer, x, idx, wts, rows, ("config5a", "bf16"))


def test_config5b_dsv2_lite_shared_full_size():
    """Config 5b: DeepSeek-V2-Lite int4 g64 (d=2048, F=1408, E=64, k=6) at T=256 plus 2 always-on shared experts of
    F=1408, built as bench.py builds it: the shared experts merged into the routed set (experts 64, 65; one call
    of 8 slots per token, 31 per expert: wave gate/up into the dense down). The two-call form (routed, then
    shared on its own small grid) is checked too; 64 sampled token rows against the oracle on the unmerged layer."""
    from moelab_amd import formats
    from moelab_amd.experts import make_state, merge_shared
    from moelab_amd.problem import baseline_int4_layer, baseline_x
    from moelab_amd.shapes import SHAPES
    from moelab_amd.variants import hip_q4_moe as q4
    sh = SHAPES["deepseek-v2-lite"]
    T = 256
    layer = baseline_int4_layer(sh, seed=4000, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(4100)
    layer["shared"] = make_state("int4", *(formats.random_int4(sh.shared, n, k, generator=g, device=DEV)
                                           for n, k in ((sh.f, sh.d), (sh.f, sh.d), (sh.d, sh.f))))
    x = baseline_x(T, sh.d, seed=T, device=DEV)
    print("case config5b dsv2-lite T=256 + 2 shared", flush=True)
    idx, wts = route_checked(x, layer["wr"], sh.k)
    grouping_checked(idx, sh.E)
    merged = merge_shared(layer)
    y32 = q4.run(merged, x, idx, wts, out_dtype=torch.float32)
    y = q4.run(merged, x, idx, wts)
    y2 = q4.run(layer, x, idx, wts, out_dtype=torch.float32)
    torch.cuda.synchronize()
    rows = sample_rows(T, seed=52)
    check_rows(y32, layer, x, idx, wts, rows, ("config5b", "fp32"))
    check_rows(y, layer, x, idx, wts, rows, ("config5b", "bf16"))
    check_rows(y2, layer, x, idx, wts, rows, ("config5b", "two calls"))
