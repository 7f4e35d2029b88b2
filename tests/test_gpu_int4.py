"""int4 g64 expert path on the GPU vs the CPU oracle (fp64 loop on the dequantised weights).

Gate (north star): max |y - y_ref| <= 1e-2 * RMS(y_ref); accumulation fp32, h and y stored bf16.
Cases follow the reference's edge-case suite (reference tests/test_edge_cases.py:55-140): dispatch
boundaries, odd shapes, zero / unnormalised weights, one expert set, slot permutation, batch
consistency, large activations, plus the full Qwen3-30B-A3B shape at T = 1 and T = 32."""
import numpy as np
import pytest
import torch

from helpers import assert_close, deq, np_u16, oracle_y, orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def q4():
    from moelab_amd.variants import hip_q4_moe
    return hip_q4_moe


def packed_state(shape, seed, biases=False):
    from moelab_amd.problem import baseline_int4_layer
    s = baseline_int4_layer(shape, seed, DEV, router=False)
    if biases:
        g = torch.Generator(device=DEV).manual_seed(seed + 1)
        s["bg"] = torch.randn((shape.E, shape.f), generator=g, device=DEV) * 0.1
        s["bu"] = torch.randn((shape.E, shape.f), generator=g, device=DEV) * 0.1
        s["bd"] = torch.randn((shape.E, shape.d), generator=g, device=DEV) * 0.1
    return s


def inputs(shape, T, routing="uniform", seed=0, scale=1.0):
    from moelab_amd.problem import make_routing
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.standard_normal((T, shape.d)).astype(np.float32) * scale).to(DEV, torch.bfloat16)
    idx, wts = make_routing(T, shape.E, shape.k, routing, rng)
    return x, torch.from_numpy(idx).to(DEV), torch.from_numpy(wts).to(DEV)


@pytest.fixture(params=["default", "forced-custom"])
def policy(request, monkeypatch):
    """'forced-custom' disables the load fallback and fails if it runs (reference test_edge_cases.py:26-37)."""
    if request.param == "forced-custom":
        mod = q4()
        monkeypatch.setattr(mod, "custom_wins", lambda *a: True)

        def no_fallback(*a, **k):
            raise AssertionError("fallback ran in forced-custom mode")
        monkeypatch.setattr(mod, "gather_moe", no_fallback)
    return request.param


def check(shape, T, routing="uniform", seed=0, idx=None, wts=None, act=0, scale=1.0, state=None, biases=False):
    s = state if state is not None else packed_state(shape, seed + 100, biases=biases)
    x, i0, w0 = inputs(shape, T, routing, seed, scale)
    idx = i0 if idx is None else torch.as_tensor(idx, dtype=torch.int32, device=DEV)
    wts = w0 if wts is None else torch.as_tensor(wts, dtype=torch.float32, device=DEV)
    print(f"case shape={shape} T={T} routing={routing} act={act}", flush=True)
    y = q4().run(s, x, idx, wts, act=act)
    y32 = q4().run(s, x, idx, wts, act=act, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert y.shape == x.shape and y.dtype == x.dtype and y32.dtype == torch.float32
    ref = oracle_y(s, x, idx, wts, act)
    assert_close(y32, ref, what=(shape, T, "fp32 out"))
    assert_close(y, ref, what=(shape, T, "bf16 out"))
    return y, s, x, idx, wts


def shape_(name, d, f, E, k):
    from moelab_amd.shapes import MoEShape
    return MoEShape(name, d=d, f=f, E=E, k=k)


@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 7, 8, 9, 15, 17, 31, 63, 65, 127, 129, 257])
def test_dispatch_boundaries(policy, T):
    check(shape_("q", 256, 384, 16, 4), T, routing="zipf", seed=T)


SHAPES = [("d192", 192, 256, 8, 2), ("f320", 256, 320, 8, 2), ("odd", 320, 448, 8, 3), ("k1", 128, 256, 8, 1),
          ("kE", 128, 256, 4, 4), ("E1", 128, 256, 1, 1), ("gptoss-like", 2880, 2880, 4, 2),
          ("tiny-baseline", 512, 256, 8, 1)]


@pytest.mark.parametrize("sh", SHAPES, ids=lambda s: s[0])
@pytest.mark.parametrize("T", [1, 2, 6, 33])
def test_shapes(policy, sh, T):
    check(shape_(*sh), T)


@pytest.mark.parametrize("T", [1, 4, 16])
def test_zero_and_unnormalized_weights(policy, T):
    sh = shape_("w", 256, 256, 8, 4)
    rng = np.random.default_rng(T)
    wts = rng.random((T, 4)).astype(np.float32) * 3
    wts[:, 1] = 0
    wts[0] = 0
    y, *_ = check(sh, T, wts=wts)
    assert float(y[0].float().abs().max()) == 0.0   # all-zero weights -> exactly zero output


@pytest.mark.parametrize("T", [2, 8, 32])
def test_all_tokens_one_expert_set(policy, T):
    check(shape_("o", 256, 256, 16, 4), T, idx=np.tile([[3, 7, 0, 15]], (T, 1)))


@pytest.mark.parametrize("T", [1, 8])
def test_permutation_invariance(policy, T):
    sh = shape_("p", 256, 256, 16, 4)
    y1, s, x, idx, wts = check(sh, T, seed=1)
    perm = torch.tensor([2, 0, 3, 1], device=DEV)
    y2 = q4().run(s, x, idx[:, perm].contiguous(), wts[:, perm].contiguous())
    rel = float((y1.float() - y2.float()).norm() / y1.float().norm())
    assert rel < 1e-2, rel


def test_batch_consistency(policy):
    sh = shape_("b", 256, 256, 16, 4)
    y, s, x, idx, wts = check(sh, 16, seed=2)
    for t in (0, 5, 15):
        one = q4().run(s, x[t:t + 1], idx[t:t + 1], wts[t:t + 1]).float()
        rel = float((one - y[t:t + 1].float()).norm() / y[t:t + 1].float().norm())
        assert rel < 1e-2, (t, rel)


def test_large_activations(policy):
    check(shape_("big", 256, 256, 8, 2), 8, seed=3, scale=100.0)


@pytest.mark.parametrize("act", [1, 2])
@pytest.mark.parametrize("T", [1, 9])
def test_activations_and_biases(act, T):
    check(shape_("a", 256, 256, 8, 2), T, act=act, biases=(act == 2))


def test_geglu_is_not_swiglu():
    """act 0 and act 1 must each match their own reference and not the other one (reference test_geglu.py:40-54)."""
    sh = shape_("g", 256, 256, 8, 2)
    s = packed_state(sh, 5)
    x, idx, wts = inputs(sh, 4, seed=5)
    for act, other in ((0, 1), (1, 0)):
        y = q4().run(s, x, idx, wts, act=act)
        assert_close(y, oracle_y(s, x, idx, wts, act))
        ref_other = oracle_y(s, x, idx, wts, other)
        err = orc.error_metrics(y.float().cpu().numpy(), ref_other)
        assert err["rel_fro"] > 0.05, err


def test_run_slots_per_slot_outputs():
    """T=1 unweighted per-slot outputs [k, D] (reference metal_q4_moe.py:49-51, test_geglu.py:57-70)."""
    sh = shape_("s", 256, 256, 8, 4)
    s = packed_state(sh, 6)
    x, idx, _ = inputs(sh, 1, seed=6)
    ys = q4().run_slots(s, x, idx)
    assert ys.shape == (4, 256)
    for j in range(4):
        ref = oracle_y(s, x, idx[:, j:j + 1], torch.ones((1, 1), device=DEV))
        assert_close(ys[j:j + 1], ref, what=j)


@pytest.mark.parametrize("T", [1, 5, 32])
def test_slots_path_equals_grouped(T):
    """The per-slot stock-style path and the grouped tiles agree (both checked against the oracle)."""
    from moelab_amd import _lib
    from moelab_amd.experts import run_experts
    sh = shape_("sg", 512, 384, 16, 4)
    s = packed_state(sh, 7)
    x, idx, wts = inputs(sh, T, seed=7)
    ref = oracle_y(s, x, idx, wts)
    for path in (_lib.PATH_SLOTS, _lib.PATH_GROUPED):
        for od in (torch.float32, torch.bfloat16):
            assert_close(run_experts(s, x, idx, wts, path=path, out_dtype=od), ref, what=(path, od))


@pytest.mark.parametrize("T", [1, 12])
def test_fused_residual(T):
    sh = shape_("r", 256, 256, 8, 2)
    s = packed_state(sh, 8)
    x, idx, wts = inputs(sh, T, seed=8)
    res = torch.randn_like(x.float()).to(torch.bfloat16)
    y = q4().run(s, x, idx, wts)
    yr = q4().run(s, x, idx, wts, residual=res)
    ref = oracle_y(s, x, idx, wts) + res.float().cpu().numpy()
    assert_close(yr, ref)
    assert_close(q4().run(s, x, idx, wts, residual=res.float(), out_dtype=torch.float32), ref)
    diff = (yr.float() - (y.float() + res.float())).abs().max().item()
    assert diff <= 2 * 2 ** -8 * max(1.0, (y.float() + res.float()).abs().max().item())


def test_prepare_dequant_roundtrip():
    """prepare() from dense weights, then run(); the fp32 reference uses dequant(state) like the
    reference harness (reference mlx_backend.py:133-143)."""
    from moelab_amd import backend
    sh = shape_("pd", 256, 384, 8, 2)
    wg, wu, wd = backend.make_weights(sh, "bfloat16", seed=3)
    s = q4().prepare(wg, wu, wd)
    x, idx, wts = backend.make_inputs(sh, 6, "bfloat16", "uniform", seed=3)
    y = q4().run(s, x, idx, wts)
    rwg, rwu, rwd = q4().dequant(s)
    err = backend.errors(y, backend.reference(rwg, rwu, rwd, x, idx, wts))
    assert err["finite"] and err["rel_fro"] < backend.TOL["bfloat16"], err
    # dequant agrees with the oracle's closed form
    np.testing.assert_allclose(rwg.cpu().numpy(), deq(s, "g"), rtol=1e-6, atol=1e-7)
    # quantisation error of the dense weights stays at int4 level
    rel = float((rwg.float() - wg.float()).norm() / wg.float().norm())
    assert rel < 0.15, rel


@pytest.mark.parametrize("T", [1, 32])
def test_qwen3_full_shape(T):
    """BASELINE config 2/3 shape: d=2048, F=768, E=128, k=8, through the fused router."""
    from moelab_amd import router
    from moelab_amd.problem import baseline_int4_layer, baseline_x
    from moelab_amd.shapes import SHAPES
    sh = SHAPES["qwen3-30b-a3b"]
    layer = baseline_int4_layer(sh, seed=11, device=DEV)
    s = layer
    x = baseline_x(T, sh.d, seed=11, device=DEV)
    idx, wts, logits = router.route(x, layer["wr"], sh.k, return_logits=True)
    lg_ref = orc.router_logits(np_u16(x), np_u16(layer["wr"]))
    idx_ref, wts_ref = orc.topk(lg_ref, sh.k)
    np.testing.assert_array_equal(idx.cpu().numpy(), idx_ref)
    ref = oracle_y(s, x, idx, wts)
    assert_close(q4().run(s, x, idx, wts, out_dtype=torch.float32), ref, what="fp32 out")
    assert_close(q4().run(s, x, idx, wts), ref, what="bf16 out")


@pytest.mark.parametrize("shape_args", [(2048, 768, 128, 8), (512, 256, 8, 1), (2048, 1408, 64, 6),
                                        (1024, 512, 16, 16), (256, 128, 4, 4)])
def test_t1_paths_agree(shape_args):
    """T=1: the default dispatch (PATH_AUTO) and the per-slot GEMV agree with the oracle, call after call (the
    workspace's leftover contents from one call never leak into the next)."""
    from moelab_amd import _lib
    from moelab_amd.experts import run_experts
    sh = shape_("f", *shape_args)
    s = packed_state(sh, 9)
    x, idx, wts = inputs(sh, 1, seed=9)
    ref = oracle_y(s, x, idx, wts)
    for _ in range(3):
        for path in (_lib.PATH_SLOTS, _lib.PATH_AUTO):
            assert_close(run_experts(s, x, idx, wts, path=path, out_dtype=torch.float32), ref, what=path)


def test_removed_fused_path_is_rejected():
    """Path 3 (a former single-launch T=1 kernel) is no longer accepted: MOE_ERR_ARG, before any launch."""
    from moelab_amd import _lib
    from moelab_amd.experts import run_experts
    sh = shape_("f", 256, 128, 4, 4)
    s = packed_state(sh, 9)
    x, idx, wts = inputs(sh, 1, seed=9)
    with pytest.raises(_lib.MoeError) as ei:
        run_experts(s, x, idx, wts, path=3)
    assert ei.value.rc == _lib.MOE_ERR_ARG


def scaled_state(base, factor=None, low=None, high=None, names=("g", "u", "d"), seed=0):
    """The packed state `base` with the int4 scales of projections `names` multiplied by `factor`, or drawn anew
    from U(low, high); biases = -8 x scale (codes centred, as the BASELINE configs)."""
    from moelab_amd.experts import make_state, unpack
    parts = {n: list(unpack(base, n)) for n in ("g", "u", "d")}
    gen = torch.Generator(device=DEV).manual_seed(seed)
    for n in names:
        sc = parts[n][1].float()
        if factor is not None:
            sc = sc * factor
        else:
            sc = low + (high - low) * torch.rand(sc.shape, generator=gen, device=DEV)
        parts[n][1] = sc.to(torch.bfloat16)
        parts[n][2] = (parts[n][1].float() * -8.0).to(torch.bfloat16)
    return make_state("int4", parts["g"], parts["u"], parts["d"])


def test_small_affine_scales():
    """Tiny scales (x1e-6 weights, x1e6 activations) stay accurate on the per-slot GEMV (T=1) and the wave tiles
    (T=7), which apply scale and bias in fp32 to exact-code sums (reference tests/test_int4_small_scales.py:23-32)."""
    from moelab_amd import formats
    sh = shape_("tiny", 256, 256, 8, 2)
    s = scaled_state(packed_state(sh, 10), factor=1e-6, names=("g", "u"))
    for T in (1, 7):
        x, idx, wts = inputs(sh, T, seed=10, scale=1e6)
        assert_close(q4().run(s, x, idx, wts, out_dtype=torch.float32), oracle_y(s, x, idx, wts), what=T)
    assert formats.GS_INT4 == 64


@pytest.mark.parametrize("T", [50, 200])
@pytest.mark.parametrize("case", ["x1e-6", "qwen3-min-scale"])
def test_small_affine_scales_dense_tiles(case, T, monkeypatch):
    """The dense tiles dequantise weights to fp16, where raw scales below 6.1e-5 would be subnormal and below ~6e-8
    zero: the tile records hold each row's scales and biases times 2^-E_row (largest at [2^10, 2^11)) and the
    epilogues scale the sums back by 2^E_row. Cases: every projection's scales x1e-6 with x x1e6; scales
    U(4e-6, 1.3e-5) around real Qwen3's smallest (8.6e-6). T=200 (100 slots per expert) runs the dense tiles on
    both projections, T=50 (25 per expert) the wave gate/up into the dense down (reference
    tests/test_int4_small_scales.py:21-32 runs its tiny-scale case through the MMA paths)."""
    monkeypatch.setenv("MOE_DENSE", "1")
    sh = shape_("tiny-dense", 256, 384, 4, 2)
    base = packed_state(sh, 12)
    if case == "x1e-6":
        s, xs = scaled_state(base, factor=1e-6), 1e6
    else:
        s, xs = scaled_state(base, low=4e-6, high=1.3e-5, seed=T), 1.0
    x, idx, wts = inputs(sh, T, "uniform", seed=T, scale=xs)
    print(f"case small scales dense {case} T={T}", flush=True)
    y32 = grouped(s, x, idx, wts, out_dtype=torch.float32)
    y = grouped(s, x, idx, wts)
    ref = oracle_y(s, x, idx, wts)
    assert np.abs(ref).max() > 0
    assert_close(y32, ref, what=(case, T, "fp32 out"))
    assert_close(y, ref, what=(case, T, "bf16 out"))


@pytest.mark.parametrize("spread", [64, 256])
@pytest.mark.parametrize("T", [50, 200])
def test_dense_tiles_within_row_scale_spread(spread, T, monkeypatch):
    """The dense tiles' fp16 weights carry one power-of-two scale per row (the largest |s|, |b| of the row), so a row
    whose scale groups differ a lot keeps its small groups' weights near fp16's subnormal range. Here the first scale
    group of every row of every projection has `spread` times the others' scale and the activations entering that
    group are 100x smaller, so the output comes from the small groups: it must still meet the gate (the decode bounds
    |w'| by 2^-1, so weights reach the subnormal range only 2^13 below the row's largest). T=200 runs the dense tiles
    on both projections, T=50 the wave gate/up into the dense down."""
    from moelab_amd.experts import make_state, unpack
    monkeypatch.setenv("MOE_DENSE", "1")
    sh = shape_("spread", 256, 384, 4, 2)
    base = packed_state(sh, 21)
    parts = {n: list(unpack(base, n)) for n in ("g", "u", "d")}
    for n in parts:
        sc = parts[n][1].float()
        sc[..., 0] *= spread
        parts[n][1] = sc.to(torch.bfloat16)
        parts[n][2] = (parts[n][1].float() * -8.0).to(torch.bfloat16)
    s = make_state("int4", parts["g"], parts["u"], parts["d"])
    x, idx, wts = inputs(sh, T, "uniform", seed=T)
    x = x.float()
    x[:, :64] *= 0.01     # the large group's inputs of the gate/up
    x = x.to(torch.bfloat16)
    print(f"case dense scale spread {spread} T={T}", flush=True)
    y32 = grouped(s, x, idx, wts, out_dtype=torch.float32)
    assert_close(y32, oracle_y(s, x, idx, wts), what=("spread", spread, T))


@pytest.mark.parametrize("fmt", ["int4", "mxfp4"])
@pytest.mark.parametrize("N,K", [(16, 128), (48, 192), (32, 2048), (48, 2880)])
def test_tiles_pack_matches_host_restatement(fmt, N, K):
    """moe_tiles_pack on the device == formats.pack_tiles_ref, byte for byte (incl. K % 128 == 64 padding)."""
    from moelab_amd import _lib, formats
    from moelab_amd.experts import FMT, tile_bytes
    g = torch.Generator(device=DEV).manual_seed(N + K)
    E = 3
    parts = (formats.random_int4 if fmt == "int4" else formats.random_mxfp4)(E, N, K, generator=g, device=DEV)
    rows = formats.pack_rows(fmt, *parts)
    tiles = torch.full((E * tile_bytes(fmt, N, K),), 0xA5, dtype=torch.uint8, device=DEV)
    print(f"case pack fmt={fmt} N={N} K={K}", flush=True)
    _lib.check("moe_tiles_pack", _lib.lib().moe_tiles_pack(FMT[fmt], E, N, K, _lib.ptr(rows), _lib.ptr(tiles),
                                                           _lib.stream_of(DEV)))
    torch.cuda.synchronize()
    assert torch.equal(tiles.cpu(), formats.pack_tiles_ref(fmt, rows, K))


def grouped(s, x, idx, wts, out_dtype=None):
    from moelab_amd import _lib
    from moelab_amd.experts import run_experts
    return run_experts(s, x, idx, wts, path=_lib.PATH_GROUPED, out_dtype=out_dtype)


@pytest.mark.parametrize("T", [2, 9, 33, 65, 130])
def test_grouped_without_tile_copies(T):
    """The grouped path forced on row records only (no tile-major copies): the row-major MFMA tiles."""
    from moelab_amd.experts import drop_tiles
    sh = shape_("r", 256, 320, 16, 4)
    s = drop_tiles(packed_state(sh, 7))
    x, idx, wts = inputs(sh, T, "zipf", seed=T)
    print(f"case grouped-rows T={T}", flush=True)
    y = grouped(s, x, idx, wts, out_dtype=torch.float32)
    assert_close(y, oracle_y(s, x, idx, wts), what=("rows", T))


@pytest.mark.parametrize("T", [2, 16, 40, 120])
def test_tile_copies_and_row_records_agree(T):
    """The grouped path forced with and without the tile-major copies (wave tiles vs row-major tiles): each
    within the gate of the oracle, and of each other up to fp32 reassociation (T * k / E <= 32 tokens per
    expert: the wave tiles; more goes to the dense tiles, tested below)."""
    from moelab_amd.experts import drop_tiles
    sh = shape_("t", 512, 384, 16, 4)
    s = packed_state(sh, 9)
    x, idx, wts = inputs(sh, T, "uniform", seed=T)
    print(f"case tiles-vs-rows T={T}", flush=True)
    y1 = grouped(s, x, idx, wts, out_dtype=torch.float32)
    y2 = grouped(drop_tiles(s), x, idx, wts, out_dtype=torch.float32)
    ref = oracle_y(s, x, idx, wts)
    assert_close(y1, ref, what=("tiles", T))
    assert_close(y2, ref, what=("rows", T))
    rms = float(y1.pow(2).mean().sqrt())
    assert float((y1 - y2).abs().max()) <= 1e-3 * rms


DENSE_CASES = [
    # (name, d, F, E, k, T, routing): tokens per expert T k / E > 32 selects the dense tiles
    ("even", 256, 384, 4, 2, 100, "uniform"),       # 50 per expert
    ("big", 512, 1024, 8, 2, 600, "uniform"),       # 150 per expert: three passes of 64; down split over K
    ("odd-K", 320, 448, 4, 2, 180, "zipf"),         # K % 128 == 64 both ways, N % 128 != 0, uneven counts
    ("one-expert", 256, 384, 1, 1, 2100, "uniform"),  # 2100 tokens: more passes than the grid's z extent
    ("k=E", 192, 256, 4, 4, 40, "uniform"),         # every token in every expert
    ("split-odd", 256, 1152, 4, 2, 200, "zipf"),    # down split over K in two parts of 5 and 4 slices
]


@pytest.mark.parametrize("case", DENSE_CASES, ids=lambda c: c[0])
def test_dense_tiles(case, monkeypatch):
    """Many tokens per expert: the dense tiles (gate/up: exact codes on bf16 MFMA with the per-group fp32 fold;
    h in fp16 with a power-of-two exponent per slot and 128-input slice; down: W_down dequantised to fp16 on f16
    MFMA; 64 tokens per pass) against the oracle at the north-star gate. MOE_DENSE=1 keeps them on at these small
    shapes (by default a grid this small goes to the wave tiles)."""
    monkeypatch.setenv("MOE_DENSE", "1")
    name, d, f, E, k, T, routing = case
    sh = shape_(name, d, f, E, k)
    s = packed_state(sh, 31)
    x, idx, wts = inputs(sh, T, routing, seed=T)
    print(f"case dense {name} T={T}", flush=True)
    y32 = grouped(s, x, idx, wts, out_dtype=torch.float32)
    y = grouped(s, x, idx, wts)
    torch.cuda.synchronize()
    ref = oracle_y(s, x, idx, wts)
    assert_close(y32, ref, what=("dense", name, "fp32 out"))
    assert_close(y, ref, what=("dense", name, "bf16 out"))


@pytest.mark.parametrize("T", [50, 150])
def test_dense_tiles_fp16_range(T, monkeypatch):
    """The dense path's fp16 activations past fp16's range. Tokens scaled by 1000 give |h| far above 65504
    (checked on the oracle's own h): their h16 rows carry exponents. Tokens scaled by 1e5 are beyond fp16
    themselves: their x16 rows carry exponents too. The other tokens stay small, so one call mixes rows with and
    without exponents (and slots whose slices need different exponents); each group of tokens meets the gate
    against its own RMS. T=50 (25 slots per expert) runs the wave gate/up with h16 output into the dense down,
    T=150 the dense tiles on both projections."""
    monkeypatch.setenv("MOE_DENSE", "1")
    sh = shape_("big-h", 256, 640, 4, 2)
    s = packed_state(sh, 35)
    x, idx, wts = inputs(sh, T, "uniform", seed=9)
    big = torch.zeros(T, dtype=torch.bool, device=DEV)
    big[::6] = True
    huge = torch.zeros(T, dtype=torch.bool, device=DEV)
    huge[3::12] = True
    x = x.float()
    x = torch.where(big[:, None], x * 1000.0, torch.where(huge[:, None], x * 1e5, x)).to(torch.bfloat16)
    xs = orc.bf16_bits_to_f32(np_u16(x))
    wg, wu = deq(s, "g", experts=[int(idx[0, 0])])[0], deq(s, "u", experts=[int(idx[0, 0])])[0]
    h0 = orc.act_fn(xs[0] @ wg.T, xs[0] @ wu.T, 0)
    assert np.abs(h0).max() > 2 * 65504.0 and np.abs(xs[3]).max() > 65504.0
    print(f"case dense fp16 range T={T}", flush=True)
    y = grouped(s, x, idx, wts, out_dtype=torch.float32)
    ref = oracle_y(s, x, idx, wts)
    small = ~(big | huge)
    for sel, what in ((big, "h beyond fp16"), (huge, "x beyond fp16"), (small, "small tokens")):
        assert_close(y[sel], ref[sel.cpu().numpy()], what=what)


MIXED_CASES = [
    # (name, d, F, E, k, T, routing): 16 < T k / E <= 32 with MOE_DENSE=1: wave gate/up (h16 out) + dense down
    ("mix", 256, 384, 4, 2, 50, "uniform"),       # 25 per expert
    ("mix-odd", 320, 448, 4, 2, 60, "zipf"),      # K % 128 == 64 both ways, uneven counts
    ("mix-many", 512, 1152, 16, 4, 100, "uniform"),  # 25 per expert over 16 experts; the down split over K
]


@pytest.mark.parametrize("d,wave_rows", [(1728, 96), (2048, 128), (1472, 64)])
def test_wave_down_row_tiles(d, wave_rows):
    """The wave down takes 8 row tiles per wave where d % 128 == 0, 6 where d % 96 == 0, else 4 (each only while
    its grid keeps >= 1024 waves: d / rows per wave x the pass list's bound of 72 at T=32, E=64, k=4)."""
    assert (d // wave_rows) * (128 // 16 + 64) >= 1024 or wave_rows == 64
    sh = shape_("wd", d, 256, 64, 4)
    s = packed_state(sh, d)
    x, idx, wts = inputs(sh, 32, "uniform", seed=d)
    print(f"case wave-down d={d} rows/wave={wave_rows}", flush=True)
    assert_close(grouped(s, x, idx, wts, out_dtype=torch.float32), oracle_y(s, x, idx, wts), what=("wave down", d))


@pytest.mark.parametrize("case", MIXED_CASES, ids=lambda c: c[0])
def test_wave_gate_up_dense_down(case, monkeypatch):
    """Mid loads: the wave tiles' gate/up writes h as fp16 with per-32-row exponents, the exponent pass makes
    one exponent per slot, the dense tiles' down reads it on its own 64-token pass list."""
    monkeypatch.setenv("MOE_DENSE", "1")
    name, d, f, E, k, T, routing = case
    sh = shape_(name, d, f, E, k)
    s = packed_state(sh, 37)
    x, idx, wts = inputs(sh, T, routing, seed=T)
    print(f"case mixed {name} T={T}", flush=True)
    y32 = grouped(s, x, idx, wts, out_dtype=torch.float32)
    y = grouped(s, x, idx, wts)
    ref = oracle_y(s, x, idx, wts)
    assert_close(y32, ref, what=("mixed", name, "fp32 out"))
    assert_close(y, ref, what=("mixed", name, "bf16 out"))


def test_dense_tiles_match_row_tiles(monkeypatch):
    """Dense tiles vs the LDS-staged row tiles (MOE_DENSE=0) on the same inputs: both at the gate, and within
    the gate of each other (the row tiles keep h as two bf16 planes and W_down exact)."""
    sh = shape_("dr", 512, 768, 8, 2)
    s = packed_state(sh, 33)
    x, idx, wts = inputs(sh, 400, "zipf", seed=5)
    print("case dense-vs-rows T=400", flush=True)
    monkeypatch.setenv("MOE_DENSE", "1")
    y1 = grouped(s, x, idx, wts, out_dtype=torch.float32)
    monkeypatch.setenv("MOE_DENSE", "0")
    y2 = grouped(s, x, idx, wts, out_dtype=torch.float32)
    ref = oracle_y(s, x, idx, wts)
    assert_close(y1, ref, what="dense")
    assert_close(y2, ref, what="rows")
    rms = float(y2.pow(2).mean().sqrt())
    assert float((y1 - y2).abs().max()) <= 1e-2 * rms


def shared_state(d, Fs, S, seed, fmt="int4"):
    from moelab_amd import formats
    from moelab_amd.experts import make_state
    g = torch.Generator(device=DEV).manual_seed(seed)
    rnd = formats.random_int4 if fmt == "int4" else formats.random_mxfp4
    return make_state(fmt, rnd(S, Fs, d, generator=g, device=DEV), rnd(S, Fs, d, generator=g, device=DEV),
                      rnd(S, d, Fs, generator=g, device=DEV))


@pytest.mark.parametrize("gated", [False, True])
@pytest.mark.parametrize("T", [1, 5, 40])
def test_shared_experts(T, gated):
    """Routed + always-on shared experts (DeepSeek ungated, reference e2e.py:146-147; Qwen-style sigmoid gate,
    e2e.py:66-68) through moe_shared_experts_run, against the oracle's shared list."""
    sh = shape_("s", 256, 384, 16, 4)
    s = packed_state(sh, 21)
    s["shared"] = shared_state(sh.d, 320, 2, seed=22)
    if gated:
        g = torch.Generator(device=DEV).manual_seed(23)
        s["shared_gate"] = (torch.randn(sh.d, generator=g, device=DEV) * 0.05).to(torch.bfloat16)
    x, idx, wts = inputs(sh, T, "uniform", seed=T)
    print(f"case shared T={T} gated={gated}", flush=True)
    y32 = q4().run(s, x, idx, wts, out_dtype=torch.float32)
    y = q4().run(s, x, idx, wts)
    ref = oracle_y(s, x, idx, wts)
    assert_close(y32, ref, what=("shared fp32", T, gated))
    assert_close(y, ref, what=("shared bf16", T, gated))


def test_shared_experts_argument_errors():
    from moelab_amd import _lib
    from moelab_amd.experts import _desc
    s = shared_state(256, 320, 2, seed=24)
    L = _lib.lib()
    x = torch.zeros((4, 256), dtype=torch.bfloat16, device=DEV)
    y = torch.empty_like(x)
    desc = _desc(s)
    assert L.moe_shared_experts_run(desc, _lib.ptr(x), 0, 4, 0, None, _lib.ptr(y), 0, None, None, 0, None) == \
        _lib.MOE_ERR_WORKSPACE
    assert L.moe_shared_experts_run(desc, _lib.ptr(x), 3, 4, 0, None, _lib.ptr(y), 0, None, _lib.ptr(y), 1 << 20,
                                    None) == _lib.MOE_ERR_DTYPE


@pytest.mark.parametrize("nt", ["1", "2"])
def test_wave_tiles_for_many_tokens(nt, monkeypatch):
    """Many tokens per expert on a grid too small for the dense tiles (a few shared-expert-like experts): the
    wave tiles with 16- or 32-token passes, several passes per expert, against the oracle."""
    monkeypatch.setenv("MOE_DENSE", "-1")
    monkeypatch.setenv("MOE_WAVE_NT", nt)
    sh = shape_("w", 256, 384, 2, 2, )
    s = packed_state(sh, 35)
    x, idx, wts = inputs(sh, 150, "uniform", seed=9)
    print(f"case wave-many nt={nt}", flush=True)
    y = grouped(s, x, idx, wts, out_dtype=torch.float32)
    assert_close(y, oracle_y(s, x, idx, wts), what=("wave many", nt))


@pytest.mark.parametrize("ks", [1, 2, 3, 4])
def test_dense_down_k_parts(ks, monkeypatch):
    """The dense down projection split into 1-4 K parts (MOE_DENSE_KSPLIT; the combine sums the parts' planes):
    each at the gate, and every split within fp32 reassociation of the unsplit result."""
    monkeypatch.setenv("MOE_DENSE", "1")
    sh = shape_("ks", 256, 1152, 4, 2)   # 9 K slices: parts of 9, 5+4, 3+3+3; 4 asks for 3+3+3 as well
    s = packed_state(sh, 41)
    x, idx, wts = inputs(sh, 200, "zipf", seed=3)
    print(f"case dense ksplit={ks}", flush=True)
    monkeypatch.setenv("MOE_DENSE_KSPLIT", "1")
    y1 = grouped(s, x, idx, wts, out_dtype=torch.float32)
    monkeypatch.setenv("MOE_DENSE_KSPLIT", str(ks))
    y = grouped(s, x, idx, wts, out_dtype=torch.float32)
    assert_close(y, oracle_y(s, x, idx, wts), what=("ksplit", ks))
    rms = float(y1.pow(2).mean().sqrt())
    assert float((y - y1).abs().max()) <= 1e-5 * rms


@pytest.mark.parametrize("T,dense", [(1, "0"), (32, "0"), (50, "1"), (150, "1")])
def test_stages_match_one_call(T, dense, monkeypatch):
    """moe_experts_run_stages: GATE_UP then DOWN as two calls on one workspace gives the one-call result bit for
    bit (the per-slot GEMVs at T=1, the wave tiles, the wave gate/up into the dense down on two pass lists, the
    dense tiles with their x16 / h16 state in between)."""
    from moelab_amd import _lib
    from moelab_amd.experts import run_experts
    monkeypatch.setenv("MOE_DENSE", dense)
    sh = shape_("st", 256, 640, 4, 2)
    s = packed_state(sh, 43)
    x, idx, wts = inputs(sh, T, "uniform", seed=T)
    print(f"case stages T={T} dense={dense}", flush=True)
    y_all = run_experts(s, x, idx, wts, out_dtype=torch.float32)
    out = torch.empty_like(y_all)
    run_experts(s, x, idx, wts, out=out, out_dtype=torch.float32, stages=_lib.STAGE_GATE_UP)
    run_experts(s, x, idx, wts, out=out, out_dtype=torch.float32, stages=_lib.STAGE_DOWN)
    torch.cuda.synchronize()
    assert torch.equal(out, y_all)
