"""MXFP4 and gpt-oss expert paths on the GPU vs the CPU oracle (fp64 loop on dequantised weights).

Gate: max |y - y_ref| <= 1e-2 * RMS(y_ref) on the fp32 output, plus the bf16 output's own rounding
(helpers.assert_close). Cases follow reference tests/test_edge_cases.py (dispatch boundaries, shapes,
zero weights, one expert set), tests/test_mxfp4_large_scales.py (E8M0 bytes >= 129) and
tests/test_gptoss_patch.py:88-113 (bytes >= 133, biases, clamped SwiGLU)."""
import numpy as np
import pytest
import torch

from helpers import assert_close, deq, oracle_y, orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def mx():
    from moelab_amd.variants import hip_mxfp4_moe
    return hip_mxfp4_moe


def gpt():
    from moelab_amd.variants import hip_mxfp4_gptoss
    return hip_mxfp4_gptoss


def shape_(name, d, f, E, k):
    from moelab_amd.shapes import MoEShape
    return MoEShape(name, d=d, f=f, E=E, k=k)


def packed_state(shape, seed, biases=False, scale_bytes=None):
    from moelab_amd.problem import baseline_mxfp4_layer
    s = baseline_mxfp4_layer(shape, seed, DEV, biases=biases, router=False)
    if scale_bytes is not None:   # re-pack with chosen E8M0 bytes
        from moelab_amd import formats
        from moelab_amd.experts import unpack
        g = torch.Generator(device=DEV).manual_seed(seed)
        for n in ("g", "u", "d"):
            codes, sc = unpack(s, n)
            lo, hi = scale_bytes
            sc = torch.randint(lo, hi + 1, sc.shape, generator=g, device=DEV).to(torch.uint8)
            s[n] = formats.pack_rows("mxfp4", codes, sc)
        s.pop("_c", None)
        if "gt" in s:   # the tile-major copies follow the new records
            from moelab_amd.experts import add_tiles
            add_tiles(s)
    return s


def inputs(shape, T, routing="uniform", seed=0, scale=1.0):
    from moelab_amd.problem import make_routing
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.standard_normal((T, shape.d)).astype(np.float32) * scale).to(DEV, torch.bfloat16)
    idx, wts = make_routing(T, shape.E, shape.k, routing, rng)
    return x, torch.from_numpy(idx).to(DEV), torch.from_numpy(wts).to(DEV)


@pytest.fixture(params=["default", "forced-custom"])
def policy(request, monkeypatch):
    if request.param == "forced-custom":
        monkeypatch.setattr(mx(), "LOAD_MAX", 1e9)

        def no_fallback(*a, **k):
            raise AssertionError("fallback ran in forced-custom mode")
        monkeypatch.setattr(mx(), "gather_moe", no_fallback)
    return request.param


def check(shape, T, routing="uniform", seed=0, idx=None, wts=None, act=0, scale=1.0, state=None, biases=False,
          scale_bytes=None):
    s = state if state is not None else packed_state(shape, seed + 200, biases=biases, scale_bytes=scale_bytes)
    x, i0, w0 = inputs(shape, T, routing, seed, scale)
    idx = i0 if idx is None else torch.as_tensor(idx, dtype=torch.int32, device=DEV)
    wts = w0 if wts is None else torch.as_tensor(wts, dtype=torch.float32, device=DEV)
    print(f"case mxfp4 shape={shape} T={T} routing={routing} act={act}", flush=True)
    y = mx().run(s, x, idx, wts, act=act)
    y32 = mx().run(s, x, idx, wts, act=act, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = oracle_y(s, x, idx, wts, act)
    assert_close(y32, ref, what=(shape, T, "fp32 out"))
    assert_close(y, ref, what=(shape, T, "bf16 out"))
    return y, s, x, idx, wts


@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 7, 8, 9, 15, 17, 31, 63, 65, 127, 129, 257])
def test_dispatch_boundaries(policy, T):
    check(shape_("q", 256, 384, 16, 4), T, routing="zipf", seed=T)


SHAPES = [("d192", 192, 256, 8, 2), ("f320", 256, 320, 8, 2), ("odd", 320, 448, 8, 3), ("k1", 128, 256, 8, 1),
          ("kE", 128, 256, 4, 4), ("E1", 128, 256, 1, 1), ("gptoss-like", 2880, 2880, 4, 2)]


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
    assert float(y[0].float().abs().max()) == 0.0


@pytest.mark.parametrize("T", [2, 8, 32])
def test_all_tokens_one_expert_set(policy, T):
    check(shape_("o", 256, 256, 16, 4), T, idx=np.tile([[3, 7, 0, 15]], (T, 1)))


@pytest.mark.parametrize("lo,hi", [(120, 140), (129, 140), (135, 145), (1, 20)])
@pytest.mark.parametrize("T", [1, 9])
def test_e8m0_scale_regimes(lo, hi, T):
    """E8M0 bytes >= 129 overflowed a half-precision scale in the reference (test_mxfp4_large_scales.py:22-34);
    here the scale is an fp32 power of two applied after the dot, exact for every byte 1..254."""
    sh = shape_("s", 256, 256, 8, 2)
    s = packed_state(sh, 3, scale_bytes=(lo, hi))
    x, idx, wts = inputs(sh, T, seed=3)
    ref = oracle_y(s, x, idx, wts)
    assert np.isfinite(ref).all() and np.abs(ref).max() < 1e30, "case must stay inside the fp32 range"
    y32 = mx().run(s, x, idx, wts, out_dtype=torch.float32)
    assert_close(y32, ref, what=(lo, hi))


@pytest.mark.parametrize("T", [1, 3, 9, 32, 100])
@pytest.mark.parametrize("act", [0, 1])
def test_gptoss_biases_and_clamped_glu(T, act):
    sh = shape_("g", 704, 704, 8, 4)
    from moelab_amd.problem import baseline_mxfp4_layer
    s = baseline_mxfp4_layer(sh, 4, DEV, biases=True, router=False)
    s["act"] = act
    x, idx, wts = inputs(sh, T, seed=4, scale=3.0)   # larger activations reach the clamp at 7
    y = gpt().run(s, x, idx, wts, out_dtype=torch.float32)
    ref = oracle_y(s, x, idx, wts, act=2 if act == 1 else 0)
    assert_close(y, ref)
    # the module's own fp32 reference agrees with the oracle (reference metal_mxfp4_gptoss.py:110-126)
    assert_close(gpt().reference(s, x.float(), idx, wts), ref, tol=2e-3)


@pytest.mark.parametrize("T", [1, 5])
def test_gptoss_small_h(T):
    """The per-slot path keeps the gpt-oss GLU's h as one fp16 plane holding h 2^8 (|h| <= 56 by the clamps).
    With activations 1e-6 of the usual size every |h| is near 2^-21, below fp16's smallest normal 2^-14: an
    unscaled fp16 h would keep ~3 significant bits there (about 10% of the output RMS), the scaled one 11."""
    sh = shape_("gs", 256, 256, 8, 4)
    s = packed_state(sh, 7)
    s["act"] = 1
    x, idx, wts = inputs(sh, T, seed=7, scale=1e-6)
    ref = oracle_y(s, x, idx, wts, act=2)
    assert 0 < np.sqrt(np.mean(ref ** 2)) < 1e-5, "the case must keep h far below fp16's normal range"
    assert_close(gpt().run(s, x, idx, wts, out_dtype=torch.float32), ref)


@pytest.mark.parametrize("T", [1, 3])
def test_gptoss_per_slot_outputs(T):
    """Unweighted per-slot outputs (run_slots) with the gpt-oss GLU and biases: the per-slot path's fp16 h plane
    (h 2^8) is scaled back before the down's bias and the per-slot store, as before the combine."""
    sh = shape_("gp", 256, 256, 8, 4)
    s = packed_state(sh, 8, biases=True)
    x, idx, _ = inputs(sh, T, seed=8, scale=3.0)   # activations large enough to reach the clamps
    ys = mx().run_slots(s, x, idx, act=2)
    assert ys.shape == (T * 4, 256)
    ones = torch.ones((T, 1), device=DEV)
    for j in range(4):
        ref = oracle_y(s, x, idx[:, j:j + 1], ones, act=2)
        assert_close(ys.view(T, 4, 256)[:, j], ref, what=(T, j))


@pytest.mark.parametrize("T", [1, 3])
def test_gptoss_per_slot_stages_split(T):
    """The per-slot path as two calls (gate/up, then down on the h the first left in the workspace) equals the whole
    call bit for bit with the gpt-oss GLU, whose h travels as one fp16 plane between the stages."""
    from moelab_amd import _lib
    from moelab_amd.experts import run_experts
    sh = shape_("gs2", 320, 448, 8, 4)
    s = packed_state(sh, 9, biases=True)
    x, idx, wts = inputs(sh, T, seed=9, scale=3.0)
    sl = _lib.PATH_SLOTS
    y = run_experts(s, x, idx, wts, act=2, path=sl, out_dtype=torch.float32)
    run_experts(s, x, idx, wts, act=2, path=sl, out_dtype=torch.float32, stages=_lib.STAGE_GATE_UP)
    y2 = run_experts(s, x, idx, wts, act=2, path=sl, out_dtype=torch.float32, stages=_lib.STAGE_DOWN)
    assert torch.equal(y, y2)
    assert_close(y, oracle_y(s, x, idx, wts, act=2))


def test_gptoss_large_scale_bytes():
    """gpt-oss checkpoints reach E8M0 bytes >= 133 (reference test_gptoss_patch.py:88-113)."""
    sh = shape_("gl", 256, 256, 8, 4)
    from moelab_amd import formats
    from moelab_amd.experts import unpack
    s = packed_state(sh, 5, biases=True, scale_bytes=(125, 137))
    s["act"] = 1
    x, idx, wts = inputs(sh, 6, seed=5)
    assert int(unpack(s, "d")[1].max()) >= 133
    assert_close(gpt().run(s, x, idx, wts, out_dtype=torch.float32), oracle_y(s, x, idx, wts, act=2))
    assert formats.E2M1_VALUES[-1] == 6.0


def test_prepare_dequant_roundtrip():
    from moelab_amd import backend
    sh = shape_("pd", 256, 384, 8, 2)
    wg, wu, wd = backend.make_weights(sh, "bfloat16", seed=3)
    s = mx().prepare(wg, wu, wd)
    x, idx, wts = backend.make_inputs(sh, 6, "bfloat16", "uniform", seed=3)
    y = mx().run(s, x, idx, wts)
    rwg, rwu, rwd = mx().dequant(s)
    err = backend.errors(y, backend.reference(rwg, rwu, rwd, x, idx, wts))
    assert err["finite"] and err["rel_fro"] < backend.TOL["bfloat16"], err
    np.testing.assert_allclose(rwg.cpu().numpy(), deq(s, "g"), rtol=1e-6, atol=0)
    rel = float((rwg.float() - wg.float()).norm() / wg.float().norm())
    assert rel < 0.25, rel


@pytest.mark.parametrize("T", [1, 32])
def test_gptoss_full_shape(T):
    """BASELINE config 4 shape: d=2880, F=2880, E=32, k=4, MXFP4 + biases, clamped SwiGLU."""
    from moelab_amd import router
    from moelab_amd.problem import baseline_mxfp4_layer, baseline_x
    from moelab_amd.shapes import SHAPES
    sh = SHAPES["gpt-oss-20b"]
    s = baseline_mxfp4_layer(sh, seed=12, device=DEV)
    s["act"] = 1
    x = baseline_x(T, sh.d, seed=12, device=DEV)
    idx, wts = router.route(x, s["wr"], sh.k)
    y = gpt().run(s, x, idx, wts, out_dtype=torch.float32)
    assert_close(y, oracle_y(s, x, idx, wts, act=2))


@pytest.mark.parametrize("T", [2, 17, 40])
def test_mxfp4_tile_copies_and_row_records_agree(T):
    """MXFP4 grouped path forced with and without the tile-major copies, against the oracle and each other."""
    from moelab_amd import _lib
    from moelab_amd.experts import drop_tiles, run_experts
    sh = shape_("t", 512, 384, 16, 4)
    s = packed_state(sh, 5)
    x, idx, wts = inputs(sh, T, "uniform", seed=T)
    print(f"case mxfp4 tiles-vs-rows T={T}", flush=True)
    y1 = run_experts(s, x, idx, wts, path=_lib.PATH_GROUPED, out_dtype=torch.float32)
    y2 = run_experts(drop_tiles(s), x, idx, wts, path=_lib.PATH_GROUPED, out_dtype=torch.float32)
    ref = oracle_y(s, x, idx, wts)
    assert_close(y1, ref, what=("tiles", T))
    assert_close(y2, ref, what=("rows", T))
    rms = float(y1.pow(2).mean().sqrt())
    assert float((y1 - y2).abs().max()) <= 1e-3 * rms


@pytest.mark.parametrize("case", [("even", 256, 384, 4, 2, 100, "uniform"), ("odd-K", 320, 448, 4, 2, 180, "zipf"),
                                  ("big", 512, 1024, 8, 2, 600, "uniform")], ids=lambda c: c[0])
def test_mxfp4_dense_tiles(case, monkeypatch):
    """MXFP4 with many tokens per expert (T k / E > 32): the dense tiles against the oracle at the gate."""
    from moelab_amd import _lib
    from moelab_amd.experts import run_experts
    monkeypatch.setenv("MOE_DENSE", "1")
    name, d, f, E, k, T, routing = case
    sh = shape_(name, d, f, E, k)
    s = packed_state(sh, 41)
    x, idx, wts = inputs(sh, T, routing, seed=T)
    print(f"case mxfp4 dense {name} T={T}", flush=True)
    y = run_experts(s, x, idx, wts, path=_lib.PATH_GROUPED, out_dtype=torch.float32)
    assert_close(y, oracle_y(s, x, idx, wts), what=("mxfp4 dense", name))
