"""fp16 and fp32 activations through the variant contract (x.dtype preserved), against the oracle.

The reference dispatcher sends bf16 and fp16 to its MMA tiles and fp32 to its exact scalar tiles
(reference metal_q4_moe.py:62-64, metal_q4_tiles_b.py:128-250) and tests both float dtypes
(tests/test_fp32_activations.py:14-22 at T = 1, 3, 16 one-hot, 32; tests/test_mlx_variants.py:30-42). Here
fp16 and fp32 x enter the gate/up products as 2 or 3 bf16 planes whose sum is x exactly (k_x_planes), on the
per-slot GEMV, the wave tiles and the row-record tiles; the int4 dense tiles take fp16 x directly (x16). Every
case runs the north-star gate on the fp32 output and on the x.dtype output (plus its own rounding); the
exactness cases show the planes carry every input bit: the fp32-x result sits at fp32-accumulation distance
from the oracle on the fp32 x, far closer than the same call on x rounded to bf16.
"""
import numpy as np
import pytest
import torch

from helpers import assert_close, oracle_y, orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def shape_(name, d, f, E, k):
    from moelab_amd.shapes import MoEShape
    return MoEShape(name, d=d, f=f, E=E, k=k)


def inputs(sh, T, dtype, routing="uniform", seed=0, scale=1.0):
    from moelab_amd.problem import make_routing
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.standard_normal((T, sh.d)).astype(np.float32) * scale).to(DEV, dtype)
    idx, wts = make_routing(T, sh.E, sh.k, routing, rng)
    return x, torch.from_numpy(idx).to(DEV), torch.from_numpy(wts).to(DEV)


def int4_state(sh, seed, tiles=True):
    from moelab_amd.experts import drop_tiles
    from moelab_amd.problem import baseline_int4_layer
    s = baseline_int4_layer(sh, seed, DEV, router=False)
    return s if tiles else drop_tiles(s)


def check_variant(mod, s, x, idx, wts, what, act=None):
    kw = {} if act is None else {"act": act}
    y = mod.run(s, x, idx, wts, **kw)
    y32 = mod.run(s, x, idx, wts, out_dtype=torch.float32, **kw)
    torch.cuda.synchronize()
    assert y.dtype == x.dtype and y.shape == x.shape, (y.dtype, x.dtype)
    ref = oracle_y(s, x, idx, wts, **({"act": kw["act"]} if "act" in kw else {}))
    assert_close(y32, ref, what=(what, "fp32 out"))
    assert_close(y, ref, what=(what, "x.dtype out"))
    return y32, ref


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["fp16", "fp32"])
@pytest.mark.parametrize("T,routing", [(1, "uniform"), (3, "uniform"), (16, "one_hot"), (32, "uniform"),
                                       (100, "zipf")])
def test_int4_variant_float_activations(dtype, T, routing):
    """reference tests/test_fp32_activations.py:14-22 (T = 1, 3, 16 one-hot, 32) plus a loaded zipf case."""
    from moelab_amd.variants import hip_q4_moe as q4
    sh = shape_("a", 512, 384, 16, 4)
    s = int4_state(sh, 1)
    x, idx, wts = inputs(sh, T, dtype, routing, seed=T)
    print(f"case int4 {dtype} T={T} {routing}", flush=True)
    check_variant(q4, s, x, idx, wts, (dtype, T, routing))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["fp16", "fp32"])
@pytest.mark.parametrize("T", [9, 40])
def test_int4_row_record_tiles_float_activations(dtype, T):
    """The grouped path without tile-major copies (k_tile, LDS-staged row records) on the x planes."""
    from moelab_amd import _lib
    from moelab_amd.experts import run_experts
    sh = shape_("r", 320, 448, 8, 3)
    s = int4_state(sh, 2, tiles=False)
    x, idx, wts = inputs(sh, T, dtype, "zipf", seed=T)
    print(f"case rows {dtype} T={T}", flush=True)
    y = run_experts(s, x, idx, wts, path=_lib.PATH_GROUPED, out_dtype=torch.float32)
    assert_close(y, oracle_y(s, x, idx, wts), what=(dtype, T))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["fp16", "fp32"])
@pytest.mark.parametrize("T", [50, 200])
def test_int4_dense_load_float_activations(dtype, T, monkeypatch):
    """Loads that take the dense down (25 and 100 slots per expert, MOE_DENSE=1): fp16 x feeds the dense gate/up
    directly as x16; fp32 x keeps the exact-operand wave gate/up on its 3 planes, then the dense down."""
    from moelab_amd.variants import hip_q4_moe as q4
    monkeypatch.setenv("MOE_DENSE", "1")
    sh = shape_("dn", 256, 384, 4, 2)
    s = int4_state(sh, 3)
    x, idx, wts = inputs(sh, T, dtype, seed=T)
    print(f"case dense-load {dtype} T={T}", flush=True)
    check_variant(q4, s, x, idx, wts, (dtype, T))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["fp16", "fp32"])
@pytest.mark.parametrize("T", [1, 8, 40])
def test_mxfp4_and_gptoss_float_activations(dtype, T):
    """MXFP4 (hip_mxfp4_moe) and gpt-oss (biases, clamped SwiGLU) with fp16 / fp32 x."""
    from moelab_amd.problem import baseline_mxfp4_layer
    from moelab_amd.variants import hip_mxfp4_gptoss as gpt, hip_mxfp4_moe as mx
    sh = shape_("m", 512, 384, 8, 4)
    x, idx, wts = inputs(sh, T, dtype, seed=T)
    print(f"case mxfp4 {dtype} T={T}", flush=True)
    s = baseline_mxfp4_layer(sh, 4, DEV, biases=False, router=False)
    check_variant(mx, s, x, idx, wts, ("mxfp4", dtype, T))
    sg = baseline_mxfp4_layer(sh, 5, DEV, biases=True, router=False)
    sg["act"] = 1
    y = gpt.run(sg, x, idx, wts)
    y32 = gpt.run(sg, x, idx, wts, out_dtype=torch.float32)
    assert y.dtype == dtype
    ref = oracle_y(sg, x, idx, wts, act=2)
    assert_close(y32, ref, what=("gptoss", dtype, T, "fp32 out"))
    assert_close(y, ref, what=("gptoss", dtype, T, "x.dtype out"))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["fp16", "fp32"])
@pytest.mark.parametrize("T", [1, 12])
def test_shared_experts_and_residual_float_activations(dtype, T):
    """Gated shared experts (the gate dot reads x in its own dtype) and a residual of x.dtype."""
    from moelab_amd import formats
    from moelab_amd.experts import make_state
    from moelab_amd.variants import hip_q4_moe as q4
    sh = shape_("s", 256, 384, 16, 4)
    s = int4_state(sh, 6)
    g = torch.Generator(device=DEV).manual_seed(7)
    s["shared"] = make_state("int4", *(formats.random_int4(2, n, k, generator=g, device=DEV)
                                       for n, k in ((320, 256), (320, 256), (256, 320))))
    s["shared_gate"] = (torch.randn(sh.d, generator=g, device=DEV) * 0.05).to(torch.bfloat16)
    x, idx, wts = inputs(sh, T, dtype, seed=T)
    res = torch.randn((T, sh.d), device=DEV).to(dtype)
    print(f"case shared {dtype} T={T}", flush=True)
    y = q4.run(s, x, idx, wts, residual=res)
    assert y.dtype == dtype
    ref = oracle_y(s, x, idx, wts) + res.float().cpu().numpy()
    assert_close(q4.run(s, x, idx, wts, residual=res.float(), out_dtype=torch.float32), ref, what=(dtype, T))
    assert_close(y, ref, what=(dtype, T, "x.dtype out"))


@pytest.mark.parametrize("T,path", [(1, 1), (32, 2), (40, 2)], ids=["T1-slots", "T32-wave", "T40-rows"])
def test_fp32_activations_reach_the_products_exactly(T, path):
    """fp32 x with bits beyond bf16: the result on the 3 planes is within fp32-accumulation distance of the
    oracle on that fp32 x (1e-4 RMS, h carried at 16 bits), while the same call on x rounded to bf16 misses it by
    far more (the rounding alone moves the outputs ~1e-3 RMS): no input bit is dropped on the way in."""
    from moelab_amd.experts import drop_tiles, run_experts
    sh = shape_("ex", 512, 384, 16, 4)
    s = int4_state(sh, 8)
    if T == 40:
        s = drop_tiles(s)
    x, idx, wts = inputs(sh, T, torch.float32, seed=11)
    x = x * (1.0 + 2.0 ** -10)   # plenty of mantissa bits below bf16's 8
    ref = oracle_y(s, x, idx, wts)
    y = run_experts(s, x, idx, wts, path=path, out_dtype=torch.float32)
    yb = run_experts(s, x.to(torch.bfloat16), idx, wts, path=path, out_dtype=torch.float32)
    torch.cuda.synchronize()
    e = orc.error_metrics(y.cpu().numpy(), ref)
    eb = orc.error_metrics(yb.cpu().numpy(), ref)
    print(f"case exact T={T}: fp32 planes {e['max_abs'] / e['rms_ref']:.2e} RMS, bf16 "
          f"{eb['max_abs'] / eb['rms_ref']:.2e} RMS", flush=True)
    assert e["max_abs"] <= 1e-4 * e["rms_ref"], e
    assert eb["max_abs"] >= 10 * e["max_abs"], (e, eb)
