"""MXFP4 grouped tiles on gfx950's block-scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4): the tile records' raw
E2M1 codes and E8M0 bytes go in as the B operand, the activations as fp8 E4M3 terms with an E8M0 byte per 32
inputs (x: two terms, h = hi + lo: three) as A. Taken by default wherever MXFP4 with bf16 x runs the dense or
the wave tiles; MOE_MXMFMA=0 selects the bf16-MFMA tiles (decoded codes, per-group fp32 fold) for comparison.

Checked against the oracle at the north-star gate and, tighter, within 2e-3 RMS (the instruction's own
accumulation keeps ~1e-4 RMS on these cases); against the bf16-MFMA tiles; on ragged passes, K % 128 == 64
(the last slice's second half is padding), gpt-oss biases and the clamped GLU, E8M0 scale regimes (reference
tests/test_mxfp4_large_scales.py:22-34), the stages as separate calls, and config 4's gpt-oss-20b shape at
T = 512 on sampled token rows (reference metal_mxfp4_moe.py:155-308 is the T >= 8 path this replaces).
"""
import numpy as np
import pytest
import torch

from helpers import assert_close, oracle_y

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def state(name, d, f, E, k, seed, biases=False, scale_bytes=None):
    from moelab_amd.problem import baseline_mxfp4_layer
    from moelab_amd.shapes import MoEShape
    sh = MoEShape(name, d=d, f=f, E=E, k=k)
    s = baseline_mxfp4_layer(sh, seed, DEV, biases=biases, router=False)
    if scale_bytes is not None:   # re-pack with E8M0 bytes drawn from [lo, hi]
        from moelab_amd import formats
        from moelab_amd.experts import add_tiles, unpack
        g = torch.Generator(device=DEV).manual_seed(seed)
        for n in ("g", "u", "d"):
            codes, sc = unpack(s, n)
            lo, hi = scale_bytes
            s[n] = formats.pack_rows("mxfp4", codes, torch.randint(lo, hi + 1, sc.shape, generator=g, device=DEV)
                                     .to(torch.uint8))
        s.pop("_c", None)
        if "gt" in s:
            add_tiles(s)
    return sh, s


def inputs(sh, T, routing, seed, scale=1.0):
    from moelab_amd.problem import make_routing
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.standard_normal((T, sh.d)).astype(np.float32) * scale).to(DEV, torch.bfloat16)
    idx, wts = make_routing(T, sh.E, sh.k, routing, rng)
    return x, torch.from_numpy(idx).to(DEV), torch.from_numpy(wts).to(DEV)


def both(monkeypatch, s, x, idx, wts, act=0, dense="1"):
    """(block-scaled MFMA, bf16-MFMA tiles) on the same call; dense: MOE_DENSE ("1": the dense tiles above 32
    tokens per expert; None: the default choice, the wave tiles up to 32)."""
    from moelab_amd import _lib
    from moelab_amd.experts import run_experts
    if dense is not None:
        monkeypatch.setenv("MOE_DENSE", dense)
    monkeypatch.setenv("MOE_MXMFMA", "1")
    y1 = run_experts(s, x, idx, wts, act=act, path=_lib.PATH_GROUPED, out_dtype=torch.float32)
    monkeypatch.setenv("MOE_MXMFMA", "0")
    y0 = run_experts(s, x, idx, wts, act=act, path=_lib.PATH_GROUPED, out_dtype=torch.float32)
    monkeypatch.delenv("MOE_MXMFMA")
    torch.cuda.synchronize()
    return y1, y0


CASES = [
    # (name, d, F, E, k, T, routing, act, biases)
    ("even", 256, 384, 4, 2, 100, "uniform", 0, False),      # ragged last passes
    ("odd-K", 320, 448, 4, 2, 180, "zipf", 0, False),        # d, F = 64 mod 128: a half slice at the end of K
    ("gptoss-act", 704, 704, 8, 4, 200, "uniform", 2, True),  # biases, clamped SwiGLU, K = 64 mod 128
    ("geglu", 512, 512, 8, 2, 300, "zipf", 1, False),
    ("one-hot", 256, 256, 16, 4, 130, "one_hot", 0, False),  # every token on the same 4 experts: 3 passes each
    ("big", 1024, 1536, 8, 2, 700, "uniform", 0, False),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: c[0])
def test_mxscale_dense_against_oracle(case, monkeypatch):
    name, d, f, E, k, T, routing, act, biases = case
    sh, s = state(name, d, f, E, k, seed=300 + T, biases=biases)
    x, idx, wts = inputs(sh, T, routing, seed=T, scale=3.0 if act == 2 else 1.0)
    print(f"case mxscale {name} T={T}", flush=True)
    y1, y0 = both(monkeypatch, s, x, idx, wts, act=act)
    ref = oracle_y(s, x, idx, wts, act=act)
    e1 = assert_close(y1, ref, what=("block-scaled", name))
    assert_close(y0, ref, what=("bf16 dense", name))
    assert e1["max_abs"] <= 2e-3 * e1["rms_ref"], (name, e1)
    assert not torch.equal(y1, y0), "MOE_MXMFMA made no difference: the block-scaled kernels did not run"


@pytest.mark.parametrize("lo,hi", [(120, 140), (135, 145), (100, 110)])
def test_mxscale_e8m0_regimes(lo, hi, monkeypatch):
    """E8M0 bytes across regimes (the hardware applies them as exponents, as the fp32 fold of the other paths)."""
    sh, s = state("sc", 256, 256, 4, 2, seed=7, scale_bytes=(lo, hi))
    x, idx, wts = inputs(sh, 160, "uniform", seed=lo)
    print(f"case mxscale scales {lo}-{hi}", flush=True)
    y1, y0 = both(monkeypatch, s, x, idx, wts)
    ref = oracle_y(s, x, idx, wts)
    assert np.isfinite(ref).all() and np.abs(ref).max() < 1e30
    e1 = assert_close(y1, ref, what=(lo, hi))
    assert e1["max_abs"] <= 2e-3 * e1["rms_ref"], e1


def test_mxscale_wide_activation_range(monkeypatch):
    """Activations spanning ~2^20 inside a 32-input block (outliers x 1000): the second term carries what the
    first one rounds away."""
    sh, s = state("wr", 512, 512, 4, 2, seed=9)
    x, idx, wts = inputs(sh, 128, "uniform", seed=9)
    xs = x.float()
    xs[:, ::37] *= 1000.0
    x = xs.to(torch.bfloat16)
    print("case mxscale wide range", flush=True)
    y1, _ = both(monkeypatch, s, x, idx, wts)
    e1 = assert_close(y1, oracle_y(s, x, idx, wts), what="wide range")
    assert e1["max_abs"] <= 2e-3 * e1["rms_ref"], e1


def test_mxscale_block_spanning_2_16(monkeypatch):
    """One input of every 32-input block at 2^16 times the others: x's two fp8 terms (each with the block's own E8M0
    scale from its largest residual) then keep the small inputs only to the second term's E4M3 subnormal step,
    2^-20 of the block's largest, not exactly; the output still holds the gate, and the 2e-3 RMS bound."""
    sh, s = state("span", 512, 512, 4, 2, seed=13)
    x, idx, wts = inputs(sh, 96, "uniform", seed=13)
    xs = x.float()
    xs[:, 5::32] = 65536.0 * torch.sign(xs[:, 5::32])
    x = xs.to(torch.bfloat16)
    print("case mxscale block spanning 2^16", flush=True)
    y1, _ = both(monkeypatch, s, x, idx, wts)
    e1 = assert_close(y1, oracle_y(s, x, idx, wts), what="span 2^16")
    assert e1["max_abs"] <= 2e-3 * e1["rms_ref"], e1


def test_mxscale_stages_split(monkeypatch):
    """Gate/up and down as two calls (h kept in the workspace between them) equal the whole call bit for bit."""
    from moelab_amd import _lib
    from moelab_amd.experts import run_experts
    monkeypatch.setenv("MOE_DENSE", "1")
    sh, s = state("st", 384, 448, 4, 2, seed=11)
    x, idx, wts = inputs(sh, 150, "zipf", seed=11)
    g = _lib.PATH_GROUPED
    y = run_experts(s, x, idx, wts, path=g, out_dtype=torch.float32)
    run_experts(s, x, idx, wts, path=g, out_dtype=torch.float32, stages=_lib.STAGE_GATE_UP)
    y2 = run_experts(s, x, idx, wts, path=g, out_dtype=torch.float32, stages=_lib.STAGE_DOWN)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)


def test_mxscale_gptoss20b_T512_sampled():
    """Config 4's gpt-oss-20b shape (d = F = 2880, E = 32, k = 4, biases, clamped SwiGLU) at T = 512: the default
    dispatch takes the block-scaled dense tiles (64 slots per expert); 64 seeded token rows against the oracle."""
    from moelab_amd.problem import baseline_mxfp4_layer, baseline_x
    from moelab_amd.shapes import SHAPES
    from moelab_amd.variants import hip_mxfp4_gptoss as gpt
    from moelab_amd import router
    sh = SHAPES["gpt-oss-20b"]
    s = baseline_mxfp4_layer(sh, seed=2000, device=DEV)
    T = 512
    x = baseline_x(T, sh.d, seed=T, device=DEV)
    idx, wts = router.route(x, s["wr"], sh.k)
    print("case mxscale gpt-oss-20b T=512", flush=True)
    y = gpt.run(s, x, idx, wts, out_dtype=torch.float32)
    rows = np.sort(np.random.default_rng(0).choice(T, size=64, replace=False))
    sel = torch.as_tensor(rows, device=DEV)
    ref = oracle_y(s, x[sel], idx[sel], wts[sel], act=2)
    e = assert_close(y[sel], ref, what="gpt-oss-20b T=512")
    assert e["max_abs"] <= 2e-3 * e["rms_ref"], e


WAVE_CASES = [
    # (name, d, F, E, k, T, routing, act, biases): at most 32 tokens per expert, the wave tiles
    ("w-uniform", 512, 512, 32, 4, 24, "uniform", 0, False),    # 16-token passes, in-kernel grouping
    ("w-zipf-gptoss", 704, 704, 16, 4, 64, "zipf", 2, True),    # K = 64 mod 128, hot experts over several passes
    ("w-32tok", 384, 448, 8, 2, 100, "uniform", 1, False),      # 25 per expert: 32-token passes
    ("w-grouping-launch", 256, 384, 64, 4, 300, "uniform", 0, False),   # 1200 slots: the grouping launch
]


@pytest.mark.parametrize("case", WAVE_CASES, ids=lambda c: c[0])
def test_mxscale_wave_tiles(case, monkeypatch):
    name, d, f, E, k, T, routing, act, biases = case
    sh, s = state(name, d, f, E, k, seed=400 + T, biases=biases)
    x, idx, wts = inputs(sh, T, routing, seed=T, scale=3.0 if act == 2 else 1.0)
    print(f"case mxscale wave {name} T={T}", flush=True)
    y1, y0 = both(monkeypatch, s, x, idx, wts, act=act, dense=None)
    ref = oracle_y(s, x, idx, wts, act=act)
    e1 = assert_close(y1, ref, what=("block-scaled wave", name))
    assert_close(y0, ref, what=("bf16 wave", name))
    assert e1["max_abs"] <= 2e-3 * e1["rms_ref"], (name, e1)
    assert not torch.equal(y1, y0), "MOE_MXMFMA made no difference: the block-scaled wave tiles did not run"


def test_mxscale_wave_stages_split_and_ingroup(monkeypatch):
    """Wave tiles: the stages as two calls, and the grouping launch (MOE_INGROUP=0) against the in-kernel
    grouping, all bit for bit."""
    from moelab_amd import _lib
    from moelab_amd.experts import run_experts
    sh, s = state("ws", 512, 384, 16, 4, seed=13)
    x, idx, wts = inputs(sh, 40, "zipf", seed=13)
    g = _lib.PATH_GROUPED
    y = run_experts(s, x, idx, wts, path=g, out_dtype=torch.float32)
    run_experts(s, x, idx, wts, path=g, out_dtype=torch.float32, stages=_lib.STAGE_GATE_UP)
    y2 = run_experts(s, x, idx, wts, path=g, out_dtype=torch.float32, stages=_lib.STAGE_DOWN)
    monkeypatch.setenv("MOE_INGROUP", "0")
    y3 = run_experts(s, x, idx, wts, path=g, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    assert torch.equal(y, y3)
