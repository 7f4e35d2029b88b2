"""moe_experts_run_static, the entry point that allocates nothing (its workspace is a device array inside the
library), against moe_experts_run with a caller workspace, through the C ABI.

Both run the same kernels on the same inputs, so the outputs must be equal bit for bit. Each case makes two
calls in a row on the static array, the second with fewer tokens than the first (the array keeps the first
call's contents, which the second must not depend on), on the per-slot GEMV, the grouped wave tiles, the dense
fp16 tiles and the T=1 default path. Sizes beyond the array are refused with MOE_ERR_WORKSPACE before any launch.
"""
import numpy as np
import pytest
import torch

from helpers import assert_close, oracle_y

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _inputs(sh, T, seed):
    from moelab_amd.problem import make_routing
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.standard_normal((T, sh.d)).astype(np.float32)).to(DEV, torch.bfloat16)
    idx, wts = make_routing(T, sh.E, sh.k, "uniform", rng)
    return x, torch.from_numpy(idx).to(DEV), torch.from_numpy(wts).to(DEV)


def run_static(s, x, idx, wts, path, out_dtype=torch.float32):
    """One moe_experts_run_static call through ctypes (no workspace argument)."""
    from moelab_amd import _lib
    from moelab_amd.experts import _desc
    T, k = idx.shape
    y = torch.full((T, x.shape[1]), float("nan"), dtype=out_dtype, device=DEV)
    rc = _lib.lib().moe_experts_run_static(_desc(s), _lib.ptr(x), _lib.DTYPE[x.dtype], _lib.ptr(idx), _lib.ptr(wts),
                                           T, k, 0, int(path), 0, _lib.ptr(y), _lib.DTYPE[out_dtype], None,
                                           _lib.stream_of(x.device))
    return rc, y


CASES = [
    # (name, path, d, F, E, k, first T, second T, MOE_DENSE)
    ("per-slot", 1, 512, 384, 16, 4, 12, 3, None),
    ("grouped-wave", 2, 512, 384, 16, 4, 40, 9, None),
    ("grouped-dense", 2, 256, 384, 4, 2, 200, 70, "1"),
    ("auto-T1", 0, 512, 384, 16, 4, 2, 1, None),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: c[0])
def test_static_entry_point_matches_the_workspace_entry_point(case, monkeypatch):
    from moelab_amd import _lib
    from moelab_amd.experts import run_experts
    from moelab_amd.problem import baseline_int4_layer
    from moelab_amd.shapes import MoEShape
    name, path, d, F, E, k, T1, T2, dense = case
    if dense is not None:
        monkeypatch.setenv("MOE_DENSE", dense)
    sh = MoEShape(name, d=d, f=F, E=E, k=k)
    s = baseline_int4_layer(sh, seed=7, device=DEV, router=False)
    assert _lib.lib().moe_experts_run_static(None, None, 0, None, None, 0, k, 0, path, 0, None, 0, None,
                                             None) == _lib.MOE_OK   # T = 0: the set-up call only
    for call, T in enumerate((T1, T2)):
        x, idx, wts = _inputs(sh, T, seed=100 * call + T)
        print(f"case static {name} call {call} T={T}", flush=True)
        rc, y = run_static(s, x, idx, wts, path)
        _lib.check("moe_experts_run_static", rc)
        y_ref = run_experts(s, x, idx, wts, path=path, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref), (name, call, float((y - y_ref).abs().max()))
        assert_close(y, oracle_y(s, x, idx, wts), what=(name, call))
        rc, yb = run_static(s, x, idx, wts, path, out_dtype=torch.bfloat16)
        _lib.check("moe_experts_run_static", rc)
        assert torch.equal(yb, run_experts(s, x, idx, wts, path=path)), (name, call, "bf16")


def test_static_entry_point_refuses_sizes_beyond_its_array():
    from moelab_amd import _lib
    from moelab_amd.experts import _desc
    from moelab_amd.problem import baseline_int4_layer
    from moelab_amd.shapes import SHAPES
    sh = SHAPES["qwen3-30b-a3b"]
    s = baseline_int4_layer(sh, seed=8, device=DEV, router=False)
    L = _lib.lib()
    fits = [T for T in (1, 32, 110, 111, 256) if L.moe_experts_workspace_bytes(_desc(s), T, sh.k, 2) <=
            _lib.STATIC_SCRATCH_BYTES]
    assert fits == [1, 32, 110]
    x, idx, wts = _inputs(sh, 111, seed=1)
    rc, y = run_static(s, x, idx, wts, 2)
    torch.cuda.synchronize()
    assert rc == _lib.MOE_ERR_WORKSPACE
    assert torch.isnan(y).all()   # refused before any launch: the output is untouched
    x, idx, wts = _inputs(sh, 110, seed=2)   # the largest call that fits, at the full Qwen3 shape
    rc, y = run_static(s, x, idx, wts, 2)
    _lib.check("moe_experts_run_static", rc)
    from moelab_amd.experts import run_experts
    y_ref = run_experts(s, x, idx, wts, path=2, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)
