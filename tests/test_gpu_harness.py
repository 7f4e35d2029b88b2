"""The A/B harness, slope timing, contention guard and random-shape sweep on the GPU (moe-lab_amd/compare.py,
slope.py, guard.py, sweep.py): one small run of each, checking that they measure and report, not any particular
speed (the sweep's correctness gates do hold)."""
import json

import pytest

import __graft_entry__

__graft_entry__.load_package()
from moelab_amd import backend as be, compare, guard, slope, sweep  # noqa: E402
from moelab_amd.shapes import MoEShape  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [16, 3 * (1 << 20) + 48, 1 << 24])
def test_probe_read_folds_every_word(nbytes):
    """moe_probe_read reads every 16-byte chunk once: the XOR of its sink equals the XOR of the buffer's words
    (a length that is not a multiple of a workgroup's 16 KB block included)."""
    import numpy as np
    import torch
    from moelab_amd import _lib
    g = torch.Generator(device="cuda").manual_seed(nbytes)
    buf = torch.randint(-2 ** 31, 2 ** 31 - 1, (nbytes // 4,), dtype=torch.int32, device="cuda", generator=g)
    sink = torch.full((_lib.PROBE_SINK,), 7, dtype=torch.int32, device="cuda")
    _lib.check("moe_probe_read", _lib.lib().moe_probe_read(_lib.ptr(buf), nbytes, _lib.ptr(sink),
                                                           _lib.stream_of(buf.device)))
    want = np.bitwise_xor.reduce(buf.cpu().numpy().view(np.uint32))
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    assert got == want
    assert _lib.lib().moe_probe_read(_lib.ptr(buf), 24, _lib.ptr(sink), None) == _lib.MOE_ERR_ARG


def test_guard_probe_reads_hbm():
    gbs = guard.probe()
    print(f"probe {gbs:.0f} GB/s", flush=True)
    assert 300.0 < gbs < 8000.0


def test_slope_of_a_chain():
    sh = MoEShape("slope", 256, 384, 8, 2)
    carry, (res,) = slope.run(sh, ["hip_q4_moe"], tokens=1, lengths=(4, 8, 16), windows=16)
    print(f"carry {carry.per_call_us:.2f} us, per-call {res.per_call_us:.2f} us, own {res.own_us:.2f} us", flush=True)
    # the carry's slope (the chain's add alone, ~1-3 us per call) is a fit over three chain lengths: on a call this
    # small its noise can exceed it, so only the report's consistency is asserted, not its sign
    assert 0.5 < res.per_call_us < 500.0 and res.floor_us > 0
    assert abs(res.own_us - (res.per_call_us - carry.per_call_us)) < 1e-9 and abs(carry.per_call_us) < 50.0


@pytest.mark.parametrize("in_process", [True, False])
def test_compare_two_launches(tmp_path, monkeypatch, in_process):
    """Two launches of the same variant as both arms: in this process, and as spawned launch processes."""
    monkeypatch.setenv("MOELAB_AMD_PROBE_HISTORY", str(tmp_path / "hist.json"))
    out = tmp_path / "cmp.json"
    args = ["hip_q4_moe", "hip_q4_moe", "--dims", "256,384,8,2", "--tokens", "1", "4", "--launches", "2",
            "--rounds", "2", "--windows", "2", "--json", str(out)] + (["--in-process"] if in_process else [])
    summaries = compare.main(args)
    assert [s["tokens"] for s in summaries] == [1, 4]
    for s in summaries:
        assert s["replays"] == 4 and 0.5 < s["ratio"] < 2.0
        assert 0.0 < s["interval95"][0] <= s["interval95"][1]
        assert s["max_over_rms"]["A"] < 1e-2 and s["max_over_rms"]["B"] < 1e-2
    rec = json.load(open(out))
    assert len(rec["probes"]) == 4 and rec["guard"]["status"] == "calibrating"
    assert {r["arm"] for r in rec["rows"]} == {"A", "B"} and len(rec["rows"]) == 2 * 2 * 2 * 2


def test_sweep_small_run():
    """Three small random cases (both formats): every default call passes its correctness gates and both arms time."""
    rows, summ, g = sweep.run(3, seed=10, max_dense_bytes=3e8, probe=False, emit=lambda m: print(m, flush=True))
    assert g is None and summ["cases"] == 3 and summ["all_correct"], rows
    for r in rows:
        assert r["ok"] and r["slots_us"] > 0 and r["default_us"] > 0 and r["max_over_rms"] <= 1e-2
