"""The A/B harness, slope timing and contention guard on the GPU (moe-lab_amd/compare.py, slope.py, guard.py):
one small run of each, checking that they measure and report, not any particular speed."""
import json

import pytest

import __graft_entry__

__graft_entry__.load_package()
from moelab_amd import backend as be, compare, guard, slope  # noqa: E402
from moelab_amd.shapes import MoEShape  # noqa: E402

pytestmark = pytest.mark.gpu


def test_guard_probe_reads_hbm():
    gbs = guard.probe()
    print(f"probe {gbs:.0f} GB/s", flush=True)
    assert 300.0 < gbs < 8000.0


def test_slope_of_a_chain():
    sh = MoEShape("slope", 256, 384, 8, 2)
    mod = be.load_variant(__graft_entry__.PKG_DIR + "/variants/hip_q4_moe.py")
    st = mod.prepare(*be.make_weights(sh, "bfloat16"))
    inp = [be.make_inputs(sh, 1, "bfloat16", "uniform", seed=s) for s in range(16)]
    per, fixed = slope.fit(lambda *z: mod.run(st, *z), inp, chains=(4, 8, 16))
    print(f"per-call {per:.2f} us, fixed {fixed:.1f} us", flush=True)
    assert 0.5 < per < 500.0


def test_compare_two_launches(tmp_path, monkeypatch):
    monkeypatch.setenv("MOELAB_AMD_PROBE_HISTORY", str(tmp_path / "hist.json"))
    out = tmp_path / "cmp.json"
    summary = compare.main(["hip_q4_moe", "hip_q4_moe", "--dims", "256,384,8,2", "--tokens", "1", "4",
                            "--launches", "2", "--rounds", "2", "--windows", "2", "--out", str(out)])
    assert [s["T"] for s in summary] == [1, 4]
    for s in summary:
        assert s["n"] == 4 and 0.5 < s["speedup_B_over_A"] < 2.0
        assert 0.0 < s["ci95"][0] <= s["ci95"][1]
        assert s["errA"] < 1e-2 and s["errB"] < 1e-2
    rec = json.load(open(out))
    assert len(rec["probes"]) == 4 and rec["guard"]["status"] == "calibrating"
