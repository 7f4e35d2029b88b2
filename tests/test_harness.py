"""A/B harness, slope fit, contention guard and random-shape sweep (host logic, CPU): moe-lab_amd/compare.py,
slope.py, guard.py, sweep.py against closed forms, an exhaustive enumeration of both bootstrap draws on a tiny case,
and the sweep's case generator against the library's shape requirements."""
import itertools
import json

import numpy as np
import pytest

import __graft_entry__

__graft_entry__.load_package()
from moelab_amd import compare, guard, slope, sweep  # noqa: E402


def rows_of(per_launch, tokens=1):
    """Long-format rows from per-launch lists of (A us, B us) rounds."""
    out = []
    for L, rs in enumerate(per_launch):
        for rd, (ua, ub) in enumerate(rs):
            out += [{"launch": L, "tokens": tokens, "round": rd, "arm": "A", "us_per_call": ua},
                    {"launch": L, "tokens": tokens, "round": rd, "arm": "B", "us_per_call": ub}]
    return out


def test_interval_closed_forms():
    a = np.linspace(90.0, 110.0, 12).reshape(3, 4)
    assert compare.Interval.of(a, a) == compare.Interval(1.0, 1.0, 1.0)
    iv = compare.Interval.of(a, a / 2, by_launch=False)
    assert iv.ratio == 2.0 and abs(iv.lo - 2.0) < 1e-12 and abs(iv.hi - 2.0) < 1e-12


def test_interval_covers_and_is_seeded():
    rng = np.random.default_rng(1)
    a, b = rng.normal(100, 5, (5, 8)), rng.normal(50, 2.5, (5, 8))
    iv = compare.Interval.of(a, b, seed=3)
    assert iv.lo < iv.ratio < iv.hi and iv.hi - iv.lo < 0.2
    assert compare.Interval.of(a, b, seed=3) == iv


def _enumerate(per, by_launch):
    """Exact distribution of the replicate ratio for a tiny [launch, round] case: every launch pick (or the launches
    as they are) times every round pick inside each, all equally likely."""
    L, R = len(per), len(per[0])
    picks = itertools.product(range(L), repeat=L) if by_launch else [tuple(range(L))]
    picks = list(picks)
    exact = {}
    for pk in picks:
        for rounds in itertools.product(itertools.product(range(R), repeat=R), repeat=L):
            samp = [per[pk[i]][j] for i in range(L) for j in rounds[i]]
            a, b = zip(*samp)
            v = round(float(np.median(a) / np.median(b)), 9)
            exact[v] = exact.get(v, 0.0) + 1.0 / (len(picks) * R ** (R * L))
    return exact


@pytest.mark.parametrize("by_launch", [True, False])
def test_resample_matches_enumeration(by_launch):
    """2 launches x 2 rounds: the sampled replicate frequencies match the enumerated probabilities of the two-stage
    draw (launches, then rounds inside each drawn launch) and of the rounds-only draw (launches fixed)."""
    per = [[(10.0, 5.0), (12.0, 5.0)], [(30.0, 10.0), (20.0, 10.0)]]
    a, b = compare.paired_arrays(rows_of(per), 1)
    exact = _enumerate(per, by_launch)
    got = compare.resample(a, b, 40000, seed=5, by_launch=by_launch)
    vals, counts = np.unique(np.round(got, 9), return_counts=True)
    freq = dict(zip(vals.tolist(), (counts / got.size).tolist()))
    assert set(freq) <= set(exact)
    for v, p in exact.items():
        assert abs(freq.get(v, 0.0) - p) < 0.01, (v, p, freq.get(v))


def test_launch_interval_wider_than_rounds_when_launches_differ():
    rng = np.random.default_rng(2)
    per = [[(100.0 * f + rng.normal(0, 0.1), 50.0) for _ in range(6)] for f in (0.9, 1.0, 1.1, 0.95, 1.05)]
    (s,) = [compare.summary_of(rows_of(per), 1)]
    wide = s["interval95"][1] - s["interval95"][0]
    narrow = s["interval95_rounds"][1] - s["interval95_rounds"][0]
    assert wide > 1.5 * narrow


def test_summary_fields_and_missing_rounds():
    rows = rows_of([[(10.0, 5.0), (11.0, 5.0)], [(9.0, 4.5), (9.0, 4.5)]])
    checks = [{1: {"A": 1e-3, "B": 2e-3}}, {1: {"A": 3e-3, "B": 1e-3}}]
    s = compare.summary_of(rows, 1, checks)
    assert s["replays"] == 4 and s["launch_ratios"] == [2.1, 2.0] and s["ratio"] == 9.5 / 4.75
    assert s["max_over_rms"] == {"A": 3e-3, "B": 2e-3}
    with pytest.raises(ValueError):
        compare.paired_arrays(rows[:-1], 1)


def test_slope_estimators():
    xs = (8, 16, 32, 64)
    s, c = slope.theil_sen(xs, [3e-6 + 2.5e-6 * n for n in xs])
    assert abs(s - 2.5e-6) < 1e-15 and abs(c - 3e-6) < 1e-15
    ys = [3e-6 + 2.5e-6 * n for n in xs]
    ys[1] += 40e-6   # one disturbed length
    s2, _ = slope.theil_sen(xs, ys)
    l2, _ = slope.least_squares(xs, ys)
    assert abs(s2 - 2.5e-6) < 0.5e-6 and abs(l2 - 2.5e-6) > abs(s2 - 2.5e-6)
    line = slope.measure(None, None, xs, timer=lambda fn, w, n: 7e-6 + 1.25e-6 * n)
    assert abs(line.per_call_us - 1.25) < 1e-9 and abs(line.fixed_us - 7.0) < 1e-9
    assert abs(line.lsq_per_call_us - 1.25) < 1e-9 and sorted(line.points) == list(xs)
    with pytest.raises(ValueError):
        slope.theil_sen([4, 4], [1.0, 2.0])


def test_guard_verdict_history(tmp_path):
    path = str(tmp_path / "hist.json")
    k = "test-device"
    v = guard.verdict([5000.0, 5100.0], path=path, device_key=k)
    assert v["status"] == "calibrating" and v["history"] == 0
    for _ in range(2):
        guard.verdict([5000.0, 5050.0], path=path, device_key=k)
    assert json.load(open(path))[k][-1] == 5050.0
    ok = guard.verdict([4900.0], path=path, device_key=k, update=False)
    assert ok["status"] == "ok" and ok["history"] == 6
    bad = guard.verdict([4000.0], path=path, device_key=k, update=False)
    assert bad["status"] == "contended" and bad["contended"]
    assert guard.report(bad).startswith("[guard contended]") and "rerun" in guard.report(bad)
    for _ in range(30):
        guard.verdict([5000.0, 5000.0], path=path, device_key=k)
    assert len(json.load(open(path))[k]) == guard.N_HISTORY


def test_grid_crossover_and_fitted_policy():
    """The crossover reading of grid.py, and the MI355X load policy against the grid's boundary rows."""
    from moelab_amd import fallback, grid
    from moelab_amd.variants import hip_mxfp4_moe, hip_q4_moe
    rows = [{"load": L, "slots_over_grouped": r} for L, r in ((0.1, 0.8), (1, 1.2), (4, 0.9), (8, 1.5), (16, 2.0))]
    assert grid.crossover(rows) == 8 and grid.crossover(rows[:3]) is None
    assert [grid.t_for_load(L, 128, 8) for L in (0.0625, 1, 32)] == [2, 16, 512]
    # (shape D, F, E, k; T where the per-slot path won; T where grouped won)
    for D, F, E, k, t_slots, t_grouped in ((2048, 768, 128, 8, 8, 16), (2048, 1024, 64, 8, 4, 8),
                                           (2048, 1408, 64, 6, 2, 3), (2880, 2880, 32, 4, 2, 4)):
        assert not hip_q4_moe.custom_wins(t_slots, k, E, D, F) and hip_q4_moe.custom_wins(t_grouped, k, E, D, F)
        assert not hip_mxfp4_moe.grouped(t_slots, k, E, D, F) and hip_mxfp4_moe.grouped(t_grouped, k, E, D, F)
    assert hip_q4_moe.custom_wins(2, 2, 8, 4096, 14336) and hip_q4_moe.custom_wins(512, 2, 8, 4096, 14336)
    assert fallback.grouped_from_load(2048, 768) == 1.0 and fallback.grouped_from_load(4096, 14336) == 0.27
    # near the threshold the grouped path also needs live gate/up wave tiles: the random-shape sweep's per-slot wins
    # go per-slot, its grouped wins near the threshold stay grouped, and high loads are grouped whatever the count
    assert abs(fallback.grouped_waves(16, 8, 128, 768) - 128 * (1 - (127 / 128) ** 128) * 24) < 1e-9
    assert fallback.grouped_waves(128, 4, 16, 3264) == 32 * 102   # passes = T k / 16 when above U
    assert not hip_q4_moe.custom_wins(8, 2, 16, 3328, 384) and not hip_mxfp4_moe.grouped(16, 2, 32, 896, 320)
    assert hip_mxfp4_moe.grouped(3, 8, 32, 5120, 832) and hip_q4_moe.custom_wins(16, 1, 32, 3840, 1664)
    assert hip_q4_moe.custom_wins(32, 2, 16, 3328, 384)   # load 4: no wave condition


def test_reference_skips_ids_outside_range():
    """backend.reference follows the library's contract: a slot whose id is outside [0, E) adds nothing (the same
    result as that slot pointing at expert 0 with weight 0)."""
    import torch
    from moelab_amd import backend as be
    g = torch.Generator().manual_seed(3)
    E, d, F = 4, 8, 16
    wg, wu = torch.randn(E, F, d, generator=g), torch.randn(E, F, d, generator=g)
    wd = torch.randn(E, d, F, generator=g)
    x = torch.randn(3, d, generator=g)
    idx = torch.tensor([[0, -1], [5, 2], [1, 1]], dtype=torch.int32)
    wts = torch.rand(3, 2, generator=g)
    keep = (idx >= 0) & (idx < E)
    y = be.reference(wg, wu, wd, x, idx, wts)
    y2 = be.reference(wg, wu, wd, x, torch.where(keep, idx, torch.zeros_like(idx)), wts * keep)
    assert torch.allclose(y, y2, atol=1e-6) and y.abs().sum() > 0


def test_sweep_cases_meet_the_library_requirements():
    """Every drawn case is a shape the library takes (d, F multiples of 64, F <= 16384, 1 <= k <= E <= 1024) under
    the weight cap; the generator is a function of its seed; 400 draws reach both formats, both dtypes, every
    routing, T = 1 and T >= 64."""
    cases = sweep.draw_cases(400, seed=11, max_dense_bytes=1.5e9)
    assert cases == sweep.draw_cases(400, seed=11, max_dense_bytes=1.5e9)
    assert cases != sweep.draw_cases(400, seed=12, max_dense_bytes=1.5e9)
    for c in cases:
        assert c.d % 64 == 0 and c.F % 64 == 0 and 256 <= c.F <= 16384 and 512 <= c.d <= 5120
        assert 1 <= c.k <= c.E <= 1024 and c.E & (c.E - 1) == 0
        assert c.dense_bytes() <= 1.5e9 and 1 <= c.T <= 128
    assert {c.fmt for c in cases} == {"int4", "mxfp4"} and {c.dtype for c in cases} == {"bfloat16", "float16"}
    assert {c.routing for c in cases} == {"uniform", "zipf", "one_hot"}
    assert min(c.T for c in cases) == 1 and max(c.T for c in cases) >= 64
    assert all(c.fmt == "int4" for c in sweep.draw_cases(50, seed=3, fmts=("int4",)))


def test_sweep_summary_flags():
    rows = [{"case": "a", "T": 1, "ok": True, "slots_over_default": 1.4, "max_over_rms": 1e-4},
            {"case": "b", "T": 8, "ok": True, "slots_over_default": 0.8, "max_over_rms": 2e-4},
            {"case": "c", "T": 32, "ok": False, "slots_over_default": 3.0, "max_over_rms": 5e-2}]
    s = sweep.summary(rows, flag=0.95)
    assert s["cases"] == 3 and not s["all_correct"] and s["worst_max_over_rms"] == 5e-2
    assert s["flagged"] == ["b T=8", "c T=32"]
    assert s["slots_over_default_min"] == 0.8 and s["slots_over_default_median"] == 1.4
