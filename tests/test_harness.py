"""A/B harness, slope fit and contention guard (host logic, CPU): moe-lab_amd/compare.py, slope.py, guard.py
against closed forms and an exhaustive enumeration of the two-stage bootstrap on a tiny case."""
import itertools
import json

import numpy as np
import pytest

import __graft_entry__

__graft_entry__.load_package()
from moelab_amd import compare, guard, slope  # noqa: E402


def rows_of(per_launch):
    return [{"launch": L, "A_us": a, "B_us": b} for L, rs in enumerate(per_launch) for a, b in rs]


def test_boot_ci_closed_forms():
    a = np.linspace(90.0, 110.0, 12)
    assert compare.boot_ci(a, a) == (1.0, 1.0, 1.0)
    sp, lo, hi = compare.boot_ci(a, a / 2)
    assert sp == 2.0 and abs(lo - 2.0) < 1e-12 and abs(hi - 2.0) < 1e-12


def test_boot_ci_interval_covers_and_is_seeded():
    rng = np.random.default_rng(1)
    a, b = rng.normal(100, 5, 40), rng.normal(50, 2.5, 40)
    sp, lo, hi = compare.boot_ci(a, b, seed=3)
    assert lo < sp < hi and hi - lo < 0.2
    assert compare.boot_ci(a, b, seed=3) == (sp, lo, hi)


def test_hier_bootstrap_matches_enumeration():
    """2 launches x 2 rounds: every replicate is one of finitely many equally likely draws (launch picks, then
    round picks inside each pick); the sampled frequencies match the enumerated probabilities."""
    per = [[(10.0, 5.0), (12.0, 5.0)], [(30.0, 10.0), (20.0, 10.0)]]
    rows = rows_of(per)
    exact = {}
    for picks in itertools.product(range(2), repeat=2):
        for r0 in itertools.product(range(2), repeat=2):
            for r1 in itertools.product(range(2), repeat=2):
                samp = [per[picks[0]][i] for i in r0] + [per[picks[1]][i] for i in r1]
                a, b = zip(*samp)
                v = round(float(np.median(a) / np.median(b)), 9)
                exact[v] = exact.get(v, 0.0) + 1.0 / 64
    got = compare.hier_samples(rows, n=40000, seed=5)
    vals, counts = np.unique(np.round(got, 9), return_counts=True)
    freq = dict(zip(vals.tolist(), (counts / got.size).tolist()))
    assert set(freq) <= set(exact)
    for v, p in exact.items():
        assert abs(freq.get(v, 0.0) - p) < 0.01, (v, p, freq.get(v))


def test_hier_interval_wider_than_rounds_when_launches_differ():
    rng = np.random.default_rng(2)
    per = [[(100.0 * f + rng.normal(0, 0.1), 50.0) for _ in range(6)] for f in (0.9, 1.0, 1.1, 0.95, 1.05)]
    rows = rows_of(per)
    lo, hi = compare.boot_ci_hier(rows)
    _, rlo, rhi = compare.boot_ci([r["A_us"] for r in rows], [r["B_us"] for r in rows])
    assert hi - lo > 1.5 * (rhi - rlo)


def test_summarize_fields():
    rows = [dict(r, T=1, errA=1e-3, errB=2e-3) for r in rows_of([[(10.0, 5.0), (11.0, 5.0)], [(9.0, 4.5)]])]
    (s,) = compare.summarize(rows, [1])
    assert s["n"] == 3 and s["per_launch"] == [2.1, 2.0] and s["speedup_B_over_A"] == 2.0


def test_slope_fit_recovers_line():
    chains = (10, 20, 40, 80)
    s, c = slope.fit_line(chains, [3e-6 + 2.5e-6 * ch for ch in chains])
    assert abs(s - 2.5e-6) < 1e-15 and abs(c - 3e-6) < 1e-15
    per, fixed = slope.fit(None, None, chains, timer=lambda fn, inp, ch: 7e-6 + 1.25e-6 * ch)
    assert abs(per - 1.25) < 1e-9 and abs(fixed - 7.0) < 1e-9


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
