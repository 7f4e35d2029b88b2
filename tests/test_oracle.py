"""Pins the CPU oracle: every oracle function is checked against something it does not restate
(known answers from the reference's tests, closed forms, exact integer arithmetic, independent
formulations), chosen so that a dropped term, a wrong index or a transposed operand fails."""
import math

import numpy as np
import pytest
import torch


# ------------------------------------------------------------------------------------------ bf16
def test_bf16_rounding_matches_torch(orc):
    rng = np.random.default_rng(0)
    a = np.concatenate([rng.standard_normal(4096).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 4096),
                        np.array([0.0, -0.0, np.inf, -np.inf, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8,
                                  3.3895314e38, 1e-40], dtype=np.float32)]).astype(np.float32)
    ours = orc.f32_to_bf16_bits(a)
    ref = torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, ref)
    assert np.isnan(orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(np.array([np.nan], np.float32))))[0]


# --------------------------------------------------------------------------------------- formats
def test_unpack_int4_low_nibble_first(orc):
    # word 0x76543210 holds codes 0..7 in element order (reference metal_q4_decode_v4.py:57-64)
    w = np.array([[0x76543210, 0xFEDCBA98]], dtype=np.uint32)
    np.testing.assert_array_equal(orc.unpack_int4(w)[0], np.arange(16))


def test_dequant_int4_known_answer(orc):
    # one group of 64: codes 0..15 repeated, scale 0.5, bias -4  ->  w = 0.5 q - 4
    q = np.tile(np.arange(16), 4)
    words = np.zeros((1, 8), dtype=np.uint32)
    for i, c in enumerate(q):
        words[0, i // 8] |= np.uint32(int(c) << (4 * (i % 8)))
    s = orc.f32_to_bf16_bits(np.array([[0.5]], np.float32))
    b = orc.f32_to_bf16_bits(np.array([[-4.0]], np.float32))
    np.testing.assert_array_equal(orc.dequant_int4(words, s, b)[0], 0.5 * q - 4.0)


def test_pack_roundtrip_against_product_packer(orc):
    from moelab_amd import formats
    rng = np.random.default_rng(1)
    q = rng.integers(0, 16, (3, 5, 128))
    words = formats.pack_nibbles(torch.from_numpy(q)).numpy().view(np.uint32)
    np.testing.assert_array_equal(orc.unpack_int4(words), q)


def test_e2m1_table_is_ocp_definition(orc):
    # E2M1: sign bit 3, exponent bits 2..1 (bias 1), mantissa bit 0; exponent 0 is subnormal (m * 0.5)
    for code in range(16):
        s, e, m = code >> 3, (code >> 1) & 3, code & 1
        v = (m * 0.5) if e == 0 else 2.0 ** (e - 1) * (1 + m / 2)
        assert orc.E2M1[code] == (-v if s else v)
        assert math.copysign(1, orc.E2M1[code]) == (-1 if s else 1)


def test_e8m0_scale_powers_of_two(orc):
    s = np.arange(256)
    v = orc.e8m0_scale(s)
    for b in range(1, 255):
        assert v[b] == math.ldexp(1.0, b - 127)
    assert v[0] == 0.0 and np.isinf(v[255])


def test_dequant_mxfp4_known_answer(orc):
    codes = np.arange(16).tolist() * 2           # 32 elements: the whole E2M1 table twice
    words = np.zeros((1, 4), dtype=np.uint32)
    for i, c in enumerate(codes):
        words[0, i // 8] |= np.uint32(c << (4 * (i % 8)))
    sb = np.array([[127 + 3]], dtype=np.uint8)   # scale 8
    np.testing.assert_array_equal(orc.dequant_mxfp4(words, sb)[0], 8.0 * orc.E2M1[np.array(codes)])


# ---------------------------------------------------------------------------------------- router

def orc_bits(a):
    return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("d", [8, 64, 512, 520, 2048, 2880])
def test_router_logits_exact_on_integers(orc, d):
    """Small-integer bf16 inputs: every partial sum is exact in fp32, so any correct order gives the
    exact integer dot product. Catches dropped, doubled or misindexed terms."""
    rng = np.random.default_rng(d)
    x = rng.integers(-8, 9, (3, d)).astype(np.float32)
    w = rng.integers(-8, 9, (5, d)).astype(np.float32)
    b = rng.integers(-100, 100, 5).astype(np.float32)
    lg = orc.router_logits(orc_bits(x), orc_bits(w), b)
    np.testing.assert_array_equal(lg, (x.astype(np.int64) @ w.T.astype(np.int64) + b.astype(np.int64)))


def test_router_logits_close_to_fp64(orc):
    rng = np.random.default_rng(3)
    x = orc.round_bf16(rng.standard_normal((4, 2048)).astype(np.float32))
    w = orc.round_bf16((rng.standard_normal((128, 2048)) * 0.02).astype(np.float32))
    lg = orc.router_logits(orc_bits(x), orc_bits(w))
    exact = x.astype(np.float64) @ w.T.astype(np.float64)
    bound = 2048 * 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(w).T.astype(np.float64))
    assert (np.abs(lg - exact) <= bound).all()


def _tree64(part):
    """The documented combination of 64 fp32 lane partials: quads, half-rows, rows, then
    (R3 + R2) + (R1 + R0), each addition rounded to fp32."""
    f = np.float32
    q = [f(f(part[4 * i] + part[4 * i + 1]) + f(part[4 * i + 2] + part[4 * i + 3])) for i in range(16)]
    h = [f(q[2 * i] + q[2 * i + 1]) for i in range(8)]
    r = [f(h[2 * i] + h[2 * i + 1]) for i in range(4)]
    return f(f(r[3] + r[2]) + f(r[1] + r[0]))


def test_router_logits_order_is_the_documented_one(orc):
    """Values whose fp32 sum depends on the order: the oracle must equal the documented order
    (lane chunks, then the quad/half-row/row tree), not a sequential sum and not an xor butterfly."""
    d = 1024
    x = np.zeros((1, d), np.float32)
    w = np.ones((1, d), np.float32)
    x[0, 0] = 2.0 ** 24        # lane 0 (chunk 0)
    x[0, 8] = 1.0              # lane 1 (chunk 1)
    x[0, 16] = -(2.0 ** 24)    # lane 2 (chunk 2)
    lg = orc.router_logits(orc_bits(x), orc_bits(w))
    part = np.zeros(64, np.float32)
    part[0], part[1], part[2] = 2.0 ** 24, 1.0, -(2.0 ** 24)
    tree = _tree64(part)
    # the tree adds 2^24 + 1 first (rounds to 2^24), then -2^24: 0; a butterfly adds 2^24 - 2^24 first: 1
    bfly = part.copy()
    for s in (32, 16, 8, 4, 2, 1):
        bfly = (bfly + bfly[np.arange(64) ^ s]).astype(np.float32)
    assert tree == 0.0 and bfly[0] == 1.0
    assert lg[0, 0] == tree
    # lanes 0, 16, 32, 48 (one per row) hold 1, 1, 2^24, 1: the tree gives (1 + 2^24) + (1 + 1) = 2^24 + 2,
    # a sequential sum ((1 + 1) + 2^24) + 1 = 2^24 + 4 (2^24 + 3 rounds to even)
    x2 = np.zeros((1, d), np.float32)
    x2[0, 8 * 0], x2[0, 8 * 16], x2[0, 8 * 32], x2[0, 8 * 48] = 1.0, 1.0, 2.0 ** 24, 1.0
    part2 = np.zeros(64, np.float32)
    part2[0], part2[16], part2[32], part2[48] = 1.0, 1.0, 2.0 ** 24, 1.0
    seq = np.float32(0.0)
    for v in part2:
        seq = np.float32(seq + v)
    tree2 = _tree64(part2)
    assert tree2 == 2.0 ** 24 + 2 and seq == 2.0 ** 24 + 4
    lg2 = orc.router_logits(orc_bits(x2), orc_bits(w))
    assert lg2[0, 0] == tree2


def test_topk_matches_stable_argsort(orc):
    rng = np.random.default_rng(5)
    for E, k in [(8, 2), (16, 6), (60, 4), (128, 8), (256, 8), (128, 1), (512, 32), (1000, 8)]:
        lg = orc.round_bf16((rng.standard_normal((33, E)) * 3).astype(np.float32))   # bf16 values: many ties
        idx, w = orc.topk(lg, k)
        idx2, w2 = orc.topk_closed_form(lg, k)
        np.testing.assert_array_equal(idx, idx2)
        np.testing.assert_allclose(w, w2, rtol=2e-6, atol=1e-7)
        np.testing.assert_allclose(w.sum(1), 1.0, atol=1e-5)
        # same multiset of values as a plain sort (reference test_router.py:28-31)
        np.testing.assert_array_equal(np.sort(np.take_along_axis(lg, idx, 1), 1),
                                      np.sort(lg, 1)[:, ::-1][:, :k][:, ::-1])


def test_topk_all_tied_known_answer(orc):
    # reference test_router.py:36-41: all equal -> k distinct ids, weights 1/k; lowest ids win
    idx, w = orc.topk(np.zeros((3, 64), np.float32), 6)
    np.testing.assert_array_equal(idx, np.tile(np.arange(6), (3, 1)))
    np.testing.assert_allclose(w, 1 / 6, atol=1e-7)


@pytest.mark.parametrize("bad", [np.nan, -np.inf])
def test_topk_nonfinite_known_answer(orc, bad):
    # reference test_router.py:73-86
    lg = np.random.default_rng(0).standard_normal((4, 64)).astype(np.float32)
    lg[0, :] = bad
    lg[1, 3:] = bad
    idx, w = orc.topk(lg, 6)
    assert ((idx >= 0) & (idx < 64)).all()
    for t in range(4):
        assert len(set(idx[t].tolist())) == 6
    assert set(idx[1, :3].tolist()) == {0, 1, 2}
    np.testing.assert_array_equal(idx[1, 3:], [3, 4, 5])
    np.testing.assert_allclose(w[1].sum(), 1.0, atol=1e-6)
    assert (w[1, 3:] == 0).all()
    np.testing.assert_array_equal(idx[0], np.arange(6))


def test_topk_full_softmax(orc):
    # reference test_router.py:44-55: norm=False gives the full-softmax probabilities
    rng = np.random.default_rng(2)
    lg = (rng.standard_normal((33, 64)) * 2).astype(np.float32)
    idx, w = orc.topk(lg, 6, norm=False)
    P = np.exp(lg.astype(np.float64) - lg.max(1, keepdims=True))
    P /= P.sum(1, keepdims=True)
    for t in range(33):
        np.testing.assert_array_equal(np.sort(idx[t]), np.sort(np.argsort(-P[t], kind="stable")[:6]))
        np.testing.assert_allclose(w[t], P[t, idx[t]], rtol=1e-5)


def test_topk_brute_force_tiny(orc):
    """Exhaustive over all 3^5 logit patterns on E=5 (values from {0, 1, 2}: ties everywhere)."""
    import itertools
    rows = np.array(list(itertools.product([0.0, 1.0, 2.0], repeat=5)), np.float32)
    idx, _ = orc.topk(rows, 3)
    for r, ids in zip(rows, idx):
        # brute force: choose the 3-subset with the largest sum, ties broken by lexicographically smallest
        # (value-descending, id-ascending) order
        order = sorted(range(5), key=lambda e: (-r[e], e))
        assert list(ids) == order[:3]


# -------------------------------------------------------------------------------------- grouping
def test_group_brute_force(orc):
    rng = np.random.default_rng(7)
    for T, k, E in [(1, 8, 128), (32, 8, 128), (17, 4, 16), (64, 2, 8), (5, 1, 1)]:
        idx = rng.integers(0, E, (T, k))
        counts, offsets, order, active = orc.group(idx, E)
        flat = idx.reshape(-1)
        for p, e in enumerate(flat):
            rank = int((flat[:p] == e).sum())
            assert order[offsets[e] + rank] == p
        np.testing.assert_array_equal(counts, [int((flat == e).sum()) for e in range(E)])
        np.testing.assert_array_equal(active, [e for e in range(E) if (flat == e).any()])


# ------------------------------------------------------------------------------- expert compute
def _problem(rng, T, d, F, E, k):
    x = rng.standard_normal((T, d))
    wg = rng.standard_normal((E, F, d)) / np.sqrt(d)
    wu = rng.standard_normal((E, F, d)) / np.sqrt(d)
    wd = rng.standard_normal((E, d, F)) / np.sqrt(F)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    wts = rng.random((T, k)).astype(np.float32)
    return x, wg, wu, wd, idx, wts


@pytest.mark.parametrize("act", [0, 1, 2])
def test_moe_reference_two_formulations(orc, act):
    rng = np.random.default_rng(act)
    x, wg, wu, wd, idx, wts = _problem(rng, 9, 64, 48, 6, 3)
    y1 = orc.moe_reference(x, wg, wu, wd, idx, wts, act)
    y2 = orc.moe_reference_per_token(x, wg, wu, wd, idx, wts, act)
    np.testing.assert_allclose(y1, y2, rtol=1e-12, atol=1e-12)


def _sigmoid_tanh(z):
    """The logistic function through the identity sigma(z) = (1 + tanh(z / 2)) / 2 (not the exp form the
    oracle uses)."""
    return 0.5 * (1.0 + np.tanh(0.5 * np.asarray(z, dtype=np.float64)))


def test_moe_reference_textbook_activations(orc):
    from scipy.special import erf, expit
    g = np.linspace(-10, 10, 101)
    u = np.linspace(-9, 9, 101)
    # SiLU against scipy's logistic and the tanh identity; silu(1) = sigma(1) = 0.7310585786 (tables)
    np.testing.assert_allclose(orc.act_fn(g, u, 0), g * expit(g) * u, rtol=1e-13)
    np.testing.assert_allclose(orc.act_fn(g, u, 0), g * _sigmoid_tanh(g) * u, rtol=1e-12, atol=1e-15)
    assert abs(orc.act_fn(np.array(1.0), np.array(1.0), 0) - 0.7310585786300049) < 1e-15
    # tanh-GELU against the erf form: the two GELUs agree to ~1e-3
    gelu_erf = 0.5 * g * (1 + erf(g / np.sqrt(2)))
    np.testing.assert_allclose(orc.act_fn(g, np.ones_like(g), 1), gelu_erf, atol=2e-3)


def test_gptoss_clamped_swiglu_pins(orc):
    """gpt-oss clamped SwiGLU (reference metal_mxfp4_gptoss.py:36-43, :116-121), pinned by what the definition
    fixes rather than by restating it: g saturates at 7 from above only, u is clipped to [-7, 7], the glu term
    is (u + 1), and alpha = 1.702 (hand values through the tanh form of the logistic)."""
    act = lambda g, u: orc.act_fn(np.asarray(g, np.float64), np.asarray(u, np.float64), 2)  # noqa: E731
    us = np.linspace(-6.5, 6.5, 27)
    for g in (7.0, 7.5, 50.0, 1e30):   # g >= 7 saturates
        np.testing.assert_array_equal(act(np.full_like(us, g), us), act(np.full_like(us, 7.0), us))
    assert act(-7.5, 0.0) != act(-7.0, 0.0)   # no clamp from below
    gs = np.linspace(-9.0, 6.9, 41)
    assert (act(gs, np.full_like(gs, -1.0)) == 0.0).all()   # u = -1 -> exactly 0 (u + 1 = 0)
    for u, lim in ((7.5, 7.0), (1e9, 7.0), (-8.0, -7.0), (-1e9, -7.0)):   # |u| > 7 saturates
        np.testing.assert_array_equal(act(gs, np.full_like(gs, u)), act(gs, np.full_like(gs, lim)))
    # hand values: act(1, 0) = sigma(1.702) = 0.8457958...; act(2, 1) = 2 * 2 * sigma(3.404); act(-1, 0) = -sigma(-1.702)
    assert abs(act(1.0, 0.0) - 0.8457958) < 1e-7
    assert abs(act(1.0, 0.0) - _sigmoid_tanh(1.702)) < 1e-14
    assert abs(act(2.0, 1.0) - 4.0 * _sigmoid_tanh(3.404)) < 1e-13
    assert abs(act(-1.0, 0.0) + _sigmoid_tanh(-1.702)) < 1e-14
    # in range it is g * sigma(1.702 g) * (u + 1): a wrong alpha, a missing + 1 or a swapped g / u fails here
    gi, ui = np.meshgrid(np.linspace(-6, 6.9, 13), np.linspace(-6.9, 6.9, 13))
    np.testing.assert_allclose(act(gi, ui), gi * _sigmoid_tanh(1.702 * gi) * (ui + 1.0), rtol=1e-12, atol=1e-14)


def test_error_metrics_hand_values(orc):
    """error_metrics on vectors small enough to compute by hand; every parity gate reads max_abs / rms_ref."""
    e = orc.error_metrics(np.array([1.0, 2.0, 3.0]), np.array([1.0, 2.0, 5.0]))
    assert e["max_abs"] == 2.0
    assert abs(e["rms_ref"] - math.sqrt(10.0)) < 1e-15          # sqrt((1 + 4 + 25) / 3)
    assert abs(e["rel_fro"] - 2.0 / math.sqrt(30.0)) < 1e-15    # |(0, 0, -2)| / |(1, 2, 5)|
    assert abs(e["cos"] - 20.0 / math.sqrt(14.0 * 30.0)) < 1e-15
    assert e["finite"] is True
    m = orc.error_metrics(np.array([[-3.0, 0.5], [4.0, 0.0]]), np.zeros((2, 2)))
    assert m["max_abs"] == 4.0 and m["rms_ref"] == 0.0            # max over every element, sign dropped
    assert orc.error_metrics(np.array([1.0, np.nan]), np.array([1.0, 1.0]))["finite"] is False
    assert orc.error_metrics(np.array([1.0, np.inf]), np.array([1.0, 1.0]))["finite"] is False
    z = orc.error_metrics(np.zeros(0), np.zeros(0))
    assert z["max_abs"] == 0.0 and z["rms_ref"] == 0.0


def test_moe_reference_invariants(orc):
    rng = np.random.default_rng(11)
    x, wg, wu, wd, idx, wts = _problem(rng, 6, 64, 32, 8, 4)
    y = orc.moe_reference(x, wg, wu, wd, idx, wts)
    np.testing.assert_allclose(orc.moe_reference(x, wg, wu, wd, idx, 3.0 * wts.astype(np.float64)), 3.0 * y,
                               rtol=1e-12, atol=1e-12)   # linear in the combine weights
    perm = np.array([2, 0, 3, 1])
    np.testing.assert_allclose(orc.moe_reference(x, wg, wu, wd, idx[:, perm], wts[:, perm]), y, rtol=1e-12)
    w0 = wts.copy()
    w0[0] = 0
    assert (orc.moe_reference(x, wg, wu, wd, idx, w0)[0] == 0).all()   # all-zero weights -> exactly 0
    # one expert, one token, identity-like weights: down(silu(g) * u) by hand
    e = int(idx[1, 0])
    h = orc.act_fn(wg[e] @ x[1], wu[e] @ x[1], 0)
    y1 = orc.moe_reference(x[1:2], wg, wu, wd, idx[1:2, :1], np.ones((1, 1)))
    np.testing.assert_allclose(y1[0], wd[e] @ h, rtol=1e-12)


def test_moe_reference_biases_and_shared(orc):
    rng = np.random.default_rng(12)
    x, wg, wu, wd, idx, wts = _problem(rng, 4, 64, 32, 4, 2)
    bg, bu, bd = rng.standard_normal((4, 32)), rng.standard_normal((4, 32)), rng.standard_normal((4, 64))
    y = orc.moe_reference(x, wg, wu, wd, idx, wts, 2, bg, bu, bd)
    for t in range(4):
        acc = np.zeros(64)
        for j in range(2):
            e = idx[t, j]
            acc += wts[t, j] * (wd[e] @ orc.act_fn(wg[e] @ x[t] + bg[e], wu[e] @ x[t] + bu[e], 2) + bd[e])
        np.testing.assert_allclose(y[t], acc, rtol=1e-12)
    sg, su, sd = rng.standard_normal((16, 64)), rng.standard_normal((16, 64)), rng.standard_normal((64, 16))
    ys = orc.moe_reference(x, wg, wu, wd, idx, wts, shared=[(sg, su, sd)])
    y0 = orc.moe_reference(x, wg, wu, wd, idx, wts)
    np.testing.assert_allclose(ys - y0, (orc.act_fn(x @ sg.T, x @ su.T, 0)) @ sd.T, rtol=1e-10, atol=1e-12)


def test_moe_reference_gated_shared_expert(orc):
    """Gated shared expert, token by token: sigmoid(x . w) * down(silu(g) * u); a gate of 0 halves it,
    a large positive gate passes it whole, a large negative one removes it."""
    rng = np.random.default_rng(14)
    x, wg, wu, wd, idx, wts = _problem(rng, 3, 64, 32, 4, 2)
    sg, su, sd = rng.standard_normal((16, 64)), rng.standard_normal((16, 64)), rng.standard_normal((64, 16))
    w = rng.standard_normal(64)
    y0 = orc.moe_reference(x, wg, wu, wd, idx, wts)
    ys = orc.moe_reference(x, wg, wu, wd, idx, wts, shared=[(sg, su, sd)], shared_gate=w)
    for t in range(3):
        sh = sd @ (sg @ x[t] / (1.0 + np.exp(-(sg @ x[t]))) * (su @ x[t]))
        np.testing.assert_allclose(ys[t] - y0[t], sh / (1.0 + np.exp(-(x[t] @ w))), rtol=1e-10, atol=1e-12)
    full = orc.moe_reference(x, wg, wu, wd, idx, wts, shared=[(sg, su, sd)])
    half = orc.moe_reference(x, wg, wu, wd, idx, wts, shared=[(sg, su, sd)], shared_gate=np.zeros(64))
    np.testing.assert_allclose(half - y0, 0.5 * (full - y0), rtol=1e-12, atol=1e-12)
    on = orc.moe_reference(x, wg, wu, wd, idx, wts, shared=[(sg, su, sd)], shared_gate=np.full(64, 1e3) * np.sign(x[0]))
    np.testing.assert_allclose(on[0], full[0], rtol=1e-12)


def test_torch_loop_matches_reference(orc):
    rng = np.random.default_rng(13)
    x, wg, wu, wd, idx, wts = _problem(rng, 5, 64, 32, 6, 2)
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))  # noqa: E731
    y = orc.torch_loop(t(wg), t(wu), t(wd), t(x), torch.from_numpy(idx).long(), t(wts))
    np.testing.assert_allclose(y.numpy(), orc.moe_reference(x, wg, wu, wd, idx, wts), rtol=1e-10)
    # gpt-oss: biases and the clamped SwiGLU (x scaled so that both clamps engage), and the tanh-GELU GLU
    bg, bu, bd = rng.standard_normal((6, 32)), rng.standard_normal((6, 32)), rng.standard_normal((6, 64))
    xs = 40.0 * x
    y2 = orc.torch_loop(t(wg), t(wu), t(wd), t(xs), torch.from_numpy(idx).long(), t(wts), act=2, bg=t(bg), bu=t(bu),
                        bd=t(bd))
    ref2 = orc.moe_reference(xs, wg, wu, wd, idx, wts, act=2, bg=bg, bu=bu, bd=bd)
    np.testing.assert_allclose(y2.numpy(), ref2, rtol=1e-10, atol=1e-10)
    g = xs @ wg[idx[0, 0]].T
    assert (g > 7).any() and (xs @ wu[idx[0, 0]].T < -7).any()   # the clamps engage
    y1 = orc.torch_loop(t(wg), t(wu), t(wd), t(x), torch.from_numpy(idx).long(), t(wts), act=1)
    np.testing.assert_allclose(y1.numpy(), orc.moe_reference(x, wg, wu, wd, idx, wts, act=1), rtol=1e-10)
