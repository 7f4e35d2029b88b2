"""Router, router tail and grouping on the GPU vs the CPU oracle: logits, ids and grouping bit-exact,
weights within 1e-6 relative (exp and summation order differ between CPU and GPU)."""
import numpy as np
import pytest
import torch

from helpers import np_u16, orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _router_inputs(T, d, E, seed, bias=False):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn((T, d), generator=g, device=DEV).to(torch.bfloat16)
    wr = (torch.randn((E, d), generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    b = None
    if bias:
        from moelab_amd.problem import zipf_bias
        b = torch.from_numpy(zipf_bias(E, 1.1, seed)).to(DEV)
    return x, wr, b


@pytest.mark.parametrize("E,k,d", [(128, 8, 2048), (32, 4, 2880), (64, 6, 2048), (8, 2, 4096), (8, 1, 512),
                                   (1000, 8, 256), (1024, 32, 64), (16, 16, 128)])
@pytest.mark.parametrize("T", [1, 7, 32, 64])
def test_route_bit_exact(E, k, d, T):
    from moelab_amd import router
    x, wr, _ = _router_inputs(T, d, E, seed=E + T + k)
    idx, wts, logits = router.route(x, wr, k, return_logits=True)
    lg_ref = orc.router_logits(np_u16(x), np_u16(wr))
    np.testing.assert_array_equal(logits.cpu().numpy().view(np.uint32), lg_ref.view(np.uint32))
    idx_ref, wts_ref = orc.topk(lg_ref, k)
    np.testing.assert_array_equal(idx.cpu().numpy(), idx_ref)
    np.testing.assert_allclose(wts.cpu().numpy(), wts_ref, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("T", [1, 32])
def test_route_bias_zipf_and_full_softmax(T):
    from moelab_amd import router
    E, k, d = 128, 8, 2048
    x, wr, b = _router_inputs(T, d, E, seed=5, bias=True)
    for norm, scale in ((True, 1.0), (False, 1.0), (False, 2.5)):
        idx, wts, logits = router.route(x, wr, k, bias=b, norm=norm, scale=scale, return_logits=True)
        lg_ref = orc.router_logits(np_u16(x), np_u16(wr), b.cpu().numpy())
        np.testing.assert_array_equal(logits.cpu().numpy().view(np.uint32), lg_ref.view(np.uint32))
        idx_ref, wts_ref = orc.topk(lg_ref, k, norm=norm, scale=scale)
        np.testing.assert_array_equal(idx.cpu().numpy(), idx_ref)
        np.testing.assert_allclose(wts.cpu().numpy(), wts_ref, rtol=1e-6, atol=1e-7)


def test_route_repeated_calls_agree():
    """Many calls in a row give identical results (the router keeps no state between calls)."""
    from moelab_amd import router
    x, wr, _ = _router_inputs(5, 512, 64, seed=1)
    first = router.route(x, wr, 6)
    for _ in range(20):
        again = router.route(x, wr, 6)
        assert torch.equal(first[0], again[0]) and torch.equal(first[1], again[1])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("E,k", [(8, 2), (60, 4), (128, 8), (256, 8), (512, 32), (1000, 8)])
def test_topk_norm_bit_exact_ids(dtype, E, k):
    from moelab_amd import router
    g = torch.Generator(device=DEV).manual_seed(E * 7 + k)
    lg = (torch.randn((64, E), generator=g, device=DEV) * 3).to(dtype)   # bf16/fp16 values tie often
    idx, wts = router.topk_norm(lg, k)
    idx_ref, wts_ref = orc.topk(lg.float().cpu().numpy(), k)
    np.testing.assert_array_equal(idx.cpu().numpy(), idx_ref)
    np.testing.assert_allclose(wts.cpu().numpy(), wts_ref, rtol=1e-6, atol=1e-7)


def test_topk_ties_and_nonfinite():
    from moelab_amd import router
    idx, wts = router.topk_norm(torch.zeros((3, 64), device=DEV), 6)
    np.testing.assert_array_equal(idx.cpu().numpy(), np.tile(np.arange(6), (3, 1)))
    np.testing.assert_allclose(wts.cpu().numpy(), 1 / 6, atol=1e-6)
    for bad in (float("nan"), float("-inf")):
        lg = torch.from_numpy(np.random.default_rng(0).standard_normal((4, 64)).astype(np.float32))
        lg[0, :] = bad
        lg[1, 3:] = bad
        idx, wts = router.topk_norm(lg.to(DEV), 6)
        idx_ref, wts_ref = orc.topk(lg.numpy(), 6)
        np.testing.assert_array_equal(idx.cpu().numpy(), idx_ref)
        np.testing.assert_allclose(wts.cpu().numpy()[1:], wts_ref[1:], rtol=1e-6, atol=1e-7)


def test_topk_full_softmax_weights():
    from moelab_amd import router
    lg = torch.randn((33, 64), device=DEV) * 2
    idx, wts = router.topk_norm(lg, 6, norm=False)
    idx_ref, wts_ref = orc.topk(lg.cpu().numpy(), 6, norm=False)
    np.testing.assert_array_equal(idx.cpu().numpy(), idx_ref)
    np.testing.assert_allclose(wts.cpu().numpy(), wts_ref, rtol=1e-5)


@pytest.mark.parametrize("T,k,E", [(1, 8, 128), (32, 8, 128), (256, 6, 64), (512, 2, 8), (17, 4, 16),
                                   (5, 1, 1), (64, 8, 1024), (1024, 8, 128), (3000, 8, 128), (4, 3, 8192),
                                   (2001, 3, 7)])
@pytest.mark.parametrize("routing", ["uniform", "one_hot"])
def test_group_bit_exact(T, k, E, routing):
    from moelab_amd import router
    from moelab_amd.problem import make_routing
    idx_np, _ = make_routing(T, E, k, routing, np.random.default_rng(T + E))
    counts, offsets, srt, active, meta = router.group(torch.from_numpy(idx_np).to(DEV), E)
    c, o, s, a = orc.group(idx_np, E)
    np.testing.assert_array_equal(counts.cpu().numpy(), c)
    np.testing.assert_array_equal(offsets.cpu().numpy(), o)
    np.testing.assert_array_equal(srt.cpu().numpy(), s)
    m = meta.cpu().numpy()
    assert m[0] == len(a) and m[1] == 0
    np.testing.assert_array_equal(active.cpu().numpy()[:len(a)], a)
    assert (active.cpu().numpy()[len(a):] == -1).all()


def test_group_rejects_out_of_range_ids():
    from moelab_amd import router
    idx = torch.tensor([[0, 5], [3, 99], [-1, 3]], dtype=torch.int32, device=DEV)
    counts, offsets, srt, active, meta = router.group(idx, 8)
    assert meta.cpu().numpy()[1] == 2
    assert counts.cpu().numpy().tolist() == [1, 0, 0, 2, 0, 1, 0, 0]
    assert srt.cpu().numpy()[:4].tolist() == [0, 2, 5, 1]


@pytest.mark.parametrize("T,E,k,d,mode", [(1, 128, 8, 2048, "plain"), (32, 128, 8, 2048, "plain"),
                                          (32, 128, 8, 2048, "zipf"), (64, 128, 8, 2048, "ties"),
                                          (65, 128, 8, 2048, "zipf"), (256, 64, 6, 2048, "plain"),
                                          (512, 8, 2, 4096, "plain"), (448, 128, 8, 256, "zipf"),
                                          (7, 1000, 8, 256, "plain"), (512, 128, 32, 128, "plain"),
                                          (300, 1000, 32, 64, "plain"), (2000, 64, 6, 128, "zipf"),
                                          (64, 1024, 32, 64, "ties"), (33, 16, 16, 128, "plain")])
def test_route_group_bit_exact(T, E, k, d, mode):
    """moe_router_group: the router launch also sorts the slots by expert (its last workgroup, a wave prefix sum of
    the counts). Ids and logits bit-exact against the oracle, the grouping equal to the oracle's stable argsort
    (reference triton_fused_moe.py:56-70) and to the separate route + group launches. (448, 128, 8): 3584 slots,
    the largest the 4-wave form takes at E = 128; E = 1000 and 1024 take the one-wave form; "ties": every router row
    equal, so every token picks experts 0..k-1 and all slots fall on k experts."""
    from moelab_amd import router
    x, wr, b = _router_inputs(T, d, E, seed=T * 3 + E + k, bias=mode == "zipf")
    if mode == "ties":
        wr = torch.full_like(wr, 0.0078125)
    print(f"case route_group T={T} E={E} k={k} {mode}", flush=True)
    idx, wts, logits, (counts, offsets, srt, active, meta) = router.route_group(x, wr, k, bias=b)
    lg_ref = orc.router_logits(np_u16(x), np_u16(wr), None if b is None else b.cpu().numpy())
    np.testing.assert_array_equal(logits.cpu().numpy().view(np.uint32), lg_ref.view(np.uint32))
    idx_ref, wts_ref = orc.topk(lg_ref, k)
    np.testing.assert_array_equal(idx.cpu().numpy(), idx_ref)
    np.testing.assert_allclose(wts.cpu().numpy(), wts_ref, rtol=1e-6, atol=1e-7)
    c, o, s, a = orc.group(idx_ref, E)
    np.testing.assert_array_equal(counts.cpu().numpy(), c)
    np.testing.assert_array_equal(offsets.cpu().numpy(), o)
    np.testing.assert_array_equal(srt.cpu().numpy(), s)
    m = meta.cpu().numpy()
    assert m[0] == len(a) and m[1] == 0
    np.testing.assert_array_equal(active.cpu().numpy()[:len(a)], a)
    assert (active.cpu().numpy()[len(a):] == -1).all()
    i2, w2 = router.route(x, wr, k, bias=b)
    g2 = router.group(i2, E)
    assert torch.equal(idx, i2) and torch.equal(wts, w2)
    for u, v in zip((counts, offsets, srt, active), g2[:4]):
        assert torch.equal(u, v)
    if mode == "ties":
        assert (idx.cpu().numpy() == np.arange(k)).all()


@pytest.mark.parametrize("T", [3, 200])
def test_route_group_repeated_calls(T):
    """20 calls in a row agree: one finishing workgroup (T = 3) and the last-workgroup grouping, whose arrival counter
    the logits launch zeroes on every call (T = 200)."""
    from moelab_amd import router
    x, wr, _ = _router_inputs(T, 512, 64, seed=2)
    first = router.route_group(x, wr, 6)
    for _ in range(20):
        again = router.route_group(x, wr, 6)
        assert torch.equal(first[0], again[0]) and all(torch.equal(u, v) for u, v in zip(first[3], again[3]))
