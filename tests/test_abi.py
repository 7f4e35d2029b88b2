"""The C-ABI library loads, exports every entry point include/moe_mi355x.h declares, and rejects
invalid arguments before touching the GPU (host-side checks only; no kernel runs here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "moe_mi355x.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(moe_\w+)\s*\(", src, flags=re.M)))


def test_header_declares_the_api():
    fns = declared_functions()
    for n in ("moe_router", "moe_topk", "moe_group", "moe_experts_run", "moe_experts_workspace_bytes"):
        assert n in fns, fns


def test_library_exports_every_declared_symbol():
    from moelab_amd import _lib
    L = _lib.lib()
    for n in declared_functions():
        assert hasattr(L, n), n
    assert set(_lib.EXPORTS) <= set(declared_functions())
    assert b"gfx950" in L.moe_version()


def _desc(E=8, d=128, F=128, fmt=0):
    from moelab_amd import _lib
    fake = ctypes.c_void_p(4096)   # never dereferenced: argument checks return before any launch
    p = _lib.Proj(fake, None, None)
    return _lib.Experts(fmt, E, d, F, p, p, p)


def test_workspace_query_host_only():
    from moelab_amd import _lib
    L = _lib.lib()
    w = _desc(E=128, d=2048, F=768)
    slots = L.moe_experts_workspace_bytes(w, 1, 8, _lib.PATH_SLOTS)
    assert slots >= 8 * 768 * 2
    grouped = L.moe_experts_workspace_bytes(w, 32, 8, _lib.PATH_GROUPED)
    assert grouped >= 256 * 768 * 2 + 256 * 2048 * 4


@pytest.mark.parametrize("case,rc", [("d_not_64", -1), ("bad_fmt", -2), ("bad_act", -1), ("no_ws", -3),
                                     ("bad_dtype", -2), ("nored_grouped", -1), ("misaligned", -5)])
def test_argument_errors_before_launch(case, rc):
    from moelab_amd import _lib
    L = _lib.lib()
    w = _desc()
    x = ctypes.c_void_p(4096)
    act, dtype, path, nored, ws, wsb = 0, 0, 0, 0, ctypes.c_void_p(8192), 1 << 30
    if case == "d_not_64":
        w = _desc(d=96)
    elif case == "bad_fmt":
        w = _desc(fmt=7)
    elif case == "bad_act":
        act = 9
    elif case == "no_ws":
        ws, wsb = None, 0
    elif case == "bad_dtype":
        dtype = 5
    elif case == "nored_grouped":
        path, nored = _lib.PATH_GROUPED, 1
    elif case == "misaligned":
        x = ctypes.c_void_p(4097)
    got = L.moe_experts_run(w, x, dtype, x, x, 4, 2, act, path, nored, ctypes.c_void_p(4096), 0, None, ws, wsb,
                            None)
    assert got == rc


def test_router_argument_errors():
    from moelab_amd import _lib
    L = _lib.lib()
    p = ctypes.c_void_p(4096)
    assert L.moe_router(p, p, None, 1, 2048, 2048, 8, 1, 1.0, p, p, p, p, None) == -1   # E > 1024
    assert L.moe_router(p, p, None, 1, 2048, 128, 33, 1, 1.0, p, p, p, p, None) == -1   # k > 32
    assert L.moe_topk(p, 0, 1, 16, 17, 1, 1.0, p, p, None) == -1                        # k > E
    assert L.moe_group(p, 4, 0, p, p, p, p, p, None) == -1                              # E < 1


def test_router_group_and_layer_argument_errors():
    """moe_router_group's and the layer calls' argument checks, before any launch."""
    from moelab_amd import _lib
    L = _lib.lib()
    p = ctypes.c_void_p(4096)
    args = (p, p, p, p, p, p, p, p)
    assert L.moe_router_group(p, p, None, 4, 2048, 128, 33, 1, 1.0, *args, None) == -1    # k > 32
    assert L.moe_router_group(p, p, None, 4, 2048, 128, 8, 1, 1.0, p, p, p, None, p, p, p, p, None) == -1
    assert L.moe_router_group(p, p, None, 0, 2048, 128, 8, 1, 1.0, *args, None) == 0
    w = _desc(E=10, d=128, F=128)
    ws = ctypes.c_void_p(8192)
    # fp16 x: the router reads bf16
    assert L.moe_layer_run(w, p, 1, p, None, 4, 2, 1, 1.0, 0, p, p, p, 0, None, ws, 1 << 30, None) == -2
    # S = 0, S >= E, k + S > 64
    for S, k in ((0, 2), (10, 2), (8, 60)):
        assert L.moe_layer_run_shared(w, S, p, 0, p, None, None, 4, k, 1, 1.0, 0, p, p, p, 0, None, ws, 1 << 30,
                                      None) == -1
    assert L.moe_layer_shared_workspace_bytes(w, 2, 4, 2) > L.moe_layer_workspace_bytes(_desc(E=8), 4, 4) > 0
    assert L.moe_layer_run_shared(w, 2, p, 0, p, None, None, 4, 2, 1, 1.0, 0, p, p, p, 0, None, ws, 100,
                                  None) == -3


def test_tile_bytes_and_pack_argument_errors():
    from moelab_amd import _lib
    L = _lib.lib()
    assert L.moe_tile_bytes(0, 768, 2048) == 48 * 16 * 1152 + 768   # int4: + one row-exponent byte per row
    assert L.moe_tile_bytes(1, 2880, 2880) == 180 * 23 * 1088
    assert L.moe_tile_bytes(0, 24, 2048) == 0 and L.moe_tile_bytes(0, 32, 96) == 0 and L.moe_tile_bytes(5, 32, 64) == 0
    p, q = ctypes.c_void_p(4096), ctypes.c_void_p(8192)
    assert L.moe_tiles_pack(0, 2, 24, 128, p, q, None) == _lib.MOE_ERR_ARG
    assert L.moe_tiles_pack(0, 2, 32, 96, p, q, None) == _lib.MOE_ERR_ARG
    assert L.moe_tiles_pack(7, 2, 32, 128, p, q, None) == _lib.MOE_ERR_DTYPE
    assert L.moe_tiles_pack(0, 2, 32, 128, ctypes.c_void_p(4100), q, None) == _lib.MOE_ERR_ALIGN
    assert L.moe_tiles_pack(0, 2, 32, 128, p, None, None) == _lib.MOE_ERR_ARG


def test_misaligned_tiles_rejected_before_launch():
    from moelab_amd import _lib
    L = _lib.lib()
    fake = ctypes.c_void_p(4096)
    p = _lib.Proj(fake, None, ctypes.c_void_p(4104))
    w = _lib.Experts(0, 8, 128, 128, p, p, p)
    x = ctypes.c_void_p(4096)
    got = L.moe_experts_run(w, x, 0, x, x, 4, 2, 0, _lib.PATH_GROUPED, 0, x, 0, None, ctypes.c_void_p(8192), 1 << 30,
                            None)
    assert got == _lib.MOE_ERR_ALIGN


def test_buffer_growth_keeps_old_buffers_and_refuses_growth_during_capture(monkeypatch):
    """_lib.grow (the per-device expert workspace): a buffer that is large enough is returned as
    is; a smaller one is replaced by one of at least twice its size and kept alive (a HIP graph captured with it
    keeps its raw pointer); growing while the current stream captures raises (host-only: the capture state is
    stubbed)."""
    import torch
    from moelab_amd import _lib
    table, made = {}, []

    def make(n):
        made.append(n)
        return torch.empty(n, dtype=torch.uint8)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    a = _lib.grow(table, 0, 1000, make, "t")
    assert a.numel() == 1000 and _lib.grow(table, 0, 999, make, "t") is a
    retired0 = len(_lib._RETIRED)
    b = _lib.grow(table, 0, 1500, make, "t")
    assert b.numel() == 2000 and made == [1000, 2000]          # at least double the old size
    assert len(_lib._RETIRED) == retired0 + 1 and _lib._RETIRED[-1] is a
    c = _lib.grow(table, 0, 10_000, make, "t")
    assert c.numel() == 10_000
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    assert _lib.grow(table, 0, 10_000, make, "t") is c          # no growth needed: fine while capturing
    with pytest.raises(RuntimeError, match="reserve"):
        _lib.grow(table, 0, 10_001, make, "t")
    assert table[0] is c
