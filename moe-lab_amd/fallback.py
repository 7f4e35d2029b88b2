"""Above-threshold fallback of the production dispatchers (reference moelab/fallback.py:17-34).

The reference falls back to mlx-lm's SwitchGLU path: a gather matmul per (token, slot) that reads the
selected expert's weights for every slot. MI355X has no stock quantised gather-matmul, so the same
per-slot semantics run on this library's per-slot GEMV (MOE_PATH_SLOTS): every slot streams its own
expert's packed rows, with no grouping, and y = sum_j wts[t, j] * expert_j(x_t). This is also the
"per-slot stock-style gather" arm the grouped path is measured against.
"""
from . import _lib
from .experts import run_layer


def gather_moe(s, x, idx, wts, group_size=None, bits=None, mode="affine", act=0, residual=None, out_dtype=None):
    return run_layer(s, x, idx, wts, act=act, path=_lib.PATH_SLOTS, residual=residual, out_dtype=out_dtype)


def grouped_from_load(D, F):
    """Load T*k/E from which the grouped path beats the per-slot path on MI355X (grid.py; int4 and MXFP4
    alike). Fitted on five shapes, grouped/per-slot time at the loads around the crossing:
        qwen3-30b-a3b   (D*F 1.6M)  loses at 0.5 (0.93x), wins at 1.0 (1.10x)
        olmoe-1b-7b     (D*F 2.1M)  loses at 0.5 (0.94x), wins at 1.0 (1.12x)
        deepseek-v2-lite (2.9M)     loses at 0.19 (0.94x), wins at 0.28 (1.18x)
        gpt-oss-20b     (8.3M)      loses at 0.25 (0.81x), wins at 0.5 (1.18x)
        mixtral-8x7b    (58.7M)     wins from the smallest grid load, 0.5 (1.09x)
    and the grouped path wins at every larger load (up to 55x at Mixtral T=512). So: 1.0 for experts below
    2.5 Mi weights per projection, 0.27 above. The reference's policy is the other way round (its custom
    kernels up to a load of 8-24, mlx-lm's gather above, reference metal_q4_moe.py:42-46), because its
    fallback is a stock gather-matmul that wins at high load; here the fallback is this library's per-slot
    GEMV, which re-reads an expert for every slot and wins only where slots rarely share an expert."""
    return 1.0 if D * F < 5 << 19 else 0.27


MIN_GROUPED_WAVES = 256   # gate/up wave tiles (32 rows each) the grouped path needs near its load threshold


def grouped_waves(T, k, E, F):
    """Expected live gate/up wave tiles of a grouped call: the expected number of distinct experts among T*k
    uniformly routed slots, U = E (1 - (1 - 1/E)^(T k)), passes max(U, T k / 16), times F / 32 row blocks."""
    n = T * k
    U = E * (1.0 - (1.0 - 1.0 / E) ** n)
    return max(U, n / 16) * F / 32


def grouped_wins(T, k, E, D, F):
    """The MI355X dispatch rule of the production dispatchers: grouped from the load grouped_from_load(D, F); near
    that threshold (below twice the load) only when the grouped gate/up has MIN_GROUPED_WAVES live wave tiles.
    With fewer, each wave walks its whole K with two slices in flight and the launch cannot fill the memory
    pipe, while the per-slot GEMV spreads the same rows over many waves: random-shape sweeps found the per-slot
    path 1.5-1.7x faster at d = 3328, F = 384, E = 16, k = 2, T = 8 (~124 such waves) and d = 896, F = 320, E = 32,
    k = 2, T = 16 (~202), while every grouped win near the threshold had 447 or more (the fitted model shapes:
    690-1950)."""
    load = T * k / E
    L0 = grouped_from_load(D, F)
    if load < L0:
        return False
    return load >= 2 * L0 or grouped_waves(T, k, E, F) >= MIN_GROUPED_WAVES

