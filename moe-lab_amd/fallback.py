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
