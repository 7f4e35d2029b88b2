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
