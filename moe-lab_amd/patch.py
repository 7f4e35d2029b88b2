"""Torch MoE blocks onto the gfx950 kernels: the model-patch caller of the path (reference moelab/e2e.py:29-72
`patch`, moelab/universal.py:26-56), for transformers' sparse MoE blocks that keep their experts as stacked
tensors (Qwen3-MoE `Qwen3MoeSparseMoeBlock`, Mixtral `MixtralSparseMoeBlock`: `gate.weight` [E, d] and
`experts.gate_up_proj` [E, 2F, d] (gate rows first), `experts.down_proj` [E, d, F], SiLU GLU).

patch_block quantises the block's experts (int4 affine g64, or MXFP4) into a state, keeps the router weight in
bf16, and replaces the block's forward: route (gate GEMV + top-k + softmax over the top-k, or the full
softmax's top-k values when the block does not renormalise) then the experts on the GPU, y in the input's
dtype. The stock forward is kept on the block (`_moelab_stock_forward`) and unpatch_block restores it.
"""
import torch

from . import router
from .experts import run_layer
from .variants import hip_mxfp4_moe, hip_q4_moe


def is_moe_block(m):
    g, e = getattr(m, "gate", None), getattr(m, "experts", None)
    return (g is not None and e is not None and isinstance(getattr(g, "weight", None), torch.Tensor)
            and isinstance(getattr(e, "gate_up_proj", None), torch.Tensor)
            and isinstance(getattr(e, "down_proj", None), torch.Tensor))


def _act_of(experts):
    name = getattr(getattr(experts, "act_fn", None), "__class__", type(None)).__name__.lower()
    for k, v in (("silu", 0), ("swish", 0), ("gelu", 1)):
        if k in name:
            return v
    raise NotImplementedError(f"activation {name}: the kernels take SiLU or tanh-GELU GLUs")


@torch.no_grad()
def block_state(block, fmt="int4"):
    """(state, k, norm, act) of a transformers sparse MoE block."""
    e = block.experts
    F = e.gate_up_proj.shape[1] // 2
    gate, up = e.gate_up_proj[:, :F], e.gate_up_proj[:, F:]
    mod = hip_q4_moe if fmt == "int4" else hip_mxfp4_moe
    s = mod.prepare(gate.contiguous(), up.contiguous(), e.down_proj.contiguous())
    s["wr"] = block.gate.weight.detach().to(torch.bfloat16).contiguous()
    k = int(getattr(block.gate, "top_k", getattr(block, "top_k", 0)))
    norm = bool(getattr(block.gate, "norm_topk_prob", True))
    return s, k, norm, _act_of(e)


def patch_block(block, fmt="int4"):
    s, k, norm, act = block_state(block, fmt)

    def forward(hidden_states):
        shape = hidden_states.shape
        x = hidden_states.reshape(-1, shape[-1]).to(torch.bfloat16).contiguous()
        idx, wts = router.route(x, s["wr"], k, norm=norm)
        y = run_layer(s, x, idx, wts, act=act)
        return y.to(hidden_states.dtype).reshape(shape)

    block._moelab_stock_forward = block.forward
    block._moelab_state = s
    block.forward = forward
    return block


def unpatch_block(block):
    block.forward = block._moelab_stock_forward
    del block._moelab_stock_forward, block._moelab_state
    return block


def patch_model(model, fmt="int4"):
    """Patch every sparse MoE block of a model; returns how many were patched."""
    n = 0
    for m in model.modules():
        if is_moe_block(m) and not hasattr(m, "_moelab_state"):
            patch_block(m, fmt)
            n += 1
    return n


@torch.no_grad()
def load_dequantised(block):
    """Give the block's stock experts the weights the patched forward computes with (the state's dequantised
    codes), so stock and patched forwards differ only by arithmetic, not by quantisation."""
    s = block._moelab_state
    mod = hip_q4_moe if s["fmt"] == "int4" else hip_mxfp4_moe
    wg, wu, wd = mod.dequant(s)
    e = block.experts
    e.gate_up_proj.copy_(torch.cat([wg, wu], dim=1).to(e.gate_up_proj.dtype))
    e.down_proj.copy_(wd.to(e.down_proj.dtype))
