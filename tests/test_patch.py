"""Torch MoE-block patch (moe-lab_amd/patch.py) on transformers' Qwen3-MoE and Mixtral sparse blocks built from
small random configs (no checkpoint): the patched forward against the stock experts in fp32 on the same
dequantised weights and the same routing, and the routing against the stock router in fp32."""
import pytest
import torch

import __graft_entry__

__graft_entry__.load_package()
from moelab_amd import patch  # noqa: E402


def qwen3_block(device, norm=True):
    from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeSparseMoeBlock
    cfg = Qwen3MoeConfig(hidden_size=256, moe_intermediate_size=384, num_experts=8, num_experts_per_tok=2,
                         norm_topk_prob=norm, hidden_act="silu")
    return init(Qwen3MoeSparseMoeBlock(cfg), device)


def mixtral_block(device):
    from transformers.models.mixtral.configuration_mixtral import MixtralConfig
    from transformers.models.mixtral.modeling_mixtral import MixtralSparseMoeBlock
    cfg = MixtralConfig(hidden_size=256, intermediate_size=320, num_local_experts=4, num_experts_per_tok=2,
                        hidden_act="silu")
    return init(MixtralSparseMoeBlock(cfg), device)


@torch.no_grad()
def init(block, device):
    g = torch.Generator().manual_seed(0)
    e = block.experts
    E, F2, d = e.gate_up_proj.shape
    e.gate_up_proj.copy_(torch.randn(E, F2, d, generator=g) * d ** -0.5)
    e.down_proj.copy_(torch.randn(E, d, F2 // 2, generator=g) * (F2 // 2) ** -0.5)
    block.gate.weight.copy_(torch.randn(block.gate.weight.shape, generator=g) * 0.05)
    return block.to(device=device, dtype=torch.bfloat16).eval()


def test_detects_blocks_and_activation():
    b = qwen3_block("cpu")
    assert patch.is_moe_block(b) and not patch.is_moe_block(b.experts)
    assert patch._act_of(b.experts) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["qwen3", "qwen3-nonorm", "mixtral"])
def test_patched_block_matches_stock(kind):
    from helpers import assert_close
    from moelab_amd import router
    block = mixtral_block("cuda") if kind == "mixtral" else qwen3_block("cuda", norm=kind == "qwen3")
    x = torch.randn(2, 24, 256, generator=torch.Generator().manual_seed(1)).to("cuda", torch.bfloat16)
    print(f"case patch {kind}", flush=True)
    patch.patch_block(block)
    block.experts.float()             # the stock experts in fp32, so the dequantised weights land exactly
    patch.load_dequantised(block)
    with torch.no_grad():
        y = block(x)
    assert y.shape == x.shape and y.dtype == x.dtype
    flat = x.reshape(-1, 256)
    s = block._moelab_state
    k = 2
    norm = kind != "qwen3-nonorm"
    idx, wts = router.route(flat, s["wr"], k, norm=norm)
    # the stock router in fp32 picks the same experts (ties aside) with the same weights
    logits = flat.float() @ s["wr"].float().T
    probs = torch.softmax(logits, -1)
    top_v, top_i = torch.topk(probs, k, -1)
    if norm:
        top_v = top_v / top_v.sum(-1, keepdim=True)
    same = (torch.sort(idx.long(), -1).values == torch.sort(top_i, -1).values).all(-1)
    assert same.float().mean() > 0.95
    order = torch.argsort(idx.long(), -1)
    assert torch.allclose(torch.gather(wts, 1, order)[same], torch.gather(top_v, 1, torch.argsort(top_i, -1))[same],
                          atol=1e-5)
    # the stock experts in fp32 with that routing and the same (dequantised) weights
    with torch.no_grad():
        ref = block.experts(flat.float(), idx.long(), wts.float()).cpu().numpy()
    assert_close(y.reshape(-1, 256), ref, what=("patch", kind))
    patch.unpatch_block(block)
    assert not hasattr(block, "_moelab_state")
