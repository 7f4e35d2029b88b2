"""Torch MoE-block patches (moe-lab_amd/patch.py) on transformers' sparse MoE blocks built from small random configs
(no checkpoint): Qwen3-MoE (renormalised and not), Mixtral, OLMoE, Qwen2-MoE with its gated shared expert (merged
into the routed set, and at a width that is not a multiple of the routed experts'), DeepSeek-V2 with 2 shared experts
(greedy gate with routed_scaling_factor, and a group-limited gate that stays stock), gpt-oss (MXFP4, router bias,
interleaved gate/up with biases, clamped SwiGLU), and the universal per-slot patch of an experts module at T = 1 and
T > 1. Each patched forward is checked against the stock modules in fp32 on the same dequantised weights and the same
routing, and the fused router's choice against the stock router in fp32."""
import pytest
import torch

import __graft_entry__

__graft_entry__.load_package()
from moelab_amd import patch  # noqa: E402

D = 256


@torch.no_grad()
def _init(block, device, seed=0):
    g = torch.Generator().manual_seed(seed)
    for n, p in block.named_parameters():
        fan_in = p.shape[-1] if p.dim() > 1 else 64
        if "gate_up_proj" in n and p.dim() == 3 and "bias" not in n and p.shape[1] == D and p.shape[2] != D:
            fan_in = p.shape[1]   # gpt-oss stores its experts transposed: x @ W
        scale = 0.05 if n.endswith("gate.weight") or "router" in n or "shared_expert_gate" in n else fan_in ** -0.5
        if "bias" in n:
            scale = 0.01
        p.copy_(torch.randn(p.shape, generator=g) * scale)
    return block.to(device=device, dtype=torch.bfloat16).eval()


def make_block(kind, device):
    if kind in ("qwen3", "qwen3-nonorm"):
        from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig
        from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeSparseMoeBlock
        cfg = Qwen3MoeConfig(hidden_size=D, moe_intermediate_size=384, num_experts=8, num_experts_per_tok=2,
                             norm_topk_prob=kind == "qwen3", hidden_act="silu")
        return _init(Qwen3MoeSparseMoeBlock(cfg), device)
    if kind == "mixtral":
        from transformers.models.mixtral.configuration_mixtral import MixtralConfig
        from transformers.models.mixtral.modeling_mixtral import MixtralSparseMoeBlock
        cfg = MixtralConfig(hidden_size=D, intermediate_size=320, num_local_experts=4, num_experts_per_tok=2,
                            hidden_act="silu")
        return _init(MixtralSparseMoeBlock(cfg), device)
    if kind == "olmoe":
        from transformers.models.olmoe.configuration_olmoe import OlmoeConfig
        from transformers.models.olmoe.modeling_olmoe import OlmoeSparseMoeBlock
        cfg = OlmoeConfig(hidden_size=D, intermediate_size=256, num_experts=16, num_experts_per_tok=4)
        return _init(OlmoeSparseMoeBlock(cfg), device)
    if kind in ("qwen2-shared", "qwen2-shared-odd"):
        from transformers.models.qwen2_moe.configuration_qwen2_moe import Qwen2MoeConfig
        from transformers.models.qwen2_moe.modeling_qwen2_moe import Qwen2MoeSparseMoeBlock
        cfg = Qwen2MoeConfig(hidden_size=D, moe_intermediate_size=256, num_experts=8, num_experts_per_tok=2,
                             shared_expert_intermediate_size=512 if kind == "qwen2-shared" else 320,
                             norm_topk_prob=False)
        return _init(Qwen2MoeSparseMoeBlock(cfg), device)
    if kind in ("deepseek", "deepseek-group"):
        from transformers.models.deepseek_v2.configuration_deepseek_v2 import DeepseekV2Config
        from transformers.models.deepseek_v2.modeling_deepseek_v2 import DeepseekV2Moe
        cfg = DeepseekV2Config(hidden_size=D, moe_intermediate_size=256, n_routed_experts=8, num_experts_per_tok=3,
                               n_shared_experts=2, routed_scaling_factor=2.5, n_group=2, topk_group=1,
                               topk_method="greedy" if kind == "deepseek" else "group_limited_greedy",
                               hidden_act="silu")
        return _init(DeepseekV2Moe(cfg), device)
    if kind == "gpt-oss":
        from transformers.models.gpt_oss.configuration_gpt_oss import GptOssConfig
        from transformers.models.gpt_oss.modeling_gpt_oss import GptOssMLP
        return _init(GptOssMLP(GptOssConfig(hidden_size=D, intermediate_size=256, num_local_experts=8,
                                            num_experts_per_tok=4)), device)
    raise ValueError(kind)


KINDS = {"qwen3": "stacked", "qwen3-nonorm": "stacked", "mixtral": "stacked", "olmoe": "stacked",
         "qwen2-shared": "qwen2-shared", "qwen2-shared-odd": "qwen2-shared", "deepseek": "deepseek",
         "deepseek-group": "deepseek", "gpt-oss": "gpt-oss"}


@pytest.mark.parametrize("kind", list(KINDS))
def test_detects_blocks_and_activation(kind):
    b = make_block(kind, "cpu")
    assert patch.block_kind(b) == KINDS[kind] and not patch.is_moe_block(b.experts)
    if kind != "gpt-oss":
        assert patch._act_of(b.experts) == 0


def _stock_routing(block, kind, flat32):
    """The stock router in fp32: (idx [T, k], wts [T, k])."""
    out = block.router(flat32) if kind == "gpt-oss" else block.gate(flat32)
    return out[2].long(), out[1].float()


def _stock_experts(block, kind, flat32, idx, wts):
    """The stock expert modules in fp32 (dequantised weights) on the given routing, plus the block's shared term."""
    y = block.experts(flat32, idx.long(), wts.float())
    if kind == "deepseek":
        y = y + block.shared_experts(flat32)
    elif kind == "qwen2-shared":
        y = y + torch.sigmoid(block.shared_expert_gate(flat32)) * block.shared_expert(flat32)
    return y


@pytest.mark.gpu
@pytest.mark.parametrize("kind", list(KINDS))
@pytest.mark.parametrize("T", [1, 24])
def test_patched_block_matches_stock(kind, T):
    from helpers import assert_close
    from moelab_amd import router
    block = make_block(kind, "cuda")
    family = KINDS[kind]
    x = torch.randn(1, T, D, generator=torch.Generator().manual_seed(T)).to("cuda", torch.bfloat16)
    print(f"case patch {kind} T={T}", flush=True)
    patch.patch_block(block)
    cfg = block._moelab_cfg
    if kind == "qwen2-shared" or kind == "deepseek":
        assert "n_shared" in block._moelab_state          # shared experts merged into the routed set
    if kind == "qwen2-shared-odd":
        assert "shared" in block._moelab_state            # 320 is not a multiple of 256: a second call
    block.float()            # the stock modules in fp32, so the dequantised weights land exactly
    patch.load_dequantised(block)
    with torch.no_grad():
        out = block(x)
    y = out[0] if family == "gpt-oss" else out
    assert y.shape == x.shape and y.dtype == x.dtype
    flat = x.reshape(-1, D)
    flat32 = flat.float()
    s = block._moelab_state
    k = cfg["k"]
    with torch.no_grad():
        if cfg["stock_gate"]:
            idx, wts = patch._route_stock(block, flat32)
        else:
            idx, wts = router.route(flat, s["wr"], k, bias=cfg["bias"], norm=cfg["norm"], scale=cfg["scale"])
        sid, swts = _stock_routing(block, family, flat32)
        # the stock router in fp32 picks the same experts (near-ties aside) with the same weights
        same = (torch.sort(idx.long(), -1).values == torch.sort(sid, -1).values).all(-1)
        assert same.float().mean() > 0.9, same
        o1, o2 = torch.argsort(idx.long(), -1), torch.argsort(sid, -1)
        assert torch.allclose(torch.gather(wts, 1, o1)[same], torch.gather(swts, 1, o2)[same], rtol=1e-4, atol=1e-5)
        if family == "gpt-oss":
            assert torch.equal(out[1].float(), wts.to(out[1].dtype).float())
        ref = _stock_experts(block, family, flat32, idx, wts).cpu().numpy()
    assert_close(y.reshape(-1, D), ref, what=("patch", kind, T))
    patch.unpatch_block(block)
    assert not hasattr(block, "_moelab_state")


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["qwen3", "olmoe", "deepseek"])
@pytest.mark.parametrize("T", [1, 24])
def test_universal_experts_patch(kind, T):
    """patch_experts replaces only the experts module's per-slot compute (run_slots at T = 1, one row per slot
    above); the weighting and the sum over each token's slots are applied after the kernels."""
    from helpers import assert_close
    block = make_block(kind, "cuda")
    e = block.experts
    x = torch.randn(T, D, generator=torch.Generator().manual_seed(T + 1)).to("cuda", torch.bfloat16)
    E = e.gate_up_proj.shape[0]
    k = 3
    g = torch.Generator(device="cuda").manual_seed(T)
    idx = torch.stack([torch.randperm(E, generator=g, device="cuda")[:k] for _ in range(T)])
    wts = torch.rand((T, k), generator=g, device="cuda")
    print(f"case universal {kind} T={T}", flush=True)
    patch.patch_experts(e)
    e.float()
    patch.load_dequantised(e)
    with torch.no_grad():
        y = e(x, idx, wts)
        ref = e._moelab_stock_forward(x.float(), idx, wts).cpu().numpy()
    assert y.dtype == x.dtype and y.shape == x.shape
    assert_close(y, ref, what=("universal", kind, T))
    patch.unpatch_experts(e)


@pytest.mark.gpu
def test_patch_model_counts_blocks():
    """patch_model on a tiny two-layer Qwen2-MoE model: every sparse block (or, universal, every experts module)."""
    from transformers.models.qwen2_moe.configuration_qwen2_moe import Qwen2MoeConfig
    from transformers.models.qwen2_moe.modeling_qwen2_moe import Qwen2MoeForCausalLM
    cfg = Qwen2MoeConfig(hidden_size=D, moe_intermediate_size=256, num_experts=8, num_experts_per_tok=2,
                         shared_expert_intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                         num_key_value_heads=4, intermediate_size=512, vocab_size=128)
    m = Qwen2MoeForCausalLM(cfg).to("cuda", torch.bfloat16).eval()
    assert patch.patch_model(m) == 2
    with torch.no_grad():
        out = m(torch.arange(6, device="cuda").reshape(1, 6)).logits
    assert out.shape == (1, 6, 128) and torch.isfinite(out.float()).all()
    m2 = Qwen2MoeForCausalLM(cfg).to("cuda", torch.bfloat16).eval()
    assert patch.patch_model(m2, universal=True) == 2
