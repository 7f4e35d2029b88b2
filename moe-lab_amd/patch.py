"""Torch MoE blocks onto the gfx950 kernels: the model-patch callers of the path (reference moelab/e2e.py:29-175
`patch` and its per-family variants, moelab/universal.py:26-56), for transformers' sparse MoE blocks.

Two levels, as in the reference:

* ``patch_block`` replaces a whole sparse MoE block's forward: the router runs inside the layer call
  (experts.run_routed: moe_layer_run / moe_layer_run_shared, the router's launches also group the slots) and the
  experts and shared experts on the kernels. Families (detected from the block's modules):
    - "stacked": Qwen3-MoE, Mixtral, OLMoE (``gate.weight`` [E, d]; ``experts.gate_up_proj`` [E, 2F, d], gate rows
      first, ``experts.down_proj`` [E, d, F]; SiLU or tanh-GELU GLU): softmax, top-k, renormalised when the router
      says so (reference e2e.py:57-64);
    - "qwen2-shared": the same plus Qwen-style gated shared expert, y + sigmoid(x . w_sg) * shared(x)
      (reference e2e.py:66-68);
    - "deepseek": DeepSeek-V2 ``DeepseekV2Moe``: greedy gate = full-softmax probabilities of the top-k times
      ``routed_scaling_factor`` (reference e2e.py:129-150: the fused router for greedy gates, the stock gate for
      group-limited ones), plus the shared experts added (e2e.py:146-147);
    - "gpt-oss": ``GptOssMLP``: router with bias, top-k of the logits, softmax over them; MXFP4 experts stored
      transposed with gate and up interleaved, per-expert biases, clamped SwiGLU (reference e2e.py:153-175); the
      forward returns (y, routing weights) as the stock one does.
  Shared experts whose width is S times the routed experts' are split into S experts of that width and merged into
  the routed set (one expert call per layer, experts.merge_shared); other widths run as a second call.
* ``patch_experts`` (the reference's SwitchGLU-level universal patch) replaces only an experts module's per-slot
  computation: every (token, expert) slot is a row of its own with weight 1 (run_slots, the per-slot GEMV without
  its k-reduction, at T = 1), and the routing weights and the sum over a token's slots are applied afterwards,
  outside the kernels, so the model's own router and any extra terms stay as they are.

The stock forwards are kept (``_moelab_stock_forward``); ``unpatch_block`` / ``unpatch_experts`` restore them.
``load_dequantised`` writes the state's dequantised weights back into the stock modules, so stock and patched
forwards then differ by arithmetic only, not by quantisation.
"""
import torch

from . import _lib
from .experts import merge_shared, run_experts, run_layer, run_routed
from .variants import hip_mxfp4_moe, hip_q4_moe

_FMT = {"int4": hip_q4_moe, "mxfp4": hip_mxfp4_moe}


def _stacked(e):
    """Experts stored as stacked tensors gate_up [E, 2F, d] (gate rows first) and down [E, d, F], no biases."""
    return (e is not None and isinstance(getattr(e, "gate_up_proj", None), torch.Tensor)
            and isinstance(getattr(e, "down_proj", None), torch.Tensor) and getattr(e, "gate_up_proj_bias", None) is None
            and e.gate_up_proj.dim() == 3 and e.down_proj.dim() == 3
            and e.gate_up_proj.shape[1] == 2 * e.down_proj.shape[2] and e.gate_up_proj.shape[2] == e.down_proj.shape[1])


def block_kind(m):
    """The family of a transformers sparse MoE block, or None."""
    e = getattr(m, "experts", None)
    router = getattr(m, "router", None)
    if (router is not None and e is not None and isinstance(getattr(e, "gate_up_proj_bias", None), torch.Tensor)
            and isinstance(getattr(router, "bias", None), torch.Tensor)):
        return "gpt-oss"
    gate = getattr(m, "gate", None)
    if gate is None or not isinstance(getattr(gate, "weight", None), torch.Tensor) or not _stacked(e):
        return None
    if getattr(m, "shared_experts", None) is not None and hasattr(gate, "routed_scaling_factor"):
        return "deepseek"
    if getattr(m, "shared_expert", None) is not None and getattr(m, "shared_expert_gate", None) is not None:
        return "qwen2-shared"
    return "stacked"


def is_moe_block(m):
    return block_kind(m) is not None


def _act_of(module):
    name = getattr(getattr(module, "act_fn", None), "__class__", type(None)).__name__.lower()
    for k, v in (("silu", _lib.ACT_SWIGLU), ("swish", _lib.ACT_SWIGLU), ("gelu", _lib.ACT_GEGLU)):
        if k in name:
            return v
    raise NotImplementedError(f"activation {name}: the kernels take SiLU, tanh-GELU or gpt-oss's clamped GLU")


def _quantise(fmt, gate, up, down):
    """Dense gate/up [E, F, d], down [E, d, F] -> a packed state of the format."""
    return _FMT[fmt].prepare(gate.contiguous(), up.contiguous(), down.contiguous())


def _mlp_as_experts(mlp, F):
    """A dense GLU MLP (gate_proj/up_proj [Fs, d], down_proj [d, Fs]) as S = Fs / F experts of width F:
    (gate [S, F, d], up [S, F, d], down [S, d, F]); the GLU acts elementwise, so the S experts' sum is the MLP."""
    g, u, dn = mlp.gate_proj.weight, mlp.up_proj.weight, mlp.down_proj.weight
    Fs, d = g.shape
    S = Fs // F
    return g.reshape(S, F, d), u.reshape(S, F, d), dn.reshape(d, S, F).permute(1, 0, 2)


@torch.no_grad()
def block_state(block, fmt=None):
    """The block's packed state and call settings: {"kind", "state", "k", "norm", "scale", "act", "bias",
    "stock_gate"} (stock_gate: route with the block's own gate, for gates the fused router does not implement)."""
    kind = block_kind(block)
    if kind is None:
        raise ValueError(f"{type(block).__name__}: not a sparse MoE block this patch knows")
    cfg = {"kind": kind, "scale": 1.0, "bias": None, "stock_gate": False}
    if kind == "gpt-oss":
        e, r = block.experts, block.router
        gu = e.gate_up_proj                       # [E, d, 2F], columns gate, up, gate, up, ...
        s = _quantise(fmt or "mxfp4", gu[..., ::2].transpose(1, 2), gu[..., 1::2].transpose(1, 2),
                      e.down_proj.transpose(1, 2))
        s["bg"] = e.gate_up_proj_bias[:, ::2].float().contiguous()
        s["bu"] = e.gate_up_proj_bias[:, 1::2].float().contiguous()
        s["bd"] = e.down_proj_bias.float().contiguous()
        s["wr"] = r.weight.detach().to(torch.bfloat16).contiguous()
        cfg.update(state=s, k=int(r.top_k), norm=True, act=_lib.ACT_GPTOSS, bias=r.bias.detach().float().contiguous())
        return cfg
    e, gate = block.experts, block.gate
    F = e.gate_up_proj.shape[1] // 2
    fmt = fmt or "int4"
    s = _quantise(fmt, e.gate_up_proj[:, :F], e.gate_up_proj[:, F:], e.down_proj)
    s["wr"] = gate.weight.detach().to(torch.bfloat16).contiguous()
    cfg.update(k=int(getattr(gate, "top_k", getattr(block, "top_k", 0))), norm=bool(getattr(gate, "norm_topk_prob", True)),
               act=_act_of(e))
    shared = None
    if kind == "deepseek":
        cfg["norm"] = False   # greedy: the full softmax's probabilities of the top-k
        cfg["scale"] = float(gate.routed_scaling_factor)
        cfg["stock_gate"] = getattr(gate, "topk_method", "greedy") != "greedy"
        shared = block.shared_experts
    elif kind == "qwen2-shared":
        shared = block.shared_expert
        s["shared_gate"] = block.shared_expert_gate.weight.detach().reshape(-1).to(torch.bfloat16).contiguous()
    if shared is not None:
        Fs = shared.gate_proj.weight.shape[0]
        if Fs % F == 0 and Fs // F + cfg["k"] <= 64:   # S experts of the routed width: merged, one call per layer
            s["shared"] = _quantise(fmt, *_mlp_as_experts(shared, F))
            s = merge_shared(s)
        else:                                          # one shared expert of its own width, a second call
            s["shared"] = _quantise(fmt, *(t.unsqueeze(0) for t in (shared.gate_proj.weight, shared.up_proj.weight,
                                                                   shared.down_proj.weight)))
    cfg["state"] = s
    return cfg


def _route_stock(block, hidden):
    """The block's own gate on the tokens (DeepSeek group-limited gates): (idx int32 [T, k], wts fp32 [T, k])."""
    out = block.gate(hidden)
    wts, idx = out[1], out[2]
    return idx.to(torch.int32).contiguous(), wts.float().contiguous()


def patch_block(block, fmt=None):
    """Replace a sparse MoE block's forward by the kernels (router inside the layer call). fmt: "int4" (default for
    the stacked families) or "mxfp4" (default for gpt-oss)."""
    cfg = block_state(block, fmt)
    s = cfg["state"]

    def forward(hidden_states):
        shape = hidden_states.shape
        x = hidden_states.reshape(-1, shape[-1]).to(torch.bfloat16).contiguous()
        if cfg["stock_gate"]:
            idx, wts = _route_stock(block, hidden_states.reshape(-1, shape[-1]))
            y = run_layer(s, x, idx, wts, act=cfg["act"])
        else:
            y, idx, wts = run_routed(s, x, s["wr"], cfg["k"], bias=cfg["bias"], norm=cfg["norm"], scale=cfg["scale"],
                                     act=cfg["act"])
        y = y.to(hidden_states.dtype).reshape(shape)
        if cfg["kind"] == "gpt-oss":
            return y, wts.to(hidden_states.dtype)
        return y

    block._moelab_stock_forward = block.forward
    block._moelab_state = s
    block._moelab_cfg = cfg
    block.forward = forward
    return block


def unpatch_block(block):
    block.forward = block._moelab_stock_forward
    del block._moelab_stock_forward, block._moelab_state, block._moelab_cfg
    return block


def patch_experts(experts, fmt="int4"):
    """Universal patch of a stacked experts module (forward(hidden_states [T, d], top_k_index [T, k],
    top_k_weights [T, k]) -> [T, d]): the kernels compute each (token, expert) slot as a row of its own with weight
    1 (T = 1: run_slots, the per-slot GEMV without its k-reduction; T > 1: the T*k slots as rows with k = 1), and
    the routing weights and the sum over each token's k slots are applied afterwards in fp32 (reference
    universal.py:26-56: only the per-slot compute is replaced, the model keeps its routing and weighting)."""
    if not _stacked(experts):
        raise ValueError(f"{type(experts).__name__}: not a stacked experts module")
    F = experts.gate_up_proj.shape[1] // 2
    with torch.no_grad():
        s = _quantise(fmt, experts.gate_up_proj[:, :F], experts.gate_up_proj[:, F:], experts.down_proj)
    act = _act_of(experts)

    def forward(hidden_states, top_k_index, top_k_weights):
        T, d = hidden_states.shape
        k = top_k_index.shape[-1]
        x = hidden_states.to(torch.bfloat16).contiguous()
        idx = top_k_index.to(torch.int32).contiguous()
        if T == 1:
            ones = torch.ones((1, k), dtype=torch.float32, device=x.device)
            slots = run_experts(s, x, idx, ones, act=act, path=_lib.PATH_SLOTS, nored=True, out_dtype=torch.float32)
        else:
            rows = x.repeat_interleave(k, dim=0)
            ones = torch.ones((T * k, 1), dtype=torch.float32, device=x.device)
            slots = run_experts(s, rows, idx.reshape(T * k, 1), ones, act=act, out_dtype=torch.float32)
        y = (slots.reshape(T, k, d) * top_k_weights.float().reshape(T, k, 1)).sum(1)
        return y.to(hidden_states.dtype)

    experts._moelab_stock_forward = experts.forward
    experts._moelab_state = s
    experts.forward = forward
    return experts


def unpatch_experts(experts):
    experts.forward = experts._moelab_stock_forward
    del experts._moelab_stock_forward, experts._moelab_state
    return experts


def patch_model(model, fmt=None, universal=False):
    """Patch every sparse MoE block of a model (universal: every stacked experts module instead); returns how many
    modules were patched."""
    n = 0
    for m in list(model.modules()):
        if hasattr(m, "_moelab_state"):
            continue
        if universal:
            if _stacked(m) and not hasattr(m, "gate_up_proj_bias"):
                patch_experts(m, fmt or "int4")
                n += 1
        elif is_moe_block(m):
            patch_block(m, fmt)
            n += 1
    return n


def _deq(s):
    mod = hip_q4_moe if s["fmt"] == "int4" else hip_mxfp4_moe
    return mod.dequant(s)


@torch.no_grad()
def load_dequantised(module):
    """Write the patched module's dequantised weights back into its stock modules (experts, shared experts), so
    stock and patched forwards see the same weights."""
    s = module._moelab_state
    cfg = getattr(module, "_moelab_cfg", {"kind": "experts"})
    wg, wu, wd = _deq(s)
    kind = cfg["kind"]
    if kind == "experts":
        e = module
    else:
        e = module.experts
    if kind == "gpt-oss":
        gu = e.gate_up_proj
        gu[..., ::2].copy_(wg.transpose(1, 2).to(gu.dtype))
        gu[..., 1::2].copy_(wu.transpose(1, 2).to(gu.dtype))
        e.down_proj.copy_(wd.transpose(1, 2).to(e.down_proj.dtype))
        return
    E = e.gate_up_proj.shape[0]
    e.gate_up_proj.copy_(torch.cat([wg[:E], wu[:E]], dim=1).to(e.gate_up_proj.dtype))
    e.down_proj.copy_(wd[:E].to(e.down_proj.dtype))
    shared = module.shared_experts if kind == "deepseek" else (module.shared_expert if kind == "qwen2-shared" else None)
    if shared is None:
        return
    if "n_shared" in s:   # merged: experts E .. E + S - 1
        sg, su, sd = wg[E:], wu[E:], wd[E:]
    else:
        sg, su, sd = _deq(s["shared"])
    S, F, d = sg.shape
    shared.gate_proj.weight.copy_(sg.reshape(S * F, d).to(shared.gate_proj.weight.dtype))
    shared.up_proj.weight.copy_(su.reshape(S * F, d).to(shared.up_proj.weight.dtype))
    shared.down_proj.weight.copy_(sd.permute(1, 0, 2).reshape(d, S * F).to(shared.down_proj.weight.dtype))
