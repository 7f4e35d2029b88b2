"""Expert (and router) weights of a packed MLX-community checkpoint, from a LOCAL directory only, into the
states the gfx950 kernels run (reference tests/test_real_checkpoints.py:14-66 reads the same keys).

Supported layouts (the keys of mlx-lm's quantised SwitchGLU experts):
    int4 affine g64   model.layers.{l}.mlp.switch_mlp.{gate,up,down}_proj.{weight,scales,biases}
                      weight uint32 [E, N, K/8] (8 codes per word, low nibble first), scales and biases bf16
                      [E, N, K/64]                          (e.g. mlx-community/Qwen3-30B-A3B-4bit)
    MXFP4 (gpt-oss)   model.layers.{l}.mlp.experts.{gate,up,down}_proj.{weight,scales,bias}
                      weight uint32 [E, N, K/8] (E2M1 codes), scales uint8 [E, N, K/32] (E8M0), bias [E, N]
                                                            (e.g. mlx-community/gpt-oss-20b-MXFP4-Q8)
    router            model.layers.{l}.mlp.{gate,router}.weight [E, d] (+ .bias), either dense or mlx-quantised
                      (weight uint32 [E, d*bits/32] + scales + biases; bits and group size from config.json's
                      "quantization" entry for that module, else the global one).
The directory holds model.safetensors.index.json (its weight_map names the shard of every key) or a single
*.safetensors file. Files are read with safetensors (no code runs from them); nothing is downloaded.
"""
import glob
import json
import os

import torch

PROJ = ("gate_proj", "up_proj", "down_proj")


class Checkpoint:
    """Lazy key -> tensor access over the safetensors shards of one local model directory."""

    def __init__(self, path):
        from safetensors import safe_open
        self._open = safe_open
        self.path = path
        idx = os.path.join(path, "model.safetensors.index.json")
        if os.path.exists(idx):
            with open(idx) as f:
                self.weight_map = json.load(f)["weight_map"]
        else:
            files = sorted(glob.glob(os.path.join(path, "*.safetensors")))
            if not files:
                raise FileNotFoundError(f"no model.safetensors.index.json or *.safetensors under {path}")
            self.weight_map = {}
            for fn in files:
                with safe_open(fn, "pt") as f:
                    for k in f.keys():
                        self.weight_map[k] = os.path.basename(fn)
        cfg = os.path.join(path, "config.json")
        self.config = json.load(open(cfg)) if os.path.exists(cfg) else {}
        self._handles = {}

    def __contains__(self, key):
        return key in self.weight_map

    def get(self, key):
        fn = self.weight_map[key]
        if fn not in self._handles:
            self._handles[fn] = self._open(os.path.join(self.path, fn), "pt")
        return self._handles[fn].get_tensor(key)

    def quantization(self, module):
        q = self.config.get("quantization") or self.config.get("quantization_config") or {}
        own = q.get(module)
        if isinstance(own, dict):
            return own.get("group_size", 64), own.get("bits", 4)
        return q.get("group_size", 64), q.get("bits", 4)


def _words(t):
    """uint32 code words as the int32 tensors the packers take (same bits)."""
    return t.contiguous().view(torch.int32) if t.dtype == torch.uint32 else t.to(torch.int32)


def int4_experts_packed(ck, layer, prefix="model.layers.{l}.mlp.switch_mlp."):
    """((codes, scales, biases) x 3) of one layer's int4 experts, in the reference layout, on the CPU."""
    p = prefix.format(l=layer)
    out = []
    for pr in PROJ:
        w, s, b = (ck.get(p + f"{pr}.{part}") for part in ("weight", "scales", "biases"))
        if s.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
            raise ValueError(f"{p}{pr}: expected bf16 scales/biases, got {s.dtype}/{b.dtype}")
        if w.shape[-1] * 8 != s.shape[-1] * 64:
            raise ValueError(f"{p}{pr}: {w.shape[-1] * 8} inputs but {s.shape[-1]} groups of 64")
        out.append((_words(w), s.contiguous(), b.contiguous()))
    return tuple(out)


def mxfp4_experts_packed(ck, layer, prefix="model.layers.{l}.mlp.experts."):
    """((codes, e8m0) x 3, (bg, bu, bd) fp32) of one layer's MXFP4 experts, on the CPU."""
    p = prefix.format(l=layer)
    packs, biases = [], []
    for pr in PROJ:
        w, s = ck.get(p + f"{pr}.weight"), ck.get(p + f"{pr}.scales")
        if s.dtype != torch.uint8:
            raise ValueError(f"{p}{pr}.scales: expected uint8 E8M0, got {s.dtype}")
        if w.shape[-1] * 8 != s.shape[-1] * 32:
            raise ValueError(f"{p}{pr}: {w.shape[-1] * 8} inputs but {s.shape[-1]} groups of 32")
        packs.append((_words(w), s.contiguous()))
        key = p + f"{pr}.bias"
        biases.append(ck.get(key).to(torch.float32) if key in ck else None)
    return tuple(packs), tuple(biases)


def dequant_affine(words, scales, biases, bits, group_size):
    """mlx affine dequantisation of `bits`-bit codes packed little-endian in uint32 words (any bits dividing
    32): w = scale * q + bias per group of `group_size` along the last axis, in fp32."""
    per = 32 // bits
    w = _words(words).to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(per, dtype=torch.int64) * bits
    q = ((w.unsqueeze(-1) >> shifts) & ((1 << bits) - 1)).reshape(*w.shape[:-1], w.shape[-1] * per)
    K = q.shape[-1]
    q = q.to(torch.float32).reshape(*q.shape[:-1], K // group_size, group_size)
    out = q * scales.float().unsqueeze(-1) + biases.float().unsqueeze(-1)
    return out.reshape(*out.shape[:-2], K)


def router(ck, layer, names=("gate", "router")):
    """(weight bf16 [E, d], bias fp32 [E] or None) of one layer's router (dense or mlx-quantised)."""
    for n in names:
        p = f"model.layers.{layer}.mlp.{n}"
        if p + ".weight" not in ck:
            continue
        w = ck.get(p + ".weight")
        if p + ".scales" in ck:   # quantised linear
            gs, bits = ck.quantization(p)
            w = dequant_affine(w, ck.get(p + ".scales"), ck.get(p + ".biases"), bits, gs)
        bias = ck.get(p + ".bias").to(torch.float32) if p + ".bias" in ck else None
        return w.to(torch.bfloat16).contiguous(), bias
    raise KeyError(f"no router weight under model.layers.{layer}.mlp.{{{','.join(names)}}}")


def load_layer(path_or_ck, layer, fmt=None, device="cuda", with_router=True, tiles=True):
    """A run_layer state of one MoE layer from a local checkpoint: experts (int4 or MXFP4, detected from the
    keys unless fmt is given) and, when present, the router ("wr", "br"). gpt-oss MXFP4 layers get act 2
    (the clamped GLU) and their fp32 biases."""
    from .experts import make_state
    ck = path_or_ck if isinstance(path_or_ck, Checkpoint) else Checkpoint(path_or_ck)
    if fmt is None:
        fmt = "int4" if f"model.layers.{layer}.mlp.switch_mlp.gate_proj.weight" in ck else "mxfp4"
    to = (lambda t: None if t is None else t.to(device))  # noqa: E731
    if fmt == "int4":
        g, u, d = (tuple(t.to(device) for t in p) for p in int4_experts_packed(ck, layer))
        s = make_state("int4", g, u, d, tiles=tiles)
    else:
        (g, u, d), (bg, bu, bd) = mxfp4_experts_packed(ck, layer)
        g, u, d = (tuple(t.to(device) for t in p) for p in (g, u, d))
        s = make_state("mxfp4", g, u, d, to(bg), to(bu), to(bd), tiles=tiles)
        s["act"] = 2
    if with_router:
        try:
            w, b = router(ck, layer)
            s["wr"], s["br"] = w.to(device), to(b)
        except KeyError:
            pass
    return s
