"""Local-checkpoint loading (moe-lab_amd/checkpoint.py) on synthetic mlx-layout safetensors written here: the
keys and dtypes of mlx-community's int4 SwitchGLU and gpt-oss MXFP4 experts (reference
tests/test_real_checkpoints.py:40-66), sharded with an index, and an 8-bit quantised router."""
import json

import numpy as np
import pytest
import torch

import __graft_entry__

__graft_entry__.load_package()
from moelab_amd import checkpoint, formats  # noqa: E402
from moelab_amd.experts import make_state  # noqa: E402

E, D, F = 4, 128, 192


def u32(words):
    return words.contiguous().view(torch.uint32)


def write(tmp_path, tensors_by_shard, config=None):
    from safetensors.torch import save_file
    wm = {}
    for shard, tensors in tensors_by_shard.items():
        save_file(tensors, str(tmp_path / shard))
        wm.update({k: shard for k in tensors})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wm}))
    if config is not None:
        (tmp_path / "config.json").write_text(json.dumps(config))


def int4_layer(seed):
    g = torch.Generator().manual_seed(seed)
    return [formats.random_int4(E, n, k, generator=g) for n, k in ((F, D), (F, D), (D, F))]


def router8(seed):
    """8-bit mlx-quantised router: codes, scales, biases and the fp32 weights they stand for (numpy)."""
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 256, (E, D)).astype(np.uint32)
    words = (q.reshape(E, D // 4, 4) << (8 * np.arange(4, dtype=np.uint32))).sum(-1).astype(np.uint32)
    s = torch.from_numpy(rng.uniform(1e-3, 2e-3, (E, D // 64)).astype(np.float32)).to(torch.bfloat16)
    b = torch.from_numpy(rng.uniform(-0.1, 0.1, (E, D // 64)).astype(np.float32)).to(torch.bfloat16)
    w = q.reshape(E, D // 64, 64) * s.float().numpy()[..., None] + b.float().numpy()[..., None]
    return torch.from_numpy(words.view(np.int32)), s, b, w.reshape(E, D)


def test_int4_layer_and_quantised_router(tmp_path):
    packs = int4_layer(1)
    rq, rs, rb, rw = router8(2)
    p = "model.layers.3.mlp."
    t0 = {p + f"switch_mlp.{pr}.{part}": (u32(t) if part == "weight" else t)
          for pr, pk in zip(checkpoint.PROJ[:2], packs[:2]) for part, t in zip(("weight", "scales", "biases"), pk)}
    t1 = {p + f"switch_mlp.down_proj.{part}": (u32(t) if part == "weight" else t)
          for part, t in zip(("weight", "scales", "biases"), packs[2])}
    t1.update({p + "gate.weight": u32(rq), p + "gate.scales": rs, p + "gate.biases": rb})
    write(tmp_path, {"model-00001-of-00002.safetensors": t0, "model-00002-of-00002.safetensors": t1},
          {"quantization": {"group_size": 64, "bits": 4, "model.layers.3.mlp.gate": {"group_size": 64, "bits": 8}}})
    ck = checkpoint.Checkpoint(str(tmp_path))
    got = checkpoint.int4_experts_packed(ck, 3)
    for (a, b_, c), (x, y, z) in zip(got, packs):
        assert torch.equal(a, x) and torch.equal(b_, y) and torch.equal(c, z)
    w, bias = checkpoint.router(ck, 3)
    assert bias is None and w.dtype == torch.bfloat16
    assert np.array_equal(w.float().numpy(), torch.from_numpy(rw.astype(np.float32)).to(torch.bfloat16).float().numpy())
    s = checkpoint.load_layer(str(tmp_path), 3, device="cpu")
    ref = make_state("int4", *packs)
    assert s["fmt"] == "int4" and all(torch.equal(s[n], ref[n]) for n in ("g", "u", "d"))
    assert torch.equal(s["wr"], w)


def test_dequant_affine_matches_int4_restatement():
    codes, scales, biases = formats.random_int4(2, 8, 128, generator=torch.Generator().manual_seed(4))
    a = checkpoint.dequant_affine(codes, scales, biases, bits=4, group_size=64)
    assert torch.equal(a, formats.dequant_int4(codes, scales, biases))


def test_mxfp4_layer(tmp_path):
    g = torch.Generator().manual_seed(5)
    packs = [formats.random_mxfp4(E, n, k, generator=g) for n, k in ((F, D), (F, D), (D, F))]
    biases = [(torch.randn(E, n, generator=g) * 0.01).to(torch.bfloat16) for n in (F, F, D)]
    p = "model.layers.0.mlp.experts."
    t = {}
    for pr, (c, sc), bb in zip(checkpoint.PROJ, packs, biases):
        t.update({p + f"{pr}.weight": u32(c), p + f"{pr}.scales": sc, p + f"{pr}.bias": bb})
    t["model.layers.0.mlp.router.weight"] = (torch.randn(E, D, generator=g) * 0.02).to(torch.bfloat16)
    t["model.layers.0.mlp.router.bias"] = (torch.randn(E, generator=g) * 0.02).to(torch.bfloat16)
    write(tmp_path, {"model.safetensors": t})
    s = checkpoint.load_layer(str(tmp_path), 0, device="cpu")
    assert s["fmt"] == "mxfp4" and s["act"] == 2
    ref = make_state("mxfp4", *packs, *(b.float() for b in biases))
    for n in ("g", "u", "d", "bg", "bu", "bd"):
        assert torch.equal(s[n], ref[n]), n
    assert torch.equal(s["wr"], t["model.layers.0.mlp.router.weight"])
    assert torch.equal(s["br"], t["model.layers.0.mlp.router.bias"].float())


def test_errors_name_the_key(tmp_path):
    packs = int4_layer(6)
    p = "model.layers.0.mlp.switch_mlp."
    t = {p + f"{pr}.{part}": (u32(x) if part == "weight" else x.float() if part == "scales" else x)
         for pr, pk in zip(checkpoint.PROJ, packs) for part, x in zip(("weight", "scales", "biases"), pk)}
    write(tmp_path, {"model.safetensors": t})
    with pytest.raises(ValueError, match="gate_proj"):
        checkpoint.int4_experts_packed(checkpoint.Checkpoint(str(tmp_path)), 0)
    with pytest.raises(FileNotFoundError):
        checkpoint.Checkpoint(str(tmp_path / "missing"))


@pytest.mark.gpu
def test_loaded_layer_runs_at_the_gate(tmp_path):
    """A layer loaded from the local checkpoint onto the GPU (with tile copies) through the router and the
    experts, against the oracle on the same packed weights."""
    from helpers import assert_close, oracle_y
    from moelab_amd import router
    from moelab_amd.experts import run_layer
    packs = int4_layer(7)
    p = "model.layers.0.mlp."
    t = {p + f"switch_mlp.{pr}.{part}": (u32(x) if part == "weight" else x)
         for pr, pk in zip(checkpoint.PROJ, packs) for part, x in zip(("weight", "scales", "biases"), pk)}
    t[p + "gate.weight"] = (torch.randn(E, D, generator=torch.Generator().manual_seed(8)) * 0.05).to(torch.bfloat16)
    write(tmp_path, {"model.safetensors": t})
    s = checkpoint.load_layer(str(tmp_path), 0, device="cuda")
    x = torch.randn(40, D, generator=torch.Generator().manual_seed(9)).to("cuda", torch.bfloat16)
    print("case checkpoint layer T=40", flush=True)
    idx, wts = router.route(x, s["wr"], 2)
    y = run_layer(s, x, idx, wts, out_dtype=torch.float32)
    assert_close(y, oracle_y(s, x, idx, wts), what="checkpoint layer")
