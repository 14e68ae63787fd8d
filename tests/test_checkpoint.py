"""Checkpoint loader (reference benchmarks/commands/run_kernel_track.py:192-207) on
synthetic safetensors files with the Qwen3 tensor naming: merge order, fp16 -> fp32 scale
widening, sharded checkpoints, and the checks that reject what the FP8 linear cannot take."""

import json
import os

import pytest
import torch
from safetensors.torch import save_file

from minillm_amd import checkpoint as ckpt

# A small Qwen3-shaped layer: hidden 256, 2 query heads of 128, 1 kv head, intermediate 384.
DIMS = {"self_attn.q_proj": (256, 256), "self_attn.k_proj": (128, 256), "self_attn.v_proj": (128, 256),
        "self_attn.o_proj": (256, 256), "mlp.gate_proj": (384, 256), "mlp.up_proj": (384, 256),
        "mlp.down_proj": (256, 384)}


def _tensors(layers=2, seed=0, scale_dtype=torch.float16):
    gen = torch.Generator().manual_seed(seed)
    out = {}
    for layer in range(layers):
        for module, (n, k) in DIMS.items():
            base = f"model.layers.{layer}.{module}"
            out[f"{base}.weight"] = (torch.randn(n, k, generator=gen) * 64).clamp(-448, 448).to(torch.float8_e4m3fn)
            out[f"{base}.weight_scale_inv"] = (torch.rand(-(-n // 128), -(-k // 128), generator=gen) * 0.01
                                               + 1e-4).to(scale_dtype)
    out["model.embed_tokens.weight"] = torch.zeros(8, 256, dtype=torch.bfloat16)
    return out


def _bits(t):
    return t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t


def test_single_file_merges_in_reference_order(tmp_path):
    tensors = _tensors()
    path = tmp_path / "model.safetensors"
    save_file(tensors, str(path))
    for source in (str(path), str(tmp_path)):
        ck = ckpt.FP8Checkpoint(source)
        assert ck.num_layers() == 2
        weights = ckpt.load_layer_weights(source, 1, device="cpu")
        assert set(weights) == {"qkv", "o", "gate_up", "down"}
        for name, modules in ckpt.PROJECTIONS.items():
            w, s = weights[name]
            ref_w = torch.cat([tensors[f"model.layers.1.{m}.weight"] for m in modules])
            ref_s = torch.cat([tensors[f"model.layers.1.{m}.weight_scale_inv"] for m in modules]).float()
            assert w.dtype == torch.float8_e4m3fn and torch.equal(_bits(w), _bits(ref_w))
            assert s.dtype == torch.float32 and torch.equal(s, ref_s)  # fp16 -> fp32 is exact
    qkv_w, qkv_s = weights["qkv"]
    assert qkv_w.shape == (512, 256) and qkv_s.shape == (4, 2)


def test_sharded_checkpoint_via_index(tmp_path):
    tensors = _tensors(layers=2, seed=3, scale_dtype=torch.bfloat16)
    names = sorted(tensors)
    shards = {"model-00001-of-00002.safetensors": names[::2], "model-00002-of-00002.safetensors": names[1::2]}
    weight_map = {}
    for shard, members in shards.items():
        save_file({n: tensors[n] for n in members}, str(tmp_path / shard))
        weight_map.update({n: shard for n in members})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    weights = ckpt.FP8Checkpoint(str(tmp_path)).layer_weights(0)
    w, s = weights["gate_up"]
    assert torch.equal(_bits(w), _bits(torch.cat([tensors["model.layers.0.mlp.gate_proj.weight"],
                                                  tensors["model.layers.0.mlp.up_proj.weight"]])))
    assert torch.equal(s, torch.cat([tensors["model.layers.0.mlp.gate_proj.weight_scale_inv"],
                                     tensors["model.layers.0.mlp.up_proj.weight_scale_inv"]]).float())


def test_rejects_what_the_linear_cannot_take(tmp_path):
    bad = _tensors(layers=1)
    bad["model.layers.0.self_attn.o_proj.weight_scale_inv"] = torch.ones(3, 2, dtype=torch.float16)  # wrong shape
    save_file(bad, str(tmp_path / "a.safetensors"))
    ck = ckpt.FP8Checkpoint(str(tmp_path / "a.safetensors"))
    with pytest.raises(ValueError, match="does not match"):
        ck.projection(0, ckpt.PROJECTIONS["o"])
    with pytest.raises(KeyError):
        ck.projection(0, ("self_attn.missing",))

    bad = _tensors(layers=1)
    bad["model.layers.0.mlp.down_proj.weight"] = torch.zeros(256, 384, dtype=torch.bfloat16)  # not fp8
    save_file(bad, str(tmp_path / "b.safetensors"))
    with pytest.raises(ValueError, match="float8_e4m3fn"):
        ckpt.FP8Checkpoint(str(tmp_path / "b.safetensors")).projection(0, ckpt.PROJECTIONS["down"])

    # A merged part whose rows are not a multiple of 128 would put two projections' rows in
    # one scale block.
    odd = {"model.layers.0.a.weight": torch.zeros(100, 256, dtype=torch.float8_e4m3fn),
           "model.layers.0.a.weight_scale_inv": torch.ones(1, 2, dtype=torch.float16),
           "model.layers.0.b.weight": torch.zeros(128, 256, dtype=torch.float8_e4m3fn),
           "model.layers.0.b.weight_scale_inv": torch.ones(1, 2, dtype=torch.float16)}
    save_file(odd, str(tmp_path / "c.safetensors"))
    ck = ckpt.FP8Checkpoint(str(tmp_path / "c.safetensors"))
    with pytest.raises(ValueError, match="multiples of 128"):
        ck.projection(0, ("a", "b"))
    w, s = ck.projection(0, ("a",))  # a single part may have a row tail
    assert w.shape == (100, 256) and s.shape == (1, 2)

    with pytest.raises(FileNotFoundError):
        ckpt.FP8Checkpoint(str(tmp_path / "nowhere"))
    os.makedirs(tmp_path / "empty")
    with pytest.raises(FileNotFoundError):
        ckpt.FP8Checkpoint(str(tmp_path / "empty"))
