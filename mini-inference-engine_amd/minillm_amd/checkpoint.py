"""FP8 checkpoint loader: the block-quantized projection weights of one decoder layer.

The reference benchmark loads Qwen3-4B-FP8 weights straight from the safetensors file
(benchmarks/commands/run_kernel_track.py:192-207, ``load_layer_weights``): per layer the
e4m3fn ``weight`` [N, K] and ``weight_scale_inv`` [ceil(N/128), ceil(K/128)] of each
projection, q/k/v and gate/up concatenated along N as the engine runs them merged, and the
scales, stored as fp16, widened to fp32 at load.  This module does the same for a single
``model.safetensors`` file, a directory holding one, or a sharded checkpoint with a
``model.safetensors.index.json`` weight map, and checks what the FP8 linear needs of
the result:
- e4m3fn 2-D weights with one K;
- scale shapes that match;
- merged parts whose row counts are multiples of 128, so no scale block straddles two
  projections.

Each merged tensor is allocated once on the target device, and the parts are copied into
its row ranges.  Scales are widened to fp32, which is exact from fp16 and bf16.
"""

from __future__ import annotations

import json
import os
from collections.abc import Iterable
from typing import Any

import torch

BLOCK = 128

# Merged projection name -> the checkpoint modules it concatenates, in order (the
# reference's ``parts``, run_kernel_track.py:200-201).
PROJECTIONS: dict[str, tuple[str, ...]] = {
    "qkv": ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"),
    "o": ("self_attn.o_proj",),
    "gate_up": ("mlp.gate_proj", "mlp.up_proj"),
    "down": ("mlp.down_proj",),
}

_SCALE_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


class FP8Checkpoint:
    """Index of the tensors of an FP8 safetensors checkpoint (single file or shards)."""

    def __init__(self, path: str, prefix: str = "model.layers.") -> None:
        self.prefix = prefix
        self._files: dict[str, str] = {}  # tensor name -> file
        if os.path.isdir(path):
            index = os.path.join(path, "model.safetensors.index.json")
            single = os.path.join(path, "model.safetensors")
            if os.path.exists(index):
                with open(index) as fh:
                    weight_map = json.load(fh)["weight_map"]
                self._files = {name: os.path.join(path, shard) for name, shard in weight_map.items()}
            elif os.path.exists(single):
                self._index_file(single)
            else:
                raise FileNotFoundError(f"no model.safetensors or model.safetensors.index.json in {path}")
        elif os.path.exists(path):
            self._index_file(path)
        else:
            raise FileNotFoundError(path)

    def _index_file(self, file: str) -> None:
        from safetensors import safe_open

        with safe_open(file, framework="pt", device="cpu") as handle:
            for name in handle.keys():
                self._files[name] = file

    def names(self) -> list[str]:
        return sorted(self._files)

    def num_layers(self) -> int:
        layers = set()
        for name in self._files:
            if name.startswith(self.prefix):
                head = name[len(self.prefix):].split(".", 1)[0]
                if head.isdigit():
                    layers.add(int(head))
        return max(layers) + 1 if layers else 0

    def _shape_dtype(self, name: str) -> tuple[tuple[int, ...], torch.dtype]:
        from safetensors import safe_open

        if name not in self._files:
            raise KeyError(f"checkpoint has no tensor {name!r}")
        with safe_open(self._files[name], framework="pt", device="cpu") as handle:
            piece = handle.get_slice(name)
            shape = tuple(int(d) for d in piece.get_shape())
            dtype = _DTYPES.get(piece.get_dtype())
        if dtype is None:
            raise ValueError(f"{name}: unsupported safetensors dtype")
        return shape, dtype

    def _copy_into(self, name: str, out: torch.Tensor) -> None:
        from safetensors import safe_open

        with safe_open(self._files[name], framework="pt", device="cpu") as handle:
            out.copy_(handle.get_tensor(name), non_blocking=False)

    def projection(self, layer: int, modules: Iterable[str], device: Any = "cpu"
                   ) -> tuple[torch.Tensor, torch.Tensor]:
        """``(weight, scales)`` of ``modules`` of one layer, concatenated along N: e4m3fn
        [sum N, K] and fp32 [sum N / 128, ceil(K / 128)]."""

        modules = tuple(modules)
        if not modules:
            raise ValueError("no modules to load")
        base = f"{self.prefix}{layer}."
        parts = []
        for module in modules:
            w_name, s_name = f"{base}{module}.weight", f"{base}{module}.weight_scale_inv"
            (w_shape, w_dtype), (s_shape, s_dtype) = self._shape_dtype(w_name), self._shape_dtype(s_name)
            if w_dtype != torch.float8_e4m3fn or len(w_shape) != 2:
                raise ValueError(f"{w_name}: expected a 2-D float8_e4m3fn weight, got {w_dtype} {w_shape}")
            if s_dtype not in _SCALE_DTYPES:
                raise ValueError(f"{s_name}: expected fp16, bf16 or fp32 scales, got {s_dtype}")
            n, k = w_shape
            if s_shape != (_cdiv(n, BLOCK), _cdiv(k, BLOCK)):
                raise ValueError(f"{s_name}: shape {s_shape} does not match a {n} x {k} weight in 128 x 128 blocks")
            parts.append((w_name, s_name, n, k))
        k = parts[0][3]
        if any(p[3] != k for p in parts):
            raise ValueError(f"layer {layer}: {modules} do not share one input width")
        if len(parts) > 1 and any(p[2] % BLOCK for p in parts):
            raise ValueError(f"layer {layer}: merged parts need row counts that are multiples of {BLOCK}")
        n_total = sum(p[2] for p in parts)
        weight = torch.empty((n_total, k), dtype=torch.float8_e4m3fn, device=device)
        scales = torch.empty((_cdiv(n_total, BLOCK), _cdiv(k, BLOCK)), dtype=torch.float32, device=device)
        row = 0
        for w_name, s_name, n, _ in parts:
            self._copy_into(w_name, weight[row:row + n])
            self._copy_into(s_name, scales[row // BLOCK:(row + n + BLOCK - 1) // BLOCK])  # widened to fp32
            row += n
        return weight, scales

    def layer_weights(self, layer: int, device: Any = "cpu",
                      projections: dict[str, tuple[str, ...]] | None = None
                      ) -> dict[str, tuple[torch.Tensor, torch.Tensor]]:
        """The reference's ``load_layer_weights``: ``{"qkv", "o", "gate_up", "down"}`` ->
        ``(weight, fp32 scales)`` with q/k/v and gate/up merged."""

        return {name: self.projection(layer, modules, device)
                for name, modules in (projections or PROJECTIONS).items()}


_DTYPES = {
    "F8_E4M3": torch.float8_e4m3fn,
    "F16": torch.float16,
    "BF16": torch.bfloat16,
    "F32": torch.float32,
}


def load_layer_weights(path: str, layer: int, device: Any = "cuda") -> dict[str, tuple[torch.Tensor, torch.Tensor]]:
    """One decoder layer's merged FP8 projections (run_kernel_track.py:192-207)."""

    return FP8Checkpoint(path).layer_weights(layer, device)
