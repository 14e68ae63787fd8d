"""Merged FP8 projections: q/k/v as one GEMM, gate/up as one GEMM.

The reference's engine/kernels/merged_projections.py concatenates the q/k/v (N = 4096 +
1024 + 1024 = 6144) and gate/up (N = 2 x 9728 = 19456) weights and their 128x128 block
scales along N, runs one FP8 linear per group and returns column views of its output.  All
split points are multiples of 128, so block scales concatenate without straddling and
every output column keeps its own weight rows, scales and K order: the merged result
equals the separate calls bit for bit (GPU test: tests/test_gpu_extensions.py).

This module mirrors that surface (install / uninstall / project_qkv / project_gate_up /
merged_linears) over duck-typed modules: an "attention" is any module with q_proj, k_proj
and v_proj children, an "MLP" any module with gate_proj and up_proj; each child carries an
e4m3fn ``weight`` [N, K] and fp32 ``weight_scale_inv`` [ceil(N/128), ceil(K/128)] (the
Transformers FP8Linear layout).  The merged call goes through ``fp8_linear`` of this
package.  After merging, the original modules' weights become views of the merged
storage, as in the reference (merged_projections.py:60-80).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import torch

QKV = ("q_proj", "k_proj", "v_proj")
GATE_UP = ("gate_proj", "up_proj")
_ATTRS = {QKV: "_minillm_qkv", GATE_UP: "_minillm_gate_up"}


@dataclass(frozen=True)
class MergedLinear:
    weight: torch.Tensor
    weight_scale_inv: torch.Tensor
    splits: tuple[int, ...]
    block_size: tuple[int, int]


def _mergeable(linears: list[Any]) -> bool:
    """The reference's _mergeable (merged_projections.py:44-57)."""

    first = linears[0]
    block = tuple(getattr(first, "block_size", None) or ())
    if len(block) != 2:
        return False
    for linear in linears:
        weight = getattr(linear, "weight", None)
        scales = getattr(linear, "weight_scale_inv", None)
        if (weight is None or weight.dtype != torch.float8_e4m3fn or not isinstance(scales, torch.Tensor)
                or getattr(linear, "bias", None) is not None or getattr(linear, "activation_scale", None) is not None
                or tuple(linear.block_size) != block or weight.shape[1] != first.weight.shape[1]
                or weight.shape[0] % block[0] or weight.device != first.weight.device):
            return False
    return True


def _replace(linear: Any, name: str, value: torch.Tensor) -> None:
    if name in getattr(linear, "_parameters", {}):
        linear._parameters[name] = torch.nn.Parameter(value, requires_grad=False)
    elif name in getattr(linear, "_buffers", {}):
        linear._buffers[name] = value
    else:
        setattr(linear, name, value)


def _merge(module: Any, names: tuple[str, ...]) -> MergedLinear | None:
    linears = [getattr(module, name, None) for name in names]
    if any(linear is None for linear in linears) or not _mergeable(linears):
        return None
    block = tuple(int(b) for b in linears[0].block_size)
    weight = torch.cat([linear.weight.data for linear in linears])
    scales = torch.cat([linear.weight_scale_inv.data for linear in linears])
    splits, start = [], 0
    for linear in linears:
        rows = int(linear.weight.shape[0])
        _replace(linear, "weight", weight[start:start + rows])
        _replace(linear, "weight_scale_inv", scales[start // block[0]:(start + rows) // block[0]])
        splits.append(rows)
        start += rows
    return MergedLinear(weight, scales, tuple(splits), block)


def _linear(merged: MergedLinear, x: torch.Tensor) -> torch.Tensor:
    from .mi355x_fp8 import mi355x_fp8_linear

    return mi355x_fp8_linear(x, merged.weight, merged.weight_scale_inv, block_size=list(merged.block_size))


def project_qkv(attention: Any, hidden_states: torch.Tensor) -> tuple[torch.Tensor, ...]:
    """``(q_proj(x), k_proj(x), v_proj(x))``; column views of one GEMM when merged."""

    merged = getattr(attention, _ATTRS[QKV], None)
    if merged is None:
        return attention.q_proj(hidden_states), attention.k_proj(hidden_states), attention.v_proj(hidden_states)
    return _linear(merged, hidden_states).split(merged.splits, dim=-1)


def project_gate_up(mlp: Any, x: torch.Tensor) -> tuple[torch.Tensor, ...]:
    """``(gate_proj(x), up_proj(x))``; column views of one GEMM when merged."""

    merged = getattr(mlp, _ATTRS[GATE_UP], None)
    if merged is None:
        return mlp.gate_proj(x), mlp.up_proj(x)
    return _linear(merged, x).split(merged.splits, dim=-1)


def install_merged_projections(model: Any, pretune_tokens: int | None = None) -> int:
    """Merge every attention's q/k/v and every MLP's gate/up; returns the merge count
    (the reference's install_merged_projections, merged_projections.py:113-140)."""

    count = 0
    for module in model.modules():
        for names in (QKV, GATE_UP):
            if not all(isinstance(getattr(module, n, None), torch.nn.Module) for n in names):
                continue
            if getattr(module, _ATTRS[names], None) is not None:
                continue
            merged = _merge(module, names)
            if merged is not None:
                # Plain attribute, not a submodule: state_dict and modules() stay unchanged.
                object.__setattr__(module, _ATTRS[names], merged)
                count += 1
    if count and pretune_tokens:
        from .mi355x_fp8 import pretune_mi355x_fp8_shapes

        dtype = next((p.dtype for p in model.parameters() if p.dtype in {torch.bfloat16, torch.float16}),
                     torch.bfloat16)
        pretune_mi355x_fp8_shapes([(m.weight, m.weight_scale_inv, m.block_size) for m in merged_linears(model)],
                                  dtype, pretune_tokens)
    return count


def uninstall_merged_projections(model: Any) -> None:
    """Go back to separate projection calls (weights stay views; results are identical)."""

    for module in model.modules():
        for attr in _ATTRS.values():
            if attr in module.__dict__:
                object.__delattr__(module, attr)


def merged_linears(model: Any) -> list[MergedLinear]:
    return [module.__dict__[attr] for module in model.modules() for attr in _ATTRS.values()
            if attr in module.__dict__]
