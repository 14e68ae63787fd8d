"""One FP8 GEMM per projection group: q/k/v together, gate/up together.

Call surface of the reference's engine/kernels/merged_projections.py (install /
uninstall / project_qkv / project_gate_up / merged_linears; the callers are the attention
and MLP forwards), implemented here as a registry of *projection groups*:

* A group is a parent module plus the names of its member linears, in output-column
  order: (q_proj, k_proj, v_proj) of an attention, (gate_proj, up_proj) of an MLP.
* Installing a group packs the members' e4m3fn weights [N_i, K] into one [sum N_i, K]
  buffer and their fp32 block scales [N_i/128, K/128] into one [sum N_i/128, K/128]
  buffer, member i at row offset sum_{j<i} N_j.  Every N_i is a multiple of the block
  height, so no scale block straddles two members and each output column keeps its own
  weight row, its own scale row and the same K order.  One linear over the packed weight
  therefore gives each member's columns bit for bit (GPU test:
  tests/test_gpu_extensions.py::test_merged_projections_equal_separate_bitwise).
* The members are then re-pointed at their slices of the packed buffers, so the model
  holds one copy of each weight and unmerged calls keep working.
* The registry is keyed weakly by the parent module and stores nothing on it, so
  ``state_dict()`` and ``modules()`` of the model are unchanged by installing.

A member qualifies when it carries a 2-D e4m3fn ``weight`` and a 2-D fp32
``weight_scale_inv`` of shape (ceil(N/bh), ceil(K/bw)) for its two-entry ``block_size``
(bh, bw), has neither a bias nor a static ``activation_scale``, and shares K, block size
and device with the other members.  ``merge_blocker`` names the first violated condition.
"""

from __future__ import annotations

import weakref
from dataclasses import dataclass
from typing import Any

import torch

# Group kind -> member attribute names, in the column order of the packed output.
GROUP_MEMBERS: dict[str, tuple[str, ...]] = {
    "qkv": ("q_proj", "k_proj", "v_proj"),
    "gate_up": ("gate_proj", "up_proj"),
}


@dataclass(frozen=True)
class MergedLinear:
    """A packed projection group: ``weight`` [sum N_i, K], ``weight_scale_inv``
    [sum N_i / bh, ceil(K / bw)], and each member's output width in ``splits``."""

    weight: torch.Tensor
    weight_scale_inv: torch.Tensor
    splits: tuple[int, ...]
    block_size: tuple[int, int]


# parent module -> {group kind: MergedLinear}
_registry: "weakref.WeakKeyDictionary[Any, dict[str, MergedLinear]]" = weakref.WeakKeyDictionary()


def merge_blocker(members: list[Any]) -> str | None:
    """Why ``members`` cannot share one GEMM, or None when they can."""

    block = tuple(getattr(members[0], "block_size", None) or ())
    if len(block) != 2:
        return "block_size must have two entries"
    bh, bw = (int(b) for b in block)
    k = None
    device = None
    for index, member in enumerate(members):
        weight = getattr(member, "weight", None)
        scales = getattr(member, "weight_scale_inv", None)
        if not isinstance(weight, torch.Tensor) or weight.dtype != torch.float8_e4m3fn or weight.ndim != 2:
            return f"member {index}: weight is not a 2-D e4m3fn tensor"
        if not isinstance(scales, torch.Tensor) or scales.dtype != torch.float32 or scales.ndim != 2:
            return f"member {index}: weight_scale_inv is not a 2-D fp32 tensor"
        if tuple(getattr(member, "block_size", None) or ()) != block:
            return f"member {index}: block_size differs"
        if getattr(member, "bias", None) is not None:
            return f"member {index}: has a bias"
        if getattr(member, "activation_scale", None) is not None:
            return f"member {index}: has a static activation scale"
        n, kk = weight.shape
        if n % bh:
            return f"member {index}: {n} output rows are not whole {bh}-row scale blocks"
        if tuple(scales.shape) != (n // bh, -(-kk // bw)):
            return f"member {index}: scale shape {tuple(scales.shape)} does not match the weight"
        if k is None:
            k, device = kk, weight.device
        elif kk != k or weight.device != device or scales.device != device:
            return f"member {index}: K or device differs"
    return None


def _rebind(module: Any, name: str, value: torch.Tensor) -> None:
    """Point ``module.name`` at ``value``, keeping its kind (parameter, buffer, attribute)."""

    params = getattr(module, "_parameters", {})
    buffers = getattr(module, "_buffers", {})
    if name in params:
        params[name] = torch.nn.Parameter(value, requires_grad=False)
    elif name in buffers:
        buffers[name] = value
    else:
        setattr(module, name, value)


def _pack(members: list[Any]) -> MergedLinear:
    block = tuple(int(b) for b in members[0].block_size)
    weights = [m.weight.detach() for m in members]
    scales = [m.weight_scale_inv.detach() for m in members]
    widths = tuple(int(w.shape[0]) for w in weights)
    k = int(weights[0].shape[1])
    packed_w = torch.empty((sum(widths), k), dtype=weights[0].dtype, device=weights[0].device)
    packed_s = torch.empty((sum(widths) // block[0], scales[0].shape[1]), dtype=torch.float32,
                           device=scales[0].device)
    row = 0
    for member, w, s, width in zip(members, weights, scales, widths):
        w_view = packed_w[row:row + width]
        s_view = packed_s[row // block[0]:(row + width) // block[0]]
        w_view.copy_(w)
        s_view.copy_(s)
        _rebind(member, "weight", w_view)
        _rebind(member, "weight_scale_inv", s_view)
        row += width
    return MergedLinear(packed_w, packed_s, widths, block)


def _run(group: MergedLinear, x: torch.Tensor) -> tuple[torch.Tensor, ...]:
    from .mi355x_fp8 import mi355x_fp8_linear

    out = mi355x_fp8_linear(x, group.weight, group.weight_scale_inv, block_size=list(group.block_size))
    return torch.split(out, group.splits, dim=-1)


def _project(module: Any, kind: str, x: torch.Tensor) -> tuple[torch.Tensor, ...]:
    group = _registry.get(module, {}).get(kind)
    if group is None:
        return tuple(getattr(module, name)(x) for name in GROUP_MEMBERS[kind])
    return _run(group, x)


def project_qkv(attention: Any, hidden_states: torch.Tensor) -> tuple[torch.Tensor, ...]:
    """``(q_proj(x), k_proj(x), v_proj(x))``: column views of one GEMM once merged."""

    return _project(attention, "qkv", hidden_states)


def project_gate_up(mlp: Any, x: torch.Tensor) -> tuple[torch.Tensor, ...]:
    """``(gate_proj(x), up_proj(x))``: column views of one GEMM once merged."""

    return _project(mlp, "gate_up", x)


def install_merged_projections(model: Any, pretune_tokens: int | None = None) -> int:
    """Pack every qualifying q/k/v and gate/up group of ``model``; returns how many groups
    were packed by this call (already packed groups count zero).  With
    ``pretune_tokens``, the packed shapes are warmed as ``pretune_mi355x_fp8`` does."""

    packed = []
    for module in model.modules():
        for kind, names in GROUP_MEMBERS.items():
            members = [getattr(module, name, None) for name in names]
            if not all(isinstance(m, torch.nn.Module) for m in members):
                continue
            if kind in _registry.get(module, {}) or merge_blocker(members) is not None:
                continue
            group = _pack(members)
            _registry.setdefault(module, {})[kind] = group
            packed.append(group)
    if packed and pretune_tokens:
        from .mi355x_fp8 import pretune_mi355x_fp8_shapes

        dtype = next((p.dtype for p in model.parameters() if p.dtype in {torch.bfloat16, torch.float16}),
                     torch.bfloat16)
        pretune_mi355x_fp8_shapes([(g.weight, g.weight_scale_inv, g.block_size) for g in packed], dtype,
                                  pretune_tokens)
    return len(packed)


def uninstall_merged_projections(model: Any) -> None:
    """Return to one call per projection.  The members keep pointing into the packed
    buffers, so their results do not change."""

    for module in model.modules():
        _registry.pop(module, None)


def merged_linears(model: Any) -> list[MergedLinear]:
    """The packed groups of ``model``, in module order (q/k/v before gate/up per module)."""

    return [group for module in model.modules() for kind in GROUP_MEMBERS
            if (group := _registry.get(module, {}).get(kind)) is not None]
