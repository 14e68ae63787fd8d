"""CPU checks of the merged-projection host logic (minillm_amd/merged_projections.py),
mirroring the reference's tests/test_merged_projections.py: q/k/v and gate/up merge into
one weight and one scale matrix along N, the originals become views, outputs split back
into the projections, and uninstall restores separate calls.  The FP8 linear itself is
replaced by the CPU oracle (its GPU path is covered by tests/test_gpu_extensions.py)."""

import numpy as np
import pytest
import torch

import oracle
from _helpers import bits16, codes
from minillm_amd import merged_projections as mp
from minillm_amd import mi355x_fp8 as fp8
from minillm_amd.validation import ModelShape, make_activations, make_weights


class FakeFP8Linear(torch.nn.Module):
    def __init__(self, n, k, seed):
        super().__init__()
        w, s = make_weights(ModelShape("p", n, k), seed)
        self.weight = torch.nn.Parameter(w, requires_grad=False)
        self.register_buffer("weight_scale_inv", s)
        self.block_size = (128, 128)
        self.bias = None
        self.activation_scale = None

    def forward(self, x):
        return oracle_linear(x, self.weight, self.weight_scale_inv)


def oracle_linear(x, w, s, block_size=None):
    out = oracle.linear(bits16(x), codes(w), s.float().numpy())
    return torch.from_numpy(out.view(np.int16)).view(torch.bfloat16)


class Attn(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.q_proj, self.k_proj, self.v_proj = FakeFP8Linear(256, 384, 1), FakeFP8Linear(128, 384, 2), FakeFP8Linear(128, 384, 3)


class MLP(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.gate_proj, self.up_proj = FakeFP8Linear(384, 384, 4), FakeFP8Linear(384, 384, 5)


@pytest.fixture
def model(monkeypatch):
    monkeypatch.setattr(fp8, "mi355x_fp8_linear", lambda x, w, s, block_size=None: oracle_linear(x, w, s))
    m = torch.nn.Module()
    m.attn, m.mlp = Attn(), MLP()
    return m


def test_merge_concatenates_along_n_and_keeps_views(model):
    separate_q = model.attn.q_proj.weight.clone()
    assert mp.install_merged_projections(model) == 2
    merged = mp.merged_linears(model)
    assert [m.splits for m in merged] == [(256, 128, 128), (384, 384)]
    qkv = merged[0]
    assert qkv.weight.shape == (512, 384) and qkv.weight_scale_inv.shape == (4, 3)
    assert model.attn.q_proj.weight.data_ptr() == qkv.weight.data_ptr()
    assert torch.equal(model.attn.q_proj.weight.view(torch.uint8), separate_q.view(torch.uint8))
    assert mp.install_merged_projections(model) == 0  # idempotent
    assert "_minillm_qkv" not in dict(model.attn.named_children())


def test_merged_outputs_equal_separate_calls(model):
    x = make_activations(5, 384, 9)
    separate = (model.attn.q_proj(x), model.attn.k_proj(x), model.attn.v_proj(x))
    gu_separate = (model.mlp.gate_proj(x), model.mlp.up_proj(x))
    mp.install_merged_projections(model)
    for got, ref in zip(mp.project_qkv(model.attn, x), separate):
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    for got, ref in zip(mp.project_gate_up(model.mlp, x), gu_separate):
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    mp.uninstall_merged_projections(model)
    assert mp.merged_linears(model) == []
    for got, ref in zip(mp.project_qkv(model.attn, x), separate):
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_unmergeable_modules_are_left_alone(model):
    model.attn.k_proj.bias = torch.nn.Parameter(torch.zeros(128))
    model.mlp.up_proj.block_size = (128, 64)
    assert mp.install_merged_projections(model) == 0
