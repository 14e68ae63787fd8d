"""Golden fixtures (tests/golden/fp8_linear_golden.npz, written by make_golden.py): the
oracle still reproduces them bit for bit, and on the GPU the HIP path matches them
(codes and scales bit-exact, outputs within the row tolerance)."""

import os

import numpy as np
import pytest
import torch

import oracle
from _helpers import assert_close_rows

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fp8_linear_golden.npz")
CASES = ("tail_259", "tail_129_fp16", "kv_slice")


def load(name):
    data = np.load(FIXTURE)  # allow_pickle=False by default
    return {k.split("/", 1)[1]: data[k] for k in data.files if k.startswith(name + "/")}


@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_golden(name):
    c = load(name)
    q, s = oracle.act_quant(c["x"], is_fp16=bool(c["fp16"]))
    assert np.array_equal(q, c["q"]) and np.array_equal(s.view(np.uint32), c["s"].view(np.uint32))
    out = oracle.block_gemm(q, s, c["w"], c["ws"], out_fp16=bool(c["fp16"]))
    assert np.array_equal(out, c["out"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_hip_matches_golden(gpu, name):
    from minillm_amd import mi355x_fp8 as fp8

    c = load(name)
    dtype = torch.float16 if bool(c["fp16"]) else torch.bfloat16
    x = torch.from_numpy(c["x"].view(np.int16)).view(dtype).to(gpu)
    w = torch.from_numpy(c["w"]).view(torch.float8_e4m3fn).to(gpu)
    ws = torch.from_numpy(c["ws"]).to(gpu)
    q, s = fp8.quantize_mi355x_fp8_activation(x)
    assert np.array_equal(q.cpu().view(torch.uint8).numpy(), c["q"])
    assert np.array_equal(s.cpu().numpy().view(np.uint32), c["s"].view(np.uint32))
    out = fp8.mi355x_fp8_linear(x, w, ws, [128, 128])
    expected = torch.from_numpy(c["out"].view(np.int16)).view(dtype)
    assert_close_rows(out, expected)
