"""GPU parity at the benchmark configurations that the other files do not run end to end.

* Config 1: the merged q/k/v projection at M = 16 tokens (K = 2560, N = 4096 + 1024 + 1024),
  N(0, 1) activations, N(0, 0.02) block-quantized weights: codes and scales bit-exact,
  GEMM output within REL_TOL of the oracle, on every path and through project_qkv.
* Config 5: the continuous-batching step, M = 512 + 24 = 536 rows with outlier channels,
  all four Qwen3-4B projections against the oracle, plus a two-layer slice of the stack
  chained through the fused ops (RMSNorm+quant -> qkv, q columns -> o_proj,
  residual+RMSNorm+quant -> gate_up, SiLU*up+quant -> down), each stage checked against
  the oracle applied to the same stage inputs.
"""

import sys

import numpy as np
import pytest
import torch

import oracle
from _helpers import assert_close_rows, bits16, record_parity, codes, oracle_gemm, oracle_linear, oracle_quant
from minillm_amd import merged_projections as mp
from minillm_amd import mi355x_fp8 as fp8
from minillm_amd.validation import (
    QWEN3_4B_PROJECTIONS, SEED, ModelShape, bit_mismatch_details, bitwise_equal, make_baseline_activations,
    make_baseline_weights,
)

pytestmark = pytest.mark.gpu
BLOCK = [128, 128]
PROJ = {p.name: p for p in QWEN3_4B_PROJECTIONS}


def _note(*parts):
    print("CASE", *parts, flush=True, file=sys.stderr)


def _bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)


@pytest.mark.parametrize("path", ["auto", "fused", "split"])
def test_config1_merged_qkv_m16(gpu, path):
    _note("config1", path)
    shape = PROJ["qkv"]
    x = make_baseline_activations(16, shape.k, SEED)
    w, ws = make_baseline_weights(shape, SEED)
    xg, wg, wsg = x.to(gpu), w.to(gpu), ws.to(gpu)
    q, s = fp8.quantize_mi355x_fp8_activation(xg)
    q_ref, s_ref = oracle_quant(x)
    assert bitwise_equal(q.cpu(), q_ref), bit_mismatch_details(q.cpu(), q_ref)
    assert bitwise_equal(s.cpu(), s_ref), bit_mismatch_details(s.cpu(), s_ref)
    out = fp8.mi355x_fp8_linear(xg, wg, wsg, BLOCK, path=path)
    assert out.shape == (16, 6144) and out.dtype == torch.bfloat16
    record_parity(f"config1 qkv m16 {path}", assert_close_rows(out, oracle_linear(x, w, ws)))
    # The GEMM entry on the oracle's own codes and scales: same tolerance.
    gemm = torch.empty_like(out)
    fp8.launch_block_gemm(q_ref.to(gpu), wg, gemm, s_ref.to(gpu), wsg)
    assert bitwise_equal(gemm, out), bit_mismatch_details(gemm, out)


def test_config1_through_project_qkv(gpu):
    """The engine's call: three separate FP8 projections merged into one GEMM (N-concatenated
    weights and scales); each column view equals its own projection's linear bit for bit and
    the oracle within tolerance."""

    _note("config1 project_qkv")

    class Proj(torch.nn.Module):
        def __init__(self, w, s):
            super().__init__()
            self.weight = torch.nn.Parameter(w, requires_grad=False)
            self.register_buffer("weight_scale_inv", s)
            self.block_size = (128, 128)
            self.bias = None
            self.activation_scale = None

        def forward(self, x):
            return fp8.mi355x_fp8_linear(x, self.weight, self.weight_scale_inv, list(self.block_size))

    shape = PROJ["qkv"]
    w, ws = make_baseline_weights(shape, SEED)
    attn = torch.nn.Module()
    attn.q_proj = Proj(w[:4096].to(gpu), ws[:32].to(gpu))
    attn.k_proj = Proj(w[4096:5120].to(gpu), ws[32:40].to(gpu))
    attn.v_proj = Proj(w[5120:].to(gpu), ws[40:].to(gpu))
    x = make_baseline_activations(16, shape.k, SEED)
    separate = [attn.q_proj(x.to(gpu)), attn.k_proj(x.to(gpu)), attn.v_proj(x.to(gpu))]
    assert mp.install_merged_projections(attn) == 1
    merged = mp.project_qkv(attn, x.to(gpu))
    assert [t.shape[-1] for t in merged] == [4096, 1024, 1024]
    for got, ref in zip(merged, separate):
        assert bitwise_equal(got.contiguous(), ref), bit_mismatch_details(got.contiguous(), ref)
    assert_close_rows(torch.cat([t.cpu() for t in merged], dim=-1), oracle_linear(x, w, ws))


@pytest.mark.parametrize("proj", [p.name for p in QWEN3_4B_PROJECTIONS])
def test_config5_projection_m536(gpu, proj):
    """Each projection of the stack step at 536 rows with outlier channels: codes and scales
    bit-exact, every row within tolerance of the oracle."""

    _note("config5", proj)
    shape = PROJ[proj]
    m = 536
    x = make_baseline_activations(m, shape.k, SEED + 5, outliers=True)
    w, ws = make_baseline_weights(shape, SEED + 5)
    xg, wg, wsg = x.to(gpu), w.to(gpu), ws.to(gpu)
    q, s = fp8.quantize_mi355x_fp8_activation(xg)
    q_ref, s_ref = oracle_quant(x)
    assert bitwise_equal(q.cpu(), q_ref) and bitwise_equal(s.cpu(), s_ref)
    out = fp8.mi355x_fp8_linear(xg, wg, wsg, BLOCK)
    record_parity(f"config5 {proj} m536", assert_close_rows(out, oracle_gemm(q_ref, s_ref, w, ws)))


def test_config5_two_layer_chain(gpu):
    """Two layers of the stack step chained through the fused producers.  Each stage is held
    to the oracle on the GPU's own stage input: RMSNorm output, residual sum, codes and
    scales bit-exact; GEMM outputs within REL_TOL; SiLU*up within one bf16 ulp and its
    codes bit-exact on the kernel's own product."""

    m, hidden, inter = 536, 2560, 9728
    eps = 1e-6
    gen = torch.Generator().manual_seed(SEED + 55)
    h = make_baseline_activations(m, hidden, SEED + 55, outliers=True)
    residual = torch.zeros(m, hidden, dtype=torch.bfloat16)
    hg, rg = h.to(gpu), residual.to(gpu)
    for layer in range(2):
        _note("config5 chain layer", layer)
        ws_ = {p.name: make_baseline_weights(p, SEED + 7919 * layer + i) for i, p in enumerate(QWEN3_4B_PROJECTIONS)}
        wsg = {k: (w.to(gpu), s.to(gpu)) for k, (w, s) in ws_.items()}
        norm1 = (torch.rand(hidden, generator=gen) + 0.5).to(torch.bfloat16)
        norm2 = (torch.rand(hidden, generator=gen) + 0.5).to(torch.bfloat16)

        # input norm (residual add of the previous layer's output) -> qkv
        y, q, s, summed = fp8.rmsnorm_quant_mi355x_fp8(hg, norm1.to(gpu), eps, rg, scale_layout="row",
                                                       return_intermediate=True)
        y_ref, summed_ref = oracle.rmsnorm(bits16(hg), bits16(norm1), eps, bits16(rg))
        assert np.array_equal(bits16(y), y_ref) and np.array_equal(bits16(summed), summed_ref), layer
        q_ref, s_ref = oracle.act_quant(y_ref)
        assert np.array_equal(codes(q), q_ref) and np.array_equal(s.cpu().numpy(), s_ref), layer
        qkv = torch.empty((m, 6144), dtype=torch.bfloat16, device=gpu)
        fp8.launch_block_gemm(q, wsg["qkv"][0], qkv, s, wsg["qkv"][1])
        w, sc = ws_["qkv"]
        record_parity(f"config5 chain{layer} qkv", assert_close_rows(qkv, _bf16(oracle.block_gemm(q_ref, s_ref, codes(w), sc.numpy()))))

        # attention is outside this path: its stand-in output is the q columns (K = 4096)
        attn = qkv[:, :4096]
        o = fp8.mi355x_fp8_linear(attn, *wsg["o_proj"], BLOCK)
        w, sc = ws_["o_proj"]
        record_parity(f"config5 chain{layer} o_proj",
                      assert_close_rows(o, _bf16(oracle.linear(bits16(attn), codes(w), sc.numpy()))))

        # post-attention norm with the residual -> gate_up -> SiLU*up + requant -> down
        y2, q2, s2, summed2 = fp8.rmsnorm_quant_mi355x_fp8(o, norm2.to(gpu), eps, summed, scale_layout="row",
                                                           return_intermediate=True)
        y2_ref, summed2_ref = oracle.rmsnorm(bits16(o), bits16(norm2), eps, bits16(summed))
        assert np.array_equal(bits16(y2), y2_ref) and np.array_equal(bits16(summed2), summed2_ref), layer
        q2_ref, s2_ref = oracle.act_quant(y2_ref)
        assert np.array_equal(codes(q2), q2_ref) and np.array_equal(s2.cpu().numpy(), s2_ref), layer
        gate_up = torch.empty((m, 2 * inter), dtype=torch.bfloat16, device=gpu)
        fp8.launch_block_gemm(q2, wsg["gate_up"][0], gate_up, s2, wsg["gate_up"][1])
        w, sc = ws_["gate_up"]
        record_parity(f"config5 chain{layer} gate_up",
                      assert_close_rows(gate_up, _bf16(oracle.block_gemm(q2_ref, s2_ref, codes(w), sc.numpy()))))

        hmid, q3, s3 = fp8.silu_mul_quant_mi355x_fp8(gate_up[:, :inter], gate_up[:, inter:], scale_layout="row",
                                                     return_intermediate=True)
        h_ref = oracle.silu_mul(bits16(gate_up[:, :inter]), bits16(gate_up[:, inter:]))
        ulps = np.abs(bits16(hmid).astype(np.int32) - h_ref.astype(np.int32))
        assert ulps.max() <= 1, layer
        q3_ref, s3_ref = oracle.act_quant(bits16(hmid))
        assert np.array_equal(codes(q3), q3_ref) and np.array_equal(s3.cpu().numpy(), s3_ref), layer
        down = torch.empty((m, hidden), dtype=torch.bfloat16, device=gpu)
        fp8.launch_block_gemm(q3, wsg["down"][0], down, s3, wsg["down"][1])
        w, sc = ws_["down"]
        record_parity(f"config5 chain{layer} down",
                      assert_close_rows(down, _bf16(oracle.block_gemm(q3_ref, s3_ref, codes(w), sc.numpy()))))

        hg, rg = down, summed2
    assert torch.isfinite(hg.float()).all()
