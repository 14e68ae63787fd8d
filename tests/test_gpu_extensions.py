"""GPU checks of the rows next to the linear: the fused SiLU-mul + requant kernel, the MLP
block built on it (baseline config 4) and merged projections (bitwise equal to separate
calls, as the reference's tests/test_merged_projections.py:42-56 requires)."""

import sys

import numpy as np
import pytest
import torch

import oracle
from _helpers import assert_close_rows, record_parity, bits16, codes, crafted_sumsq_rows, oracle_linear, sumsq_eps_sweep
from minillm_amd import _lib
from minillm_amd import merged_projections as mp
from minillm_amd import mi355x_fp8 as fp8
from minillm_amd.validation import (
    SEED, ModelShape, bit_mismatch_details, bitwise_equal, make_activations, make_baseline_activations,
    make_baseline_weights, make_weights,
)

pytestmark = pytest.mark.gpu


def _note(*parts):
    print("CASE", *parts, flush=True, file=sys.stderr)


def _bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


@pytest.mark.parametrize("rows,inter", [(1, 9728), (7, 259), (64, 1024), (300, 9728)])
def test_silu_mul_quant_matches_oracle(gpu, rows, inter):
    """h within one bf16 ulp of the oracle (exp may differ in the last place), and the
    codes/scales bit-exact against the oracle's quantizer applied to the kernel's own h."""

    _note("silu_mul_quant", rows, inter)
    gen = torch.Generator().manual_seed(rows * 7 + inter)
    gate_up = (torch.randn(rows, 2 * inter, generator=gen) * 3).to(torch.bfloat16)
    gate_up[0, :8] = torch.tensor([0.0, -0.0, 30.0, -30.0, 88.0, -100.0, 1e-3, 5.0]).to(torch.bfloat16)
    g, u = gate_up[:, :inter], gate_up[:, inter:]
    dev = gate_up.to(gpu)
    h, q, s = fp8.silu_mul_quant_mi355x_fp8(dev[:, :inter], dev[:, inter:], scale_layout="row",
                                           return_intermediate=True)
    ref_h = oracle.silu_mul(bits16(g.contiguous()), bits16(u.contiguous()))
    got_h = bits16(h)
    ulps = np.abs(got_h.astype(np.int32) - ref_h.astype(np.int32))
    assert ulps.max() <= 1 and (ulps == 0).mean() > 0.999
    q_ref, s_ref = oracle.act_quant(got_h)
    assert np.array_equal(codes(q), q_ref)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    # K-group-major scales: same values.
    q2, s2 = fp8.silu_mul_quant_mi355x_fp8(dev[:, :inter], dev[:, inter:])
    assert bitwise_equal(q2, q) and bitwise_equal(s2.contiguous(), s)


def test_silu_mul_quant_rejects_fp16(gpu):
    x = torch.zeros(2, 256, dtype=torch.float16, device=gpu)
    with pytest.raises(ValueError, match="bf16"):
        fp8.silu_mul_quant_mi355x_fp8(x, x)


@pytest.mark.parametrize("rows", [8, 512])
def test_mlp_block_config4(gpu, rows):
    """Baseline config 4 at M in {8, 512}: x -> gate_up -> SiLU*up -> requant -> down, against
    the oracle run on the same chain (its quantizer applied to the GPU's bf16 product)."""

    _note("mlp", rows)
    gu_shape, down_shape = ModelShape("gate_up", 19456, 2560), ModelShape("down", 2560, 9728)
    x = make_baseline_activations(rows, 2560, SEED, outliers=True)
    wgu, sgu = make_baseline_weights(gu_shape, SEED)
    wd, sd = make_baseline_weights(down_shape, SEED + 1)
    xg = x.to(gpu)
    out = fp8.mlp_forward_mi355x_fp8(xg, wgu.to(gpu), sgu.to(gpu), wd.to(gpu), sd.to(gpu))
    # Reference chain on the oracle, stage by stage, each against the GPU's intermediate.
    gate_up = fp8.mi355x_fp8_linear(xg, wgu.to(gpu), sgu.to(gpu), [128, 128])
    record_parity(f"config4 gate_up m{rows}", assert_close_rows(gate_up, oracle_linear(x, wgu, sgu)))
    h, q, s = fp8.silu_mul_quant_mi355x_fp8(gate_up[:, :9728], gate_up[:, 9728:], return_intermediate=True)
    q_ref, s_ref = oracle.act_quant(bits16(h))
    assert np.array_equal(codes(q), q_ref)
    down_ref = oracle.block_gemm(q_ref, s_ref, codes(wd), sd.numpy())
    record_parity(f"config4 down m{rows}", assert_close_rows(out, _bf16(down_ref)))


@pytest.mark.parametrize("rows", [1, 8, 100, 300, 2048])
def test_merged_projections_equal_separate_bitwise(gpu, rows):
    _note("merged", rows)

    class Lin(torch.nn.Module):
        def __init__(self, n, k, seed):
            super().__init__()
            w, s = make_weights(ModelShape("p", n, k), seed)
            self.weight = torch.nn.Parameter(w.to(gpu), requires_grad=False)
            self.register_buffer("weight_scale_inv", s.to(gpu))
            self.block_size = (128, 128)
            self.bias = None
            self.activation_scale = None

        def forward(self, x):
            return fp8.mi355x_fp8_linear(x, self.weight, self.weight_scale_inv, list(self.block_size))

    attn = torch.nn.Module()
    attn.q_proj, attn.k_proj, attn.v_proj = Lin(4096, 2560, 1), Lin(1024, 2560, 2), Lin(1024, 2560, 3)
    mlp = torch.nn.Module()
    mlp.gate_proj, mlp.up_proj = Lin(9728, 2560, 4), Lin(9728, 2560, 5)
    model = torch.nn.Module()
    model.attn, model.mlp = attn, mlp
    x = make_activations(rows, 2560, SEED).to(gpu)
    separate = [attn.q_proj(x), attn.k_proj(x), attn.v_proj(x), mlp.gate_proj(x), mlp.up_proj(x)]
    assert mp.install_merged_projections(model) == 2
    merged = list(mp.project_qkv(attn, x)) + list(mp.project_gate_up(mlp, x))
    for got, ref in zip(merged, separate):
        assert bitwise_equal(got.contiguous(), ref), rows


def test_checkpoint_loader_feeds_the_linear(gpu, tmp_path):
    """Weights loaded from a safetensors checkpoint straight into HBM run through the
    linear: merged q/k/v against the oracle, and its column ranges bitwise equal to the
    separately loaded projections."""

    from safetensors.torch import save_file

    from minillm_amd import checkpoint as ckpt

    gen = torch.Generator().manual_seed(11)
    tensors = {}
    for module, n in (("self_attn.q_proj", 512), ("self_attn.k_proj", 128), ("self_attn.v_proj", 128)):
        w, s = make_weights(ModelShape(module, n, 384), 11 + n)
        tensors[f"model.layers.0.{module}.weight"] = w
        tensors[f"model.layers.0.{module}.weight_scale_inv"] = s.to(torch.float16)
    save_file(tensors, str(tmp_path / "model.safetensors"))
    ck = ckpt.FP8Checkpoint(str(tmp_path))
    w, s = ck.projection(0, ckpt.PROJECTIONS["qkv"], device=gpu)
    assert w.is_cuda and s.dtype == torch.float32
    x = make_activations(40, 384, 7)
    out = fp8.mi355x_fp8_linear(x.to(gpu), w, s, [128, 128])
    assert_close_rows(out, oracle_linear(x, w.cpu(), s.cpu()))
    row = 0
    for module in ckpt.PROJECTIONS["qkv"]:
        wp, sp = ck.projection(0, (module,), device=gpu)
        part = fp8.mi355x_fp8_linear(x.to(gpu), wp, sp, [128, 128])
        assert bitwise_equal(part, out[:, row:row + wp.shape[0]].contiguous())
        row += wp.shape[0]


@pytest.mark.parametrize("rows,width", [(1, 2560), (2, 2560), (4, 2560), (8, 2560), (16, 2560), (300, 2560),
                                        (3, 260), (64, 128), (5, 4096), (3, 16000), (1, 128), (256, 2560),
                                        (257, 2560), (513, 2560), (200, 16000)])
@pytest.mark.parametrize("with_residual", [False, True])
def test_rmsnorm_quant_matches_oracle(gpu, rows, width, with_residual):
    """The fused RMSNorm + quantizer against the oracle: y and the residual sum bitwise (same
    summation order, same correctly rounded 1/sqrt), codes and scales bit-exact."""

    _note("rmsnorm_quant", rows, width, with_residual)
    gen = torch.Generator().manual_seed(rows * 31 + width)
    x = (torch.randn(rows, width, generator=gen) * 2).to(torch.bfloat16)
    x[0, :4] = torch.tensor([0.0, -0.0, 200.0, -3.0e-3]).to(torch.bfloat16)
    r = torch.randn(rows, width, generator=gen).to(torch.bfloat16) if with_residual else None
    w = (torch.rand(width, generator=gen) + 0.5).to(torch.bfloat16)
    outs = fp8.rmsnorm_quant_mi355x_fp8(x.to(gpu), w.to(gpu), 1e-6, None if r is None else r.to(gpu),
                                        scale_layout="row", return_intermediate=True)
    y, q, s = outs[0], outs[1], outs[2]
    y_ref, summed_ref = oracle.rmsnorm(bits16(x), bits16(w), 1e-6, None if r is None else bits16(r))
    assert np.array_equal(bits16(y), y_ref)
    if with_residual:
        assert np.array_equal(bits16(outs[3]), summed_ref)
    q_ref, s_ref = oracle.act_quant(y_ref)
    assert np.array_equal(codes(q), q_ref)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    # K-group-major scales: same values.
    outs2 = fp8.rmsnorm_quant_mi355x_fp8(x.to(gpu), w.to(gpu), 1e-6, None if r is None else r.to(gpu))
    assert bitwise_equal(outs2[0], q)
    assert np.array_equal(outs2[1].cpu().numpy().view(np.uint32), s.cpu().numpy().view(np.uint32))


@pytest.mark.parametrize("rows,width", [(1, 2560), (2, 2560), (16, 2560), (3, 1024), (1, 128)])
def test_rmsnorm_summation_order_on_crafted_rows(gpu, rows, width):
    """The kernel's row sum follows the reference's order (fused.py:61-75, 95-115): on rows
    whose fp32 sum of squares that order fixes in closed form, and other orders change
    (_helpers.crafted_sumsq_rows), over an eps sweep at which those sums give different y
    (_helpers.sumsq_eps_sweep), y equals the oracle's bit for bit, and its 4096 element
    equals the value the closed-form sum gives."""

    _note("rmsnorm order", rows, width)
    bw = oracle.rmsnorm_block_width(rows, width)
    w = torch.ones(width, dtype=torch.bfloat16)
    for name, x, expect in crafted_sumsq_rows(rows, width, bw):
        xg = x.to(gpu)
        for eps in sumsq_eps_sweep(width, expect, name):
            y = fp8.rmsnorm_quant_mi355x_fp8(xg, w.to(gpu), eps, scale_layout="row", return_intermediate=True)[0]
            y_ref, _ = oracle.rmsnorm(bits16(x), bits16(w), eps)
            got = bits16(y)
            assert np.array_equal(got, y_ref), (name, eps)
            var = np.float32(np.float32(expect) * np.float32(np.float32(1.0) / np.float32(width)))
            inv = np.float32(1.0 / np.sqrt(np.float64(np.float32(var + np.float32(eps)))))
            y0 = torch.tensor(float(np.float32(np.float32(4096.0) * inv))).to(torch.bfloat16)
            assert int(got[0, 0]) == int(bits16(y0.reshape(1))[0]), (name, eps)


@pytest.mark.parametrize("rows,width", [(1, 2560), (2, 2560), (8, 2560), (3, 1024), (4, 1536), (1, 256)])
def test_rmsnorm_linear_one_launch_summation_order(gpu, rows, width):
    """The one-launch norm-linear's row sum (its own cross-lane tree) in the reference's
    order: on the crafted rows whose sum of squares only that order gives, over the eps
    sweep at which other sums change y (hence the group's scale, hence every output of the
    row), its output equals the two launches' bit for bit (the two-launch norm is pinned to
    the closed-form sums by test_rmsnorm_summation_order_on_crafted_rows)."""

    _note("rmsnorm linear order", rows, width)
    bw = oracle.rmsnorm_block_width(rows, width)
    shape = ModelShape("c", 256, width)
    w, ws = make_weights(shape, 17)
    wg, wsg = w.to(gpu), ws.to(gpu)
    nw = torch.ones(width, dtype=torch.bfloat16, device=gpu)
    lib = _lib.load()
    stream = torch.cuda.current_stream(gpu).cuda_stream
    for name, x, expect in crafted_sumsq_rows(rows, width, bw):
        xg = x.to(gpu)
        for eps in sumsq_eps_sweep(width, expect, name):
            direct = torch.empty((rows, shape.n), dtype=torch.bfloat16, device=gpu)
            code = lib.mi355x_fp8_rmsnorm_linear(xg.data_ptr(), rows, width, xg.stride(0), None, 0, None, width,
                                                 nw.data_ptr(), eps, wg.data_ptr(), wg.stride(0), wsg.data_ptr(),
                                                 wsg.stride(0), wsg.stride(1), shape.n, direct.data_ptr(),
                                                 direct.stride(0), stream)
            assert code == 0, (name, eps, code)
            q, sc = fp8.rmsnorm_quant_mi355x_fp8(xg, nw, eps, scale_layout="row")[:2]
            ref = torch.empty_like(direct)
            fp8.launch_block_gemm(q, wg, ref, sc, wsg)
            assert bitwise_equal(direct, ref), (name, eps, bit_mismatch_details(direct, ref))


def test_rmsnorm_linear_equals_unfused(gpu):
    """Norm + quantizer fused in front of the GEMM gives the same bits as the linear on the
    normalized activations (one quantizer, one GEMM arithmetic)."""

    gen = torch.Generator().manual_seed(3)
    x = torch.randn(40, 2560, generator=gen).to(torch.bfloat16).to(gpu)
    r = torch.randn(40, 2560, generator=gen).to(torch.bfloat16).to(gpu)
    nw = (torch.rand(2560, generator=gen) + 0.5).to(torch.bfloat16).to(gpu)
    w, ws = make_baseline_weights(ModelShape("qkv", 6144, 2560), SEED)
    wg, wsg = w.to(gpu), ws.to(gpu)
    out, summed = fp8.rmsnorm_linear_mi355x_fp8(x, nw, 1e-6, wg, wsg, residual=r)
    y, _, _, summed2 = fp8.rmsnorm_quant_mi355x_fp8(x, nw, 1e-6, r, return_intermediate=True)
    assert bitwise_equal(summed, summed2)
    assert bitwise_equal(out, fp8.mi355x_fp8_linear(y, wg, wsg, [128, 128]))
    assert_close_rows(out, oracle_linear(y.cpu(), w, ws))


@pytest.mark.parametrize("shape", [ModelShape("qkv", 6144, 2560), ModelShape("gate_up", 19456, 2560),
                                   ModelShape("k256", 1024, 256), ModelShape("k1024", 2560, 1024)],
                         ids=lambda s: s.name)
@pytest.mark.parametrize("rows", [1, 2, 3, 4, 5, 7, 8, 9])
@pytest.mark.parametrize("with_residual", [False, True])
def test_rmsnorm_linear_one_launch_equals_two(gpu, shape, rows, with_residual):
    """Up to 8 rows the norm, the quantizer and the GEMM run as one launch (the decode kernel
    recomputing each row's norm in the reference's order); its output and residual sum equal,
    bit for bit, rmsnorm_quant followed by the GEMM on its codes and scales.  Rows carry
    zeros, a huge value and -0.0; 9 rows take the two launches."""

    _note("rmsnorm linear", shape.name, rows, with_residual)
    gen = torch.Generator().manual_seed(rows * 7 + shape.k)
    x = (torch.randn(rows, shape.k, generator=gen) * 2).to(torch.bfloat16)
    x[0, :3] = torch.tensor([0.0, -0.0, 3000.0]).to(torch.bfloat16)
    if rows > 1:
        x[1] = 0.0
    r = torch.randn(rows, shape.k, generator=gen).to(torch.bfloat16) if with_residual else None
    nw = (torch.rand(shape.k, generator=gen) + 0.5).to(torch.bfloat16)
    w, ws = make_weights(shape, 11)
    xg, nwg, wg, wsg = x.to(gpu), nw.to(gpu), w.to(gpu), ws.to(gpu)
    rg = None if r is None else r.to(gpu)
    got = fp8.rmsnorm_linear_mi355x_fp8(xg, nwg, 1e-6, wg, wsg, residual=rg)
    outs = fp8.rmsnorm_quant_mi355x_fp8(xg, nwg, 1e-6, rg, scale_layout="row")
    ref = torch.empty((rows, shape.n), dtype=torch.bfloat16, device=gpu)
    fp8.launch_block_gemm(outs[0], wg, ref, outs[1], wsg)
    if with_residual:
        assert bitwise_equal(got[0], ref), bit_mismatch_details(got[0], ref)
        assert bitwise_equal(got[1], outs[2])
    else:
        assert bitwise_equal(got, ref), bit_mismatch_details(got, ref)
    if rows <= 8:
        # The one-launch entry point itself (the wrapper above falls back to two launches
        # where the entry point answers unsupported): it must take these shapes.
        direct = torch.empty((rows, shape.n), dtype=torch.bfloat16, device=gpu)
        summed = torch.empty((rows, shape.k), dtype=torch.bfloat16, device=gpu) if with_residual else None
        code = _lib.load().mi355x_fp8_rmsnorm_linear(
            xg.data_ptr(), rows, shape.k, xg.stride(0), None if rg is None else rg.data_ptr(),
            0 if rg is None else rg.stride(0), None if summed is None else summed.data_ptr(), shape.k,
            nwg.data_ptr(), 1e-6, wg.data_ptr(), wg.stride(0), wsg.data_ptr(), wsg.stride(0), wsg.stride(1),
            shape.n, direct.data_ptr(), direct.stride(0), torch.cuda.current_stream(gpu).cuda_stream)
        assert code == 0, f"one-launch entry point returned {code}"
        torch.cuda.synchronize(gpu)
        assert bitwise_equal(direct, ref), bit_mismatch_details(direct, ref)
        if with_residual:
            assert bitwise_equal(summed, outs[2])
    # A column view with a padded row stride: the same bits.
    pad = torch.zeros(rows, shape.k + 64, dtype=torch.bfloat16, device=gpu)
    pad[:, : shape.k] = xg
    got2 = fp8.rmsnorm_linear_mi355x_fp8(pad[:, : shape.k], nwg, 1e-6, wg, wsg, residual=rg)
    assert bitwise_equal(got2[0] if with_residual else got2, ref)


def test_rmsnorm_quant_strided_rows(gpu):
    """Rows with a padded stride (not a multiple of 8 elements: the unvectorized path) give
    the same bits as contiguous rows."""

    gen = torch.Generator().manual_seed(9)
    base = torch.randn(6, 2563, generator=gen).to(torch.bfloat16).to(gpu)
    x = base[:, :2560]
    w = (torch.rand(2560, generator=gen) + 0.5).to(torch.bfloat16).to(gpu)
    got = fp8.rmsnorm_quant_mi355x_fp8(x, w, 1e-6, return_intermediate=True)
    ref = fp8.rmsnorm_quant_mi355x_fp8(x.contiguous(), w, 1e-6, return_intermediate=True)
    assert bitwise_equal(got[0], ref[0]) and bitwise_equal(got[1], ref[1])


def test_rmsnorm_quant_rejects(gpu):
    w = torch.ones(256, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(RuntimeError, match="unsupported"):
        fp8.rmsnorm_quant_mi355x_fp8(torch.zeros(1, 16132, dtype=torch.bfloat16, device=gpu),
                                     torch.ones(16132, dtype=torch.bfloat16, device=gpu), 1e-6)
    with pytest.raises(ValueError, match="bf16"):
        fp8.rmsnorm_quant_mi355x_fp8(torch.zeros(2, 256, dtype=torch.float16, device=gpu), w, 1e-6)
    with pytest.raises(ValueError, match="multiple of 4"):
        fp8.rmsnorm_quant_mi355x_fp8(torch.zeros(2, 130, dtype=torch.bfloat16, device=gpu), w[:130], 1e-6)
    with pytest.raises(ValueError, match="multiple of 4"):
        fp8.rmsnorm_quant_mi355x_fp8(torch.zeros(2, 124, dtype=torch.bfloat16, device=gpu), w[:124], 1e-6)


def test_hip_graph_replays_match_eager(gpu):
    """The ops under HIP-graph capture (the workspace warmed first, as pretune does): decode
    and prefill linears, the fused SiLU·mul quantizer and the fused RMSNorm quantizer,
    replayed three times with new inputs copied in eagerly between replays, every replay
    bitwise equal to the eager calls on the same inputs."""

    shape = ModelShape("kv", 1024, 2560)
    w, ws = make_baseline_weights(shape, SEED)
    wg, wsg = w.to(gpu), ws.to(gpu)
    x_dec = torch.empty(8, 2560, dtype=torch.bfloat16, device=gpu)
    x_pre = torch.empty(300, 2560, dtype=torch.bfloat16, device=gpu)
    gate = torch.empty(40, 1024, dtype=torch.bfloat16, device=gpu)
    up = torch.empty_like(gate)
    xn = torch.empty(24, 2560, dtype=torch.bfloat16, device=gpu)
    res = torch.empty_like(xn)
    nw = (torch.rand(2560, generator=torch.Generator().manual_seed(1)) + 0.5).to(torch.bfloat16).to(gpu)

    def fill(seed):
        gen = torch.Generator().manual_seed(seed)
        for t in (x_dec, x_pre, gate, up, xn, res):
            t.copy_((torch.randn(t.shape, generator=gen) * 3).to(torch.bfloat16))

    def run():
        return (fp8.mi355x_fp8_linear(x_dec, wg, wsg, [128, 128]), fp8.mi355x_fp8_linear(x_pre, wg, wsg, [128, 128]),
                *fp8.silu_mul_quant_mi355x_fp8(gate, up), *fp8.rmsnorm_quant_mi355x_fp8(xn, nw, 1e-6, res))

    stream = torch.cuda.Stream()
    fill(0)
    with torch.cuda.stream(stream):
        run()  # sizes this stream's workspace, so the capture allocates nothing of ours
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            captured = run()
    for replay in range(3):
        fill(100 + replay)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
        stream.synchronize()
        eager = run()
        torch.cuda.synchronize()
        for got, want in zip(captured, eager):
            assert bitwise_equal(got, want), (replay, bit_mismatch_details(got, want))


@pytest.mark.parametrize("shape", [ModelShape("gate_up", 19456, 2560), ModelShape("gate_up_small", 1024, 1024),
                                   ModelShape("gate_up_ragged", 2 * 1408, 2560), ModelShape("gate_up_odd", 2 * 259, 256),
                                   ModelShape("gate_up_tiny", 2 * 16, 512)], ids=lambda s: s.name)
@pytest.mark.parametrize("rows", [1, 2, 3, 4, 5, 8, 9])
@pytest.mark.parametrize("with_residual", [False, True])
def test_rmsnorm_gate_up_silu_one_launch_equals_separate(gpu, shape, rows, with_residual):
    """Up to 8 rows the post-attention norm, the merged gate/up GEMM and SiLU(gate) * up run as
    one launch (each workgroup owning matching gate and up rows); h and the residual sum equal,
    bit for bit, the norm-linear's gate_up output followed by the SiLU*up kernel's h.  The
    widths cover the Qwen3-4B intermediate (three 16-row tiles per half, 38 rows per CU), a
    narrow one (one tile) and one whose halves end inside a 128-row weight-scale block; 9 rows
    take the separate launches.  h is also held to the oracle chain (rms_norm, linear,
    silu_mul on its bf16 outputs)."""

    _note("rmsnorm gate_up silu", shape.name, rows, with_residual)
    gen = torch.Generator().manual_seed(rows * 13 + shape.n)
    x = (torch.randn(rows, shape.k, generator=gen) * 2).to(torch.bfloat16)
    x[0, :3] = torch.tensor([0.0, -0.0, 3000.0]).to(torch.bfloat16)
    r = torch.randn(rows, shape.k, generator=gen).to(torch.bfloat16) if with_residual else None
    nw = (torch.rand(shape.k, generator=gen) + 0.5).to(torch.bfloat16)
    w, ws = make_weights(shape, 17)
    xg, nwg, wg, wsg = x.to(gpu), nw.to(gpu), w.to(gpu), ws.to(gpu)
    rg = None if r is None else r.to(gpu)
    inter = shape.n // 2
    got = fp8.rmsnorm_gate_up_silu_mi355x_fp8(xg, nwg, 1e-6, wg, wsg, residual=rg)
    lin = fp8.rmsnorm_linear_mi355x_fp8(xg, nwg, 1e-6, wg, wsg, residual=rg)
    gu = lin[0] if with_residual else lin
    h_ref = fp8.silu_mul_quant_mi355x_fp8(gu[:, :inter], gu[:, inter:], return_intermediate=True)[0]
    h = got[0] if with_residual else got
    assert h.shape == (rows, inter) and h.dtype == torch.bfloat16
    assert bitwise_equal(h, h_ref), bit_mismatch_details(h, h_ref)
    if with_residual:
        assert bitwise_equal(got[1], lin[1])
    if rows <= 8:
        # The one-launch entry point itself must take these shapes.
        direct = torch.full((rows, inter), float("nan"), dtype=torch.bfloat16, device=gpu)
        summed = torch.empty((rows, shape.k), dtype=torch.bfloat16, device=gpu) if with_residual else None
        code = _lib.load().mi355x_fp8_rmsnorm_gate_up_silu(
            xg.data_ptr(), rows, shape.k, xg.stride(0), None if rg is None else rg.data_ptr(),
            0 if rg is None else rg.stride(0), None if summed is None else summed.data_ptr(), shape.k,
            nwg.data_ptr(), 1e-6, wg.data_ptr(), wg.stride(0), wsg.data_ptr(), wsg.stride(0), wsg.stride(1),
            shape.n, direct.data_ptr(), direct.stride(0), torch.cuda.current_stream(gpu).cuda_stream)
        assert code == 0, f"one-launch entry point returned {code}"
        torch.cuda.synchronize(gpu)
        assert bitwise_equal(direct, h_ref), bit_mismatch_details(direct, h_ref)
        if with_residual:
            assert bitwise_equal(summed, lin[1])
    # The oracle chain on the same stage inputs: the norm and the GEMM within the GEMM
    # tolerance, SiLU*up on the GPU's own bf16 gate/up outputs within one bf16 ulp.
    y_ref, _ = oracle.rmsnorm(bits16(xg), bits16(nwg), 1e-6, None if rg is None else bits16(rg))
    gu_ref = _bf16(oracle.linear(y_ref, codes(w), ws.numpy()))
    assert_close_rows(gu, gu_ref)
    ulps = np.abs(bits16(h).astype(np.int32) - oracle.silu_mul(bits16(gu[:, :inter]), bits16(gu[:, inter:])).astype(np.int32))
    assert ulps.max() <= 1


def test_rmsnorm_gate_up_silu_edge_cases(gpu):
    """Zero rows give an empty h (and residual sum); an odd merged width is not a gate/up pair
    and is refused by the one-launch entry point (status UNSUPPORTED, nothing launched)."""

    k, n = 512, 2 * 64
    nw = torch.ones(k, dtype=torch.bfloat16, device=gpu)
    w, ws = make_weights(ModelShape("gu_edge", n, k), 3)
    wg, wsg = w.to(gpu), ws.to(gpu)
    empty = torch.empty((0, k), dtype=torch.bfloat16, device=gpu)
    h, summed = fp8.rmsnorm_gate_up_silu_mi355x_fp8(empty, nw, 1e-6, wg, wsg, residual=empty)
    assert h.shape == (0, n // 2) and summed.shape == (0, k)
    x = torch.ones((2, k), dtype=torch.bfloat16, device=gpu)
    w_odd, ws_odd = make_weights(ModelShape("gu_odd", n + 1, k), 3)
    out = torch.full((2, n), 7.0, dtype=torch.bfloat16, device=gpu)
    code = _lib.load().mi355x_fp8_rmsnorm_gate_up_silu(
        x.data_ptr(), 2, k, k, None, 0, None, k, nw.data_ptr(), 1e-6, w_odd.to(gpu).data_ptr(), k,
        ws_odd.to(gpu).data_ptr(), ws_odd.shape[1], 1, n + 1, out.data_ptr(), n, torch.cuda.current_stream(gpu).cuda_stream)
    torch.cuda.synchronize(gpu)
    assert code in (_lib.ERR_INVALID, _lib.ERR_UNSUPPORTED)
    assert (out == 7.0).all().item()
