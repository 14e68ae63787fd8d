"""CPU-only checks of the host layer: dispatch helpers, config contract, error paths and
validation data.  Mirrors the reference's tests/test_sm89_fp8_cpu.py where the behaviour
carries over; no GPU and no kernel launch."""

from dataclasses import FrozenInstanceError

import pytest
import torch

from minillm_amd import _lib
from minillm_amd import mi355x_fp8 as fp8
from minillm_amd.validation import (
    EXACT_MS, MODEL_SHAPES, QWEN3_4B_PROJECTIONS, bit_mismatch_details, bitwise_equal, gemm_bytes,
    make_activations, make_baseline_activations, make_baseline_weights, make_weights, quant_bytes, tflops,
)


@pytest.mark.parametrize("rows,expected", [(0, 1), (1, 1), (2, 2), (3, 4), (17, 32), (255, 256),
                                          (1000, 1024), (4097, 8192), (16384, 16384), (20000, 16384)])
def test_m_bucket(rows, expected):
    assert fp8.m_bucket(rows) == expected


def test_dispatch_threshold_is_inclusive_and_explicit_paths_override(monkeypatch):
    monkeypatch.setattr(fp8, "SPLIT_M_THRESHOLD", 100)
    assert fp8.select_fp8_path(99) == "fused"
    assert fp8.select_fp8_path(100) == "split"
    assert fp8.select_fp8_path(20000, "fused") == "fused"
    assert fp8.select_fp8_path(1, "split") == "split"
    with pytest.raises(ValueError, match="Unknown"):
        fp8.select_fp8_path(1, "typo")
    with pytest.raises(ValueError, match="nonnegative"):
        fp8.m_bucket(-1)


@pytest.mark.parametrize("limit,expected", [(0, (1,)), (1, (1,)), (3, (1, 2, 4)), (8, (1, 2, 4, 8)),
                                          (9, (1, 2, 4, 8, 16))])
def test_pretune_covers_ceiling_bucket(limit, expected):
    assert fp8.pretune_row_buckets(limit) == expected
    assert fp8.pretune_row_buckets(20000)[-1] == fp8.MAX_M_BUCKET


def test_gemm_config_contract():
    configs = fp8.GEMM_CONFIGS
    assert len(set(configs)) == len(configs) and fp8.SPLIT_GEMM_CONFIGS is configs
    assert {c.name for c in configs} >= {"stream", "tile128", "tile256"}
    assert [c.kernel for c in configs] == list(range(1, 19))  # every C-ABI config code, once
    assert [c.name for c in configs if not c.needs_dma] == ["stream", "tile128"]
    for config in configs:
        assert config.block_k == 128
        assert config.label.startswith(config.name)
    with pytest.raises(FrozenInstanceError):
        configs[0].block_k = 256


@pytest.fixture
def fp8_model():
    model = torch.nn.Module()
    for name in ("q", "same_shape"):
        projection = torch.nn.Module()
        projection.weight = torch.nn.Parameter(torch.zeros((129, 259)).to(torch.float8_e4m3fn), requires_grad=False)
        projection.weight_scale_inv = torch.ones((2, 3), dtype=torch.float32)
        model.add_module(name, projection)
    model.register_parameter("bf16", torch.nn.Parameter(torch.zeros(1, dtype=torch.bfloat16)))
    return model


@pytest.mark.parametrize("max_tokens", [1, 3, 17, 1000])
def test_pretune_reserves_workspace_once_and_warms_each_bucket_once(monkeypatch, fp8_model, max_tokens):
    calls, reserved = [], []
    monkeypatch.setattr(fp8, "mi355x_fp8_linear", lambda x, w, s, **kw: calls.append((x.shape[0], tuple(w.shape))))
    monkeypatch.setattr(fp8._workspace, "get", lambda device, nbytes, stream=None: reserved.append(nbytes))
    monkeypatch.setattr(torch.cuda, "synchronize", lambda: None)
    buckets = fp8.pretune_row_buckets(max_tokens)
    # Two modules share one (N, K): it is warmed once per bucket.
    assert fp8.pretune_mi355x_fp8(fp8_model, max_tokens=max_tokens) == len(buckets)
    assert calls == [(b, (129, 259)) for b in buckets]
    lib = _lib.load()
    assert reserved == [lib.mi355x_fp8_linear_workspace_bytes(buckets[-1], 129, 259, _lib.CONFIG_AUTO)]
    assert reserved[0] >= lib.mi355x_fp8_linear_workspace_bytes(max(1, max_tokens), 129, 259, _lib.CONFIG_AUTO)


def test_unsupported_calls_raise_without_fallback():
    x, w, s = torch.zeros(1, 128), torch.zeros(1, 128).to(torch.float8_e4m3fn), torch.ones(1, 1)
    with pytest.raises(RuntimeError, match="no fallback"):
        fp8.mi355x_fp8_linear(x, w, s, [128, 128])
    with pytest.raises(ValueError, match="Unknown"):
        fp8.mi355x_fp8_linear(x, w, s, [128, 128], path="typo")
    with pytest.raises(ValueError, match="gemm_config"):
        fp8.mi355x_fp8_linear(x, w, s, gemm_config=fp8.GEMM_CONFIGS[0])
    with pytest.raises(ValueError, match="2D"):
        fp8.quantize_mi355x_fp8_activation(torch.zeros(2, 3, 4, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="gfx950"):
        fp8.quantize_mi355x_fp8_activation(torch.zeros(2, 4, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="gfx950"):
        fp8.install_mi355x_fp8_dispatch()


def test_supports_call_rejects_each_contract_violation(monkeypatch):
    monkeypatch.setattr(fp8, "mi355x_available", lambda *a: True)

    class FakeCuda(torch.Tensor):
        is_cuda = True

    def t(x):
        return x.as_subclass(FakeCuda)

    x = t(torch.zeros(2, 256, dtype=torch.bfloat16))
    w = t(torch.zeros(130, 256).to(torch.float8_e4m3fn))
    s = t(torch.ones(2, 2))
    assert fp8._supports_call(x, w, s, [128, 128], None)
    assert not fp8._supports_call(x, w, s, [128, 64], None)
    assert not fp8._supports_call(x, w, s, None, None)
    assert not fp8._supports_call(x, w, s, [128, 128], torch.ones(1))
    assert not fp8._supports_call(t(torch.zeros(2, 256)), w, s, [128, 128], None)          # fp32 input
    assert not fp8._supports_call(x, t(torch.zeros(130, 256, dtype=torch.bfloat16)), s, [128, 128], None)
    assert not fp8._supports_call(x, w, t(torch.ones(2, 3)), [128, 128], None)              # scale shape
    assert not fp8._supports_call(t(torch.zeros(2, 255, dtype=torch.bfloat16)), w, s, [128, 128], None)


def test_bit_comparison_detects_zero_sign_and_reports_mismatch():
    left = torch.tensor([[0.0, 1.0]], dtype=torch.bfloat16)
    right = torch.tensor([[-0.0, 1.0]], dtype=torch.bfloat16)
    assert torch.equal(left, right)
    assert not bitwise_equal(left, right)
    assert "1/2 elements" in bit_mismatch_details(left, right)
    assert "first=(0, 0)" in bit_mismatch_details(left, right)
    assert bitwise_equal(left, left.clone())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_validation_data_is_deterministic_finite_and_covers_scale_extremes(dtype):
    x = make_activations(17, 259, 42, dtype)
    assert bitwise_equal(x, make_activations(17, 259, 42, dtype))
    assert torch.isfinite(x).all()
    assert not x[1].count_nonzero()
    assert x[2].abs().max() > x[0].abs().max()
    assert x[3].abs().max() < 1e-4
    w, s = make_weights(MODEL_SHAPES[1], 42)
    assert w.dtype == torch.float8_e4m3fn and s.dtype == torch.float32 and s.shape == (8, 20)
    assert sum(shape.count for shape in MODEL_SHAPES) == 7
    assert EXACT_MS[0] == 1 and EXACT_MS[-1] == 20000


def test_baseline_data_recipe():
    shape = QWEN3_4B_PROJECTIONS[0]
    w, s = make_baseline_weights(shape, 1)
    assert w.shape == (6144, 2560) and s.shape == (48, 20)
    # Each 128x128 block's largest magnitude encodes to +-448 under its own scale.
    blocks = w.view(torch.uint8).reshape(48, 128, 20, 128) & 0x7F
    assert (blocks.amax(dim=(1, 3)) == 0x7E).all()
    x = make_baseline_activations(8, 2560, 1, outliers=True)
    assert x.dtype == torch.bfloat16 and bitwise_equal(x, make_baseline_activations(8, 2560, 1, outliers=True))
    big = (x.float().abs() > 10).any(0).sum().item()
    assert 20 <= big <= 40  # about 1 % of 2560 channels carry the x20 outliers


def test_roofline_byte_and_flop_counts():
    assert tflops(2048, 4096, 2560, 1.0) == pytest.approx(42.94967296)  # reference: bench_fp8_gemm.py
    assert gemm_bytes(8, 6144, 2560) == 6144 * 2560 + 4 * 48 * 20 + 2 * 8 * 2560 + 2 * 8 * 6144
    assert quant_bytes(8, 2560) == 3 * 8 * 2560 + 4 * 8 * 20
    assert sum(p.n * p.k for p in QWEN3_4B_PROJECTIONS) == 100_925_440


def _gemm_operands(m=5, n=130, k=260):
    f8 = torch.float8_e4m3fn
    return dict(activation=torch.zeros(m, k).to(f8), weight=torch.zeros(n, k).to(f8),
                output=torch.empty(m, n, dtype=torch.bfloat16),
                activation_scales=torch.ones(m, (k + 127) // 128), weight_scales=torch.ones((n + 127) // 128, (k + 127) // 128))


@pytest.mark.parametrize("field,bad,match", [
    ("output", torch.empty(4, 130, dtype=torch.bfloat16), "output shape"),
    ("output", torch.empty(5, 130, dtype=torch.float32), "output must be"),
    ("weight", torch.zeros(130, 259).to(torch.float8_e4m3fn), "weight K"),
    ("weight_scales", torch.ones(1, 3), "weight scales shape"),
    ("activation_scales", torch.ones(5, 2), "activation scales shape"),
    ("activation_scales", torch.ones(4, 3), "activation scales shape"),
    ("activation", torch.zeros(5, 260, dtype=torch.bfloat16), "e4m3fn"),
    ("weight_scales", torch.ones(2, 3, dtype=torch.float64), "float32"),
])
def test_launch_block_gemm_rejects_mismatched_operands(field, bad, match):
    """The C-ABI sees bare pointers: the Python entry checks every shape first."""

    ops = _gemm_operands()
    ops[field] = bad
    with pytest.raises(ValueError, match=match):
        fp8.launch_block_gemm(**ops)
    with pytest.raises(ValueError, match="one GPU"):  # well-formed, but on the CPU
        fp8.launch_block_gemm(**_gemm_operands())
