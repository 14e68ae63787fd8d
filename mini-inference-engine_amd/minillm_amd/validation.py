"""Deterministic test/bench data and raw-bit comparisons for the FP8 linear.

Restates the reference's engine/kernels/sm89_fp8_validation.py (shapes, special rows,
raw-bit checks) on torch's CPU generator, so that the host oracle and the GPU see the
same bytes, and adds the Qwen3-4B merged projection shapes and the synthetic
weight/activation recipe of the benchmark configurations.  Importing this module does not
initialise the GPU.  It is not part of inference.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

SEED = 20261008  # scripts/check_fp8_exact.py:43 of the reference


@dataclass(frozen=True)
class ModelShape:
    name: str
    n: int
    k: int
    count: int = 1


# Separate projections of one Qwen3-4B layer (sm89_fp8_validation.py:21-27).
MODEL_SHAPES = (
    ModelShape("q", 4096, 2560),
    ModelShape("kv", 1024, 2560, 2),
    ModelShape("o", 2560, 4096),
    ModelShape("gate_up", 9728, 2560, 2),
    ModelShape("down", 2560, 9728),
)
# The merged projections the engine runs (merged_projections.py: N-concatenation).
QWEN3_4B_PROJECTIONS = (
    ModelShape("qkv", 6144, 2560),
    ModelShape("o_proj", 2560, 4096),
    ModelShape("gate_up", 19456, 2560),
    ModelShape("down", 2560, 9728),
)
# N and K masks, including a tail crossing a scale boundary (sm89_fp8_validation.py:29-30).
TAIL_SHAPES = (ModelShape("tail_1", 129, 1), ModelShape("tail_127", 257, 127),
               ModelShape("tail_129", 193, 129), ModelShape("tail_259", 321, 259))
EXACT_MS = (1, 2, 3, 7, 16, 17, 64, 100, 128, 255, 256, 1000, 2048,
            4097, 8192, 16384, 20000)
BENCH_MS = (1, 16, 64, 256, 1024, 2048, 4096, 8192, 16384)


def make_weights(shape: ModelShape, seed: int, device: str = "cpu"):
    """Signed non-uniform e4m3 weights and non-power-of-two scales
    (sm89_fp8_validation.py:36-46), drawn from a CPU generator."""

    generator = torch.Generator(device="cpu").manual_seed(seed + shape.n * 101 + shape.k * 17)
    weights = (torch.randn((shape.n, shape.k), generator=generator) * 32).clamp(-448, 448)
    weights = weights.to(torch.float8_e4m3fn)
    scales = torch.rand(((shape.n + 127) // 128, (shape.k + 127) // 128), generator=generator,
                        dtype=torch.float32) * 0.09 + 0.001
    return weights.to(device), scales.to(device)


def make_activations(rows: int, k: int, seed: int, dtype=torch.bfloat16, device: str = "cpu"):
    """Activations with outlier columns and the special rows of
    sm89_fp8_validation.py:49-71: zero row, huge row, tiny row (scales below the 1e-12
    clamp), a zero group followed by a tiny group, a -0.0 row, and a +-448 row."""

    generator = torch.Generator(device="cpu").manual_seed(seed + k * 31 + rows * 7)
    x = torch.randn((rows, k), generator=generator)
    x[:, ::31] *= 80
    if rows > 1:
        x[1] = 0
    if rows > 2:
        x[2] *= 1e2 if dtype == torch.float16 else 1e12
        if dtype == torch.float16:
            x[2].clamp_(-60000, 60000)
    if rows > 3:
        x[3] *= 1e-7 if dtype == torch.float16 else 1e-15
    if rows > 4:
        x[4, :min(128, k)] = 0
        x[4, 128:min(256, k)] *= 1e-7 if dtype == torch.float16 else 1e-15
    if rows > 5:
        x[5] = -0.0
    if rows > 6:
        x[6, ::2] = 448
        x[6, 1::2] = -448
    return x.to(dtype).to(device)


def block_quantize_weights(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per 128x128 block: scale = amax/448 in fp32 (1.0 for an all-zero block),
    codes = e4m3fn(w / scale).  The benchmark's fixture recipe for synthetic
    Qwen3-4B-shaped weights (the real checkpoint ships pre-quantized)."""

    n, k = w.shape
    gn, gk = (n + 127) // 128, (k + 127) // 128
    wf = w.float()
    padded = torch.zeros((gn * 128, gk * 128), dtype=torch.float32, device=w.device)
    padded[:n, :k] = wf
    amax = padded.abs().reshape(gn, 128, gk, 128).amax(dim=(1, 3))
    scale = amax / 448.0
    scale = torch.where(amax == 0, torch.ones_like(scale), scale)
    full = scale.repeat_interleave(128, 0).repeat_interleave(128, 1)[:n, :k]
    return (wf / full).to(torch.float8_e4m3fn), scale.contiguous()


def make_baseline_weights(shape: ModelShape, seed: int, device: str = "cpu"):
    """Benchmark weights: N(0, 0.02) in bf16, block-quantized (configs of the baseline)."""

    generator = torch.Generator(device=device).manual_seed(seed + shape.n * 101 + shape.k * 17)
    w = (torch.randn((shape.n, shape.k), generator=generator, device=device) * 0.02).to(torch.bfloat16)
    return block_quantize_weights(w)


def make_baseline_activations(rows: int, k: int, seed: int, outliers: bool = False,
                              device: str = "cpu") -> torch.Tensor:
    """Benchmark activations: N(0, 1) in bf16; with ``outliers`` a seeded 1% of the K
    channels is scaled by 20 before the bf16 cast."""

    generator = torch.Generator(device=device).manual_seed(seed + k * 31 + rows * 7)
    x = torch.randn((rows, k), generator=generator, device=device)
    if outliers:
        count = max(1, k // 100)
        channels = torch.randperm(k, generator=generator, device=device)[:count]
        x[:, channels] *= 20
    return x.to(torch.bfloat16)


def bitwise_equal(left: torch.Tensor, right: torch.Tensor) -> bool:
    """Compare representations, including zero signs and NaN payloads."""

    return bool(
        left.shape == right.shape and left.dtype == right.dtype
        and torch.equal(left.contiguous().view(torch.uint8), right.contiguous().view(torch.uint8))
    )


def bit_mismatch_details(left: torch.Tensor, right: torch.Tensor) -> str:
    if left.shape != right.shape or left.dtype != right.dtype:
        return f"shape/dtype {left.shape}/{left.dtype} != {right.shape}/{right.dtype}"
    view = torch.int16 if left.element_size() == 2 else torch.uint8
    bits_left = left.contiguous().view(view)
    bits_right = right.contiguous().view(view)
    bad = bits_left != bits_right
    count = int(bad.sum().item())
    if not count:
        return "identical"
    first = tuple(int(i) for i in bad.nonzero()[0].tolist())
    mask = 0xffff if view == torch.int16 else 0xff
    return (f"{count}/{left.numel()} elements; first={first}; "
            f"bits=0x{int(bits_left[first].item()) & mask:04x}/0x{int(bits_right[first].item()) & mask:04x}; "
            f"values={left[first].float().item()}/{right[first].float().item()}")


def linear_flops(rows: int, n: int, k: int) -> int:
    """2*M*N*K, the reference's count (scripts/bench_fp8_gemm.py:50-52)."""

    return 2 * rows * n * k


def gemm_bytes(rows: int, n: int, k: int) -> int:
    """Op-level minimum HBM traffic of the GEMM: e4m3 W + fp32 W scales + bf16 x + bf16 out."""

    return n * k + 4 * ((n + 127) // 128) * ((k + 127) // 128) + 2 * rows * k + 2 * rows * n


def quant_bytes(rows: int, k: int) -> int:
    """Quantizer traffic: bf16 in + e4m3 out + fp32 scales."""

    return 3 * rows * k + 4 * rows * ((k + 127) // 128)


def tflops(rows: int, n: int, k: int, milliseconds: float) -> float:
    return linear_flops(rows, n, k) / (milliseconds * 1e9)
