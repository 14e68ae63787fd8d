"""The reference's exactness gate at its full row range (scripts/check_fp8_exact.py:142-246,
data of engine/kernels/sm89_fp8_validation.py:21-32).

For every shape of MODEL_SHAPES and TAIL_SHAPES (plus the merged q/k/v and gate/up widths,
whose N selects the 256-row kernel's 192- and 224-wide tiles) and every M of EXACT_MS
(1 ... 20000, including 2048, 4097, 8192 and 16384, where the prefill kernels run with
partial last waves), in bf16 and fp16:

* the fused, auto and split paths give the same bits;
* every GEMM config (stream, tile128, tile256 where K % 128 == 0) on the quantized input
  gives those bits, and one-row GEMM calls on the sampled rows give the batch's rows;
* the linear on one row alone gives the batch's row;
* the quantizer on one row alone gives the batch's codes and scales.

Row samples follow the reference's sampled mode: the special rows 0-6, the last row, the
rows on both sides of every 128- and 256-row tile boundary below M (up to 8 of them), and
four seeded random rows.
"""

import sys

import pytest
import torch

from minillm_amd import mi355x_fp8 as fp8
from minillm_amd.validation import (
    EXACT_MS, MODEL_SHAPES, QWEN3_4B_PROJECTIONS, SEED, TAIL_SHAPES, bit_mismatch_details, bitwise_equal,
    make_activations, make_weights,
)

pytestmark = pytest.mark.gpu
BLOCK = [128, 128]
SHAPES = tuple(MODEL_SHAPES) + tuple(TAIL_SHAPES) + tuple(p for p in QWEN3_4B_PROJECTIONS if p.name in ("qkv", "gate_up"))
_DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16}
_data = {}


def _note(*parts):
    print("CASE", *parts, flush=True, file=sys.stderr)


def _inputs(shape, rows, dtype, gpu):
    """The first ``rows`` rows of one EXACT_MS[-1]-row activation matrix per (K, dtype)
    (its special rows 1-6 come first), and the shape's weights, on the GPU."""

    key = (shape.k, dtype)
    if key not in _data:
        _data[key] = make_activations(EXACT_MS[-1], shape.k, SEED, dtype).to(gpu)
    wkey = ("w", shape)
    if wkey not in _data:
        w, ws = make_weights(shape, SEED)
        _data[wkey] = (w.to(gpu), ws.to(gpu))
    return _data[key][:rows], _data[wkey]


def sample_rows(rows: int) -> list[int]:
    picked = set(range(min(rows, 7))) | {rows - 1}
    edges = [b for b in range(128, rows, 128)][:4]
    for b in edges:
        picked |= {b - 1, b}
    gen = torch.Generator().manual_seed(rows)
    picked |= {int(i) for i in torch.randint(0, rows, (4,), generator=gen)}
    return sorted(picked)


@pytest.mark.parametrize("dtype", list(_DTYPES))
@pytest.mark.parametrize("rows", EXACT_MS)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: s.name)
def test_exactness_gate(gpu, shape, rows, dtype):
    _note("gate", shape.name, shape.n, shape.k, rows, dtype)
    x, (w, ws) = _inputs(shape, rows, _DTYPES[dtype], gpu)
    reference = fp8.mi355x_fp8_linear(x, w, ws, BLOCK, path="fused")
    for path in ("auto", "split"):
        actual = fp8.mi355x_fp8_linear(x, w, ws, BLOCK, path=path)
        assert bitwise_equal(reference, actual), (path, bit_mismatch_details(reference, actual))
    picked = sample_rows(rows)
    index = torch.tensor(picked, device=gpu)
    alone = torch.cat([fp8.mi355x_fp8_linear(x[r:r + 1], w, ws, BLOCK, path="fused") for r in picked])
    assert bitwise_equal(alone, reference[index]), ("row alone", bit_mismatch_details(alone, reference[index]))

    q, s = fp8.quantize_mi355x_fp8_activation(x)
    for r in picked:
        q1, s1 = fp8.quantize_mi355x_fp8_activation(x[r:r + 1])
        assert bitwise_equal(q1, q[r:r + 1]) and bitwise_equal(s1, s[r:r + 1]), ("quantizer row", r)
    qk, sk = fp8.quantize_mi355x_fp8_activation(x, scale_layout="kgroup")
    output = torch.empty_like(reference)
    singles = torch.empty((len(picked), shape.n), dtype=reference.dtype, device=gpu)
    for config in fp8.GEMM_CONFIGS:
        if config.needs_dma and shape.k % 128:
            continue
        # tile256 reads K-group-major scales; the others take either layout.
        qa, sa = (qk, sk) if config.needs_dma else (q, s)
        fp8.launch_block_gemm(qa, w, output, sa, ws, config)
        assert bitwise_equal(reference, output), (config.name, bit_mismatch_details(reference, output))
        for pos, r in enumerate(picked):
            fp8.launch_block_gemm(qa[r:r + 1], w, singles[pos:pos + 1], sa[r:r + 1], ws, config)
        assert bitwise_equal(singles, reference[index]), (config.name, "1-row calls",
                                                          bit_mismatch_details(singles, reference[index]))
