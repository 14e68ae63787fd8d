"""Writes tests/golden/fp8_linear_golden.npz: small seeded inputs and the oracle's outputs.

Inputs follow the reference's validation recipe (special rows, outlier columns, tail
shapes; engine/kernels/sm89_fp8_validation.py), drawn from torch's CPU generator.  The
reference ships no known-answer vectors and its kernels need an NVIDIA SM89 GPU, so the
expected values come from the oracle, which tests/test_oracle.py pins independently; the
fixture freezes them so that a later change to the oracle or the kernels shows up as a
diff.  Run: python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "mini-inference-engine_amd"), os.path.join(ROOT, "oracle")]

import torch  # noqa: E402

import oracle  # noqa: E402
from minillm_amd.validation import ModelShape, make_activations, make_weights  # noqa: E402

CASES = [("tail_259", 7, ModelShape("tail_259", 321, 259), torch.bfloat16),
         ("tail_129_fp16", 9, ModelShape("tail_129", 193, 129), torch.float16),
         ("kv_slice", 17, ModelShape("kv_slice", 128, 1280), torch.bfloat16)]


def main() -> None:
    arrays = {}
    for name, rows, shape, dtype in CASES:
        x = make_activations(rows, shape.k, 20261008, dtype)
        w, ws = make_weights(shape, 20261008)
        xb = x.view(torch.int16).numpy().view(np.uint16)
        q, s = oracle.act_quant(xb, is_fp16=dtype == torch.float16)
        out = oracle.block_gemm(q, s, w.view(torch.uint8).numpy(), ws.numpy(), out_fp16=dtype == torch.float16)
        arrays.update({f"{name}/x": xb, f"{name}/w": w.view(torch.uint8).numpy(), f"{name}/ws": ws.numpy(),
                       f"{name}/q": q, f"{name}/s": s, f"{name}/out": out,
                       f"{name}/fp16": np.array(dtype == torch.float16)})
    np.savez_compressed(os.path.join(HERE, "fp8_linear_golden.npz"), **arrays)


if __name__ == "__main__":
    main()
