"""Build recipe for libmi355x_fp8.so (gfx950 only, compiled in-tree).

``python -m minillm_amd.build`` (or ``build()``) compiles every HIP source of ``csrc/``
with hipcc into ``minillm_amd/lib/libmi355x_fp8.so``.  It compiles every time it is
called.  hipcc cross-compiles, so no GPU is needed.
"""

from __future__ import annotations

import os
import subprocess
import sys

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC_DIR = os.path.join(os.path.dirname(PACKAGE_DIR), "csrc")
LIB_DIR = os.path.join(PACKAGE_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libmi355x_fp8.so")
SOURCES = ("act_quant.hip", "block_gemm.hip", "tile_gemm_dma.hip", "tile_gemm_256.hip", "silu_mul_quant.hip",
           "rmsnorm_quant.hip", "read_probe.hip", "abi.hip")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = (
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared", "-Wall",
    # Keep fp32 math as separate IEEE operations: no fast-math, correctly rounded division,
    # and no contraction of a multiply and an add into one fma (hipcc contracts by default;
    # the RMSNorm's var = ss * (1 / K) and var + eps are two roundings, as in the reference).
    # Every fma the kernels mean is written as one (__builtin_fmaf).
    "-fno-fast-math", "-ffp-contract=off",
    # No packed-fp32 VALU instructions (v_pk_*_f32) anywhere in the library.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in ordinary VGPRs: the per-K-group fold (acc = fma(partial, scale, acc))
    # then reads them directly instead of copying each element out of an AGPR first.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
)


def build(verbose: bool = False) -> str:
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB_PATH + ".tmp"
    cmd = [HIPCC, *FLAGS, *(os.path.join(CSRC_DIR, s) for s in SOURCES), "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed with exit code {proc.returncode}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
