"""Build recipe for libmi355x_fp8.so (gfx950 only, compiled in-tree).

``python -m minillm_amd.build`` (or ``build()``) compiles every HIP source of ``csrc/``
with hipcc into ``minillm_amd/lib/libmi355x_fp8.so``: one object per source, compiled in
parallel (every kernel is launched from its own source file, so no device code crosses
files), then one link.  It compiles every time it is called.  hipcc cross-compiles, so no
GPU is needed.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC_DIR = os.path.join(os.path.dirname(PACKAGE_DIR), "csrc")
LIB_DIR = os.path.join(PACKAGE_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libmi355x_fp8.so")
SOURCES = ("act_quant.hip", "block_gemm.hip", "tile_gemm_dma.hip", "tile_gemm_256.hip", "silu_mul_quant.hip",
           "rmsnorm_quant.hip", "read_probe.hip", "abi.hip")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = (
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
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


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed with exit code {proc.returncode}: {' '.join(cmd)}")


def build(verbose: bool = False) -> str:
    os.makedirs(LIB_DIR, exist_ok=True)
    obj_dir = os.path.join(LIB_DIR, "obj")
    os.makedirs(obj_dir, exist_ok=True)
    objs = [os.path.join(obj_dir, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    jobs = max(1, min(len(SOURCES), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(jobs) as pool:
        list(pool.map(lambda so: _run([HIPCC, *FLAGS, "-c", os.path.join(CSRC_DIR, so[0]), "-o", so[1]], verbose),
                      zip(SOURCES, objs)))
    tmp = LIB_PATH + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
