"""The committed rocprofv3 summaries under profiles/ name kernels that the current library
still contains, and carry the HBM-traffic lines bench.py reads (host-only checks)."""

import os
import re
import subprocess

import pytest

from minillm_amd import _lib
from minillm_amd.build import LIB_PATH

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROFILES = os.path.join(ROOT, "profiles")


def _library_kernels():
    """Demangled kernel names of the built library (host-side kernel handles), written as the
    profiles write them: no namespaces or spaces, 'unsigned char' as u8, no argument list."""

    _lib.load()
    text = subprocess.run(["nm", "-C", LIB_PATH], capture_output=True, text=True, check=True).stdout
    names = set()
    for line in text.splitlines():
        m = re.search(r"mi355x::(?:\(anonymous namespace\)::)?(\w+_kernel<.*?>)\(", line)
        if m and "__device_stub__" not in line:
            k = m.group(1).replace("mi355x::", "").replace("unsigned char", "u8").replace(" ", "")
            names.add(k)
    return names


def test_profiled_kernel_names_exist_in_the_current_build():
    kernels = _library_kernels()
    assert any(k.startswith("tile256_gemm_kernel<") for k in kernels)
    named = set()
    for f in sorted(os.listdir(PROFILES)):
        if f.endswith((".txt", ".md")):
            named |= {(f, k) for k in re.findall(r"\b([a-z_0-9]+_kernel<[^ >]*>)", open(os.path.join(PROFILES, f)).read())}
    assert named
    missing = sorted((f, k) for f, k in named if k not in kernels)
    assert not missing, f"profiles name kernels the library no longer has: {missing}"


def test_traffic_lines_cover_the_benchmark_phases():
    lines = [l.split() for l in open(os.path.join(PROFILES, "hbm_traffic_qwen3.txt")) if l.startswith("TRAFFIC")]
    keys = {(p[1], p[2]) for p in lines if len(p) == 4}
    for phase in ("prefill", "decode"):
        for proj in ("qkv", "o_proj", "gate_up", "down"):
            assert (phase, proj) in keys
