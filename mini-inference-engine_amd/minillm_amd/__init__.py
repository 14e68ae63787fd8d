"""MI355X-native (gfx950) dynamic block-scaled FP8 linear for Qwen3-4B-FP8 projections.

Public surface mirrors the reference's engine/kernels/sm89_fp8.py: see
``minillm_amd.mi355x_fp8``.  The compute runs in hand-written HIP kernels in
``lib/libmi355x_fp8.so`` (C-ABI in include/mi355x_fp8.h), loaded through ctypes.
"""

from . import mi355x_fp8  # noqa: F401
