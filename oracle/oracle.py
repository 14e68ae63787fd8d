"""ctypes front end of the C oracle (``fp8_oracle.c``).  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import this module, as the checker or as the timed CPU baseline.  The product path
(``minillm_amd``) never imports it.

Arrays are numpy: bf16/fp16 values travel as their uint16 bit patterns, e4m3fn codes as
uint8, scales as float32.  Every function restates the reference's arithmetic; see the
C source for the file:line each one follows.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libfp8_oracle.so")
_lib = None

_i64 = ctypes.c_int64
_ptr = ctypes.c_void_p


def build() -> str:
    """Compile the oracle library with the committed Makefile."""

    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        handle = ctypes.CDLL(_LIB_PATH)
        handle.orc_f32_to_e4m3_array.argtypes = [_ptr, _ptr, _i64]
        handle.orc_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        handle.orc_e4m3_to_f32.restype = ctypes.c_float
        handle.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        handle.orc_f32_to_bf16.restype = ctypes.c_uint16
        handle.orc_f32_to_f16.argtypes = [ctypes.c_float]
        handle.orc_f32_to_f16.restype = ctypes.c_uint16
        handle.orc_act_quant.argtypes = [_ptr, ctypes.c_int, _i64, _i64, _i64, _i64, _ptr, _ptr]
        handle.orc_block_gemm.argtypes = [
            _ptr, _i64, _ptr, _i64, _i64, _ptr, _i64, _ptr, _i64, _i64, _ptr, ctypes.c_int,
            _i64, _i64, _i64, _i64, ctypes.c_int]
        handle.orc_linear.argtypes = [
            _ptr, ctypes.c_int, _i64, _i64, _i64, _i64, _ptr, _ptr, _i64, _ptr, ctypes.c_int,
            _ptr, _ptr, ctypes.c_int]
        handle.orc_max_threads.restype = ctypes.c_int
        handle.orc_silu_mul.argtypes = [_ptr, _ptr, _i64, _ptr]
        handle.orc_rmsnorm_block_width.argtypes = [_i64, _i64]
        handle.orc_rmsnorm_block_width.restype = _i64
        handle.orc_rmsnorm.argtypes = [_ptr, _ptr, _i64, _ptr, _i64, _i64, ctypes.c_float, _ptr, _ptr]
        handle.orc_rmsnorm_sumsq.argtypes = [_ptr, _ptr, _i64, _i64, _i64, _ptr]
        _lib = handle
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def groups(k: int) -> int:
    return (k + 127) // 128


def f32_to_e4m3(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even, saturating fp32 -> e4m3fn codes."""

    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().orc_f32_to_e4m3_array(_p(x), _p(out), x.size)
    return out


def e4m3_to_f32(codes: np.ndarray) -> np.ndarray:
    table = np.array([lib().orc_e4m3_to_f32(c) for c in range(256)], dtype=np.float32)
    return table[np.asarray(codes, dtype=np.uint8)]


def act_quant(x_bits: np.ndarray, is_fp16: bool = False) -> tuple[np.ndarray, np.ndarray]:
    """Per-row 1x128 quantizer (reference engine/kernels/sm89_fp8.py:304-332).

    ``x_bits``: [M, K] uint16 bit patterns (any strides).  Returns ``(q, s)``: q [M, K]
    uint8 e4m3fn codes, s [M, ceil(K/128)] float32 raw scales.
    """

    x_bits = np.asarray(x_bits, dtype=np.uint16)
    m, k = x_bits.shape
    if k == 0:
        raise ValueError("Activation width must be positive")
    q = np.empty((m, k), dtype=np.uint8)
    s = np.empty((m, groups(k)), dtype=np.float32)
    sm, sk = (st // 2 for st in x_bits.strides)
    lib().orc_act_quant(_p(x_bits), int(is_fp16), m, k, sm, sk, _p(q), _p(s))
    return q, s


def block_gemm(q: np.ndarray, a_s: np.ndarray, w: np.ndarray, w_s: np.ndarray,
               out_fp16: bool = False, threads: int = 0) -> np.ndarray:
    """Block-scaled GEMM (reference engine/kernels/sm89_fp8.py:344-398).

    q [M, K] uint8, a_s [M, G] f32, w [N, K] uint8, w_s [ceil(N/128), G] f32.
    Returns [M, N] uint16 bit patterns of bf16 (or fp16) outputs.
    """

    q = np.ascontiguousarray(q, dtype=np.uint8)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    a_s = np.ascontiguousarray(a_s, dtype=np.float32)
    w_s = np.ascontiguousarray(w_s, dtype=np.float32)
    m, k = q.shape
    n = w.shape[0]
    g = groups(k)
    if w.shape[1] != k or a_s.shape != (m, g) or w_s.shape != (groups(n), g):
        raise ValueError("shape mismatch")
    out = np.empty((m, n), dtype=np.uint16)
    lib().orc_block_gemm(_p(q), k, _p(a_s), g, 1, _p(w), k, _p(w_s), g, 1, _p(out),
                         int(out_fp16), n, m, n, k, threads)
    return out


def linear(x_bits: np.ndarray, w: np.ndarray, w_s: np.ndarray, is_fp16: bool = False,
           out_fp16: bool = False, threads: int = 0) -> np.ndarray:
    """Quantize then GEMM: the reference's split path (sm89_fp8.py:501-505)."""

    q, s = act_quant(x_bits, is_fp16)
    return block_gemm(q, s, w, w_s, out_fp16, threads)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    f = np.vectorize(lambda v: lib().orc_f32_to_bf16(float(v)), otypes=[np.uint16])
    return f(x) if x.size else np.empty(x.shape, dtype=np.uint16)


def silu_mul(gate_bits: np.ndarray, up_bits: np.ndarray) -> np.ndarray:
    """bf16 SiLU(gate) * up (reference engine/kernels/fused.py:127-137), as bf16 bits."""

    g = np.ascontiguousarray(gate_bits, dtype=np.uint16)
    u = np.ascontiguousarray(up_bits, dtype=np.uint16)
    if g.shape != u.shape:
        raise ValueError("shape mismatch")
    out = np.empty(g.shape, dtype=np.uint16)
    lib().orc_silu_mul(_p(g), _p(u), g.size, _p(out))
    return out


def rmsnorm_block_width(rows: int, n_cols: int) -> int:
    return int(lib().orc_rmsnorm_block_width(rows, n_cols))


def rmsnorm(x_bits: np.ndarray, w_bits: np.ndarray, eps: float,
            residual_bits: np.ndarray | None = None) -> tuple[np.ndarray, np.ndarray | None]:
    """Qwen3 RMSNorm in the reference's arithmetic and summation order
    (engine/kernels/fused.py:89-124, 165-199), bf16 bits in and out.  Returns ``(y, summed)``;
    ``summed`` (bf16(x + residual)) is None without a residual."""

    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    rows, n_cols = x.shape
    if n_cols % 4 or w.shape != (n_cols,):
        raise ValueError("width must be a multiple of 4 and match the weight")
    y = np.empty((rows, n_cols), dtype=np.uint16)
    summed = None
    r = None
    if residual_bits is not None:
        r = np.ascontiguousarray(residual_bits, dtype=np.uint16)
        if r.shape != x.shape:
            raise ValueError("shape mismatch")
        summed = np.empty((rows, n_cols), dtype=np.uint16)
    lib().orc_rmsnorm(_p(x), None if r is None else _p(r), n_cols, _p(w), rows, n_cols, float(eps), _p(y),
                      None if summed is None else _p(summed))
    return y, summed


def rmsnorm_sumsq(x_bits: np.ndarray, residual_bits: np.ndarray | None = None) -> np.ndarray:
    """Per-row fp32 sum of squares that ``rmsnorm`` forms (same order, same rows in a batch
    of this many rows), for tests that pin the summation order."""

    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    rows, n_cols = x.shape
    r = None if residual_bits is None else np.ascontiguousarray(residual_bits, dtype=np.uint16)
    out = np.empty(rows, dtype=np.float32)
    lib().orc_rmsnorm_sumsq(_p(x), None if r is None else _p(r), n_cols, rows, n_cols, _p(out))
    return out


def max_threads() -> int:
    return int(lib().orc_max_threads())


def weight_quant(w_f32: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Fixture recipe for weights: per 128x128 block, scale = amax/448 (1.0 for an
    all-zero block), codes = e4m3(w / scale).  Not on the reference's path (its
    checkpoint is pre-quantized); used to build synthetic Qwen3-4B-shaped weights."""

    w_f32 = np.ascontiguousarray(w_f32, dtype=np.float32)
    n, k = w_f32.shape
    gn, gk = groups(n), groups(k)
    pad = np.zeros((gn * 128, gk * 128), dtype=np.float32)
    pad[:n, :k] = w_f32
    blocks = np.abs(pad.reshape(gn, 128, gk, 128))
    amax = blocks.max(axis=(1, 3)).astype(np.float32)
    scale = (amax / np.float32(448.0)).astype(np.float32)
    scale[amax == 0] = 1.0
    full = np.repeat(np.repeat(scale, 128, axis=0), 128, axis=1)[:n, :k]
    codes = f32_to_e4m3((w_f32 / full).astype(np.float32))
    return codes, scale
