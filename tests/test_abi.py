"""The C-ABI library loads on a CPU-only machine and exports every symbol the header
declares; argument validation and workspace sizing (host-only paths) behave as
documented.  No call here reaches a kernel launch."""

import ctypes
import os
import re

import pytest

from minillm_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mi355x_fp8.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(mi355x_fp8_\w+)\s*\(", text, re.MULTILINE)))


def test_header_declares_the_bound_entry_points():
    assert declared_functions() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert getattr(lib, name) is not None
    assert lib.mi355x_fp8_abi_version() == _lib.ABI_VERSION


def test_header_constants_match_binding():
    text = open(HEADER).read()
    for macro, value in {"MI355X_FP8_DTYPE_BF16": _lib.DTYPE_BF16, "MI355X_FP8_DTYPE_F16": _lib.DTYPE_F16,
                         "MI355X_FP8_CONFIG_AUTO": _lib.CONFIG_AUTO, "MI355X_FP8_CONFIG_STREAM": _lib.CONFIG_STREAM,
                         "MI355X_FP8_CONFIG_TILE128": _lib.CONFIG_TILE128,
                         "MI355X_FP8_CONFIG_TILE256": _lib.CONFIG_TILE256, "MI355X_FP8_OK": _lib.OK,
                         "MI355X_FP8_ERR_INVALID": _lib.ERR_INVALID, "MI355X_FP8_ERR_UNSUPPORTED": _lib.ERR_UNSUPPORTED,
                         "MI355X_FP8_ERR_WORKSPACE": _lib.ERR_WORKSPACE, "MI355X_FP8_ERR_LAUNCH": _lib.ERR_LAUNCH,
                         "MI355X_FP8_ERR_SCRATCH": _lib.ERR_SCRATCH,
                         "MI355X_FP8_CONFIG_DMA128_64": _lib.CONFIG_DMA128_64,
                         "MI355X_FP8_CONFIG_DMA128_160": _lib.CONFIG_DMA128_160,
                         "MI355X_FP8_CONFIG_T256_128": _lib.CONFIG_T256_128,
                         "MI355X_FP8_CONFIG_T256_256": _lib.CONFIG_T256_256,
                         "MI355X_FP8_CONFIG_T192_128": _lib.CONFIG_T192_128,
                         "MI355X_FP8_CONFIG_T192_256": _lib.CONFIG_T192_256,
                         "MI355X_FP8_CONFIG_DMA64_64": _lib.CONFIG_DMA64_64,
                         "MI355X_FP8_CONFIG_DMA64_128": _lib.CONFIG_DMA64_128,
                         "MI355X_FP8_ABI_VERSION": _lib.ABI_VERSION}.items():
        assert re.search(rf"#define {macro} {value}\b", text), macro


def test_status_strings_and_exception_mapping():
    lib = _lib.load()
    assert lib.mi355x_fp8_status_string(0) == b"ok"
    assert b"workspace" in lib.mi355x_fp8_status_string(_lib.ERR_WORKSPACE)
    with pytest.raises(ValueError):
        _lib.check(_lib.ERR_INVALID)
    with pytest.raises(ValueError):
        _lib.check(_lib.ERR_WORKSPACE)
    with pytest.raises(RuntimeError):
        _lib.check(_lib.ERR_UNSUPPORTED)
    _lib.check(_lib.OK)


def test_workspace_sizes():
    lib = _lib.load()
    # The GEMM needs no workspace; the linear needs room for q (M x Kpad) and scales.
    assert lib.mi355x_fp8_block_gemm_workspace_bytes(8, 6144, 2560, 0) == 0
    need = lib.mi355x_fp8_linear_workspace_bytes(8, 6144, 2560, 0)
    assert need >= 8 * 2560 + 4 * 20 * 8
    assert lib.mi355x_fp8_linear_workspace_bytes(2048, 2560, 9728, 0) >= 2048 * 9728 + 4 * 76 * 2048
    assert lib.mi355x_fp8_linear_workspace_bytes(8, 6144, 0, 0) == 0     # K == 0: invalid
    assert lib.mi355x_fp8_linear_workspace_bytes(8, 6144, 2560, 99) == 0  # unknown config


def test_argument_validation_happens_before_any_launch():
    lib = _lib.load()
    null = None
    # Invalid dtype / K / kpad: rejected on the host.
    assert lib.mi355x_fp8_act_quant(null, 7, 4, 128, 128, 1, null, 128, 128, null, 1, 1, null) == _lib.ERR_INVALID
    assert lib.mi355x_fp8_act_quant(null, 0, 4, 0, 128, 1, null, 128, 128, null, 1, 1, null) == _lib.ERR_INVALID
    assert lib.mi355x_fp8_act_quant(null, 0, 4, 128, 128, 1, null, 128, 64, null, 1, 1, null) == _lib.ERR_INVALID
    # M == 0 is a no-op even with null pointers.
    assert lib.mi355x_fp8_act_quant(null, 0, 0, 128, 128, 1, null, 128, 128, null, 1, 1, null) == _lib.OK
    assert lib.mi355x_fp8_block_gemm(null, 128, null, 1, 1, null, 128, null, 1, 1, null, 0, 64, 0, 64, 128,
                                     null, 0, 0, null) == _lib.OK
    assert lib.mi355x_fp8_block_gemm(null, 64, null, 1, 1, null, 128, null, 1, 1, null, 0, 64, 4, 64, 128,
                                     null, 0, 0, null) == _lib.ERR_INVALID   # ldq < K
    assert lib.mi355x_fp8_block_gemm(null, 128, null, 1, 1, null, 128, null, 1, 1, null, 0, 64, 4, 64, 128,
                                     null, 0, 19, null) == _lib.ERR_INVALID  # unknown config
    # The linear refuses a missing workspace before launching anything.
    dummy = ctypes.c_void_p(16)
    assert lib.mi355x_fp8_linear(dummy, 0, 4, 128, 128, 1, dummy, 128, dummy, 1, 1, 64, dummy, 0, 64, null, 0, 0,
                                 null) == _lib.ERR_WORKSPACE


def test_read_probe_validates_on_the_host():
    lib = _lib.load()
    dummy = ctypes.c_void_p(16)
    assert lib.mi355x_fp8_read_probe(None, 16, dummy, 4096, None) == _lib.ERR_INVALID
    assert lib.mi355x_fp8_read_probe(dummy, 15, dummy, 4096, None) == _lib.ERR_INVALID   # not whole 16-byte units
    assert lib.mi355x_fp8_read_probe(dummy, 0, dummy, 4096, None) == _lib.OK             # nothing to read


# The automatic prefill dispatch's picks on 256 CUs (tile rows, tile width), from the table of
# measured wave times in block_gemm.hip (choose_prefill): M -> (qkv, o_proj, gate_up, down).
PREFILL_PICKS = {
    96: [(64, 64), (64, 64), (128, 128), (64, 64)],
    160: [(128, 64), (64, 64), (128, 160), (64, 64)],
    300: [(64, 128), (64, 64), (192, 160), (64, 64)],
    536: [(128, 128), (128, 64), (192, 256), (128, 64)],
    864: [(192, 128), (128, 128), (128, 160), (128, 128)],
    1024: [(192, 160), (128, 128), (256, 160), (128, 128)],
    2048: [(256, 192), (128, 160), (256, 224), (128, 160)],
    2208: [(256, 224), (192, 128), (256, 256), (192, 128)],
    4096: [(256, 192), (256, 160), (256, 256), (256, 160)],
}


@pytest.mark.parametrize("m", sorted(PREFILL_PICKS))
def test_prefill_dispatch_picks(m):
    """The cost model's kernel for each Qwen3-4B projection (host computation only): the
    M=2048 benchmark shapes, the 192-row tiles past multiples of 256 or 128 (config 5's 536
    rows for gate_up), the 64-row tiles at small M."""

    lib = _lib.load()
    rows, bn = ctypes.c_int(), ctypes.c_int()
    got = []
    for n in (6144, 2560, 19456, 2560):
        assert lib.mi355x_fp8_prefill_choice(m, n, 256, ctypes.byref(rows), ctypes.byref(bn)) == _lib.OK
        got.append((rows.value, bn.value))
    assert got == PREFILL_PICKS[m]
    assert lib.mi355x_fp8_prefill_choice(0, 2560, 256, ctypes.byref(rows), ctypes.byref(bn)) == _lib.ERR_INVALID


def test_rmsnorm_linear_rejects_a_residual_sum_over_its_inputs():
    """The one-launch norm-linear refuses residual_out overlapping x or residual (every
    workgroup reads them while one writes the sum) before touching the device; a disjoint
    sum passes that check (and then fails on the invalid stride, still host-side)."""

    lib = _lib.load()
    m, k, n = 4, 2560, 6144
    x, res = 0x10000000, 0x20000000
    ws, w, nw, out = 0x30000000, 0x40000000, 0x50000000, 0x60000000

    def call(res_out, ldo=n):
        return lib.mi355x_fp8_rmsnorm_linear(x, m, k, k, res, k, res_out, k, nw, 1e-6, w, k, ws, 20, 1, n, out,
                                            ldo, None)

    assert call(res) == _lib.ERR_UNSUPPORTED
    assert call(x) == _lib.ERR_UNSUPPORTED
    assert call(res + 2 * k * (m - 1)) == _lib.ERR_UNSUPPORTED  # last row of the residual
    assert call(res - 2 * k * m + 2) == _lib.ERR_UNSUPPORTED   # ends one element inside it
    assert call(res - 2 * k * m, ldo=n - 1) == _lib.ERR_INVALID  # adjacent, not overlapping


def test_dispatch_choice_names_the_stream_kernel_then_the_prefill_tiles():
    """The automatic dispatch's kernel family (host computation only): the weight-streaming
    kernel at decode sizes (one 16-token slice up to 16 rows; 32-row slices above while the
    weight rows give few workgroups), then the prefill tile the cost model picks (the same
    as mi355x_fp8_prefill_choice)."""

    from minillm_amd import mi355x_fp8 as fp8

    shapes = ((6144, 2560), (2560, 4096), (19456, 2560), (2560, 9728))
    for n, k in shapes:
        for m in (1, 8, 16):
            name = fp8.dispatch_name(m, n, k)
            assert name.startswith("stream ") and name.endswith("x16"), (m, n, name)
    assert [fp8.dispatch_name(32, n, k) for n, k in shapes] == [
        "stream 24x32", "stream 10x32", "tile 64x128", "stream 16x32"]
    for m in (160, 536, 2048):
        assert [fp8.dispatch_name(m, n, k) for n, k in shapes] == [f"tile {r}x{c}" for r, c in PREFILL_PICKS[m]]
    lib = _lib.load()
    a, b, c = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    assert lib.mi355x_fp8_dispatch_choice(0, 2560, 2560, 256, ctypes.byref(a), ctypes.byref(b),
                                          ctypes.byref(c)) == _lib.ERR_INVALID
