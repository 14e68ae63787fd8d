"""Dynamic block-scaled FP8 linear for AMD MI355X (gfx950), Transformers-compatible.

Mirrors the call surface of the reference's engine/kernels/sm89_fp8.py: the same
``fp8_linear`` signature (so ``FP8Linear.forward`` and the merged projections call it
unchanged), the same dispatch/bucket helpers, the same exception types.  The arithmetic
runs in two hand-written gfx950 HIP kernels behind a C-ABI (include/mi355x_fp8.h):

* a per-token 1x128 activation quantizer: s = amax/448 stored raw,
  q = e4m3fn(x / max(s, 1e-12)) -- bit-exact with the reference's quantizer;
* a block-scaled FP8 GEMM on CDNA4 fp8 MFMA that accumulates, per 128-wide K group in
  increasing order, dot(q, w) * a_s * w_s in fp32 and rounds once to bf16/fp16.

There is no second backend: a call outside the supported set raises instead of
delegating (the reference delegates to Transformers, sm89_fp8.py:467-481).
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass
from typing import Any

import torch

from . import _lib

SUPPORTED_BLOCK_SIZE = (128, 128)
# Same bucket cap and dispatch threshold names as sm89_fp8.py:26-34.  Both paths run
# the same quantizer + GEMM here; the names stay for call-surface compatibility.
MAX_M_BUCKET = 16384
SPLIT_M_THRESHOLD = 256
# Rows at or below which the auto GEMM choice is the weight-streaming (decode) kernel.
STREAM_M_THRESHOLD = 64
_original_fp8_linear: Callable[..., torch.Tensor] | None = None


@dataclass(frozen=True)
class FP8GemmConfig:
    """A forced GEMM kernel choice (the reference's FP8GemmConfig, sm89_fp8.py:38-62).

    ``block_k`` is fixed at 128: one K group per MFMA, so a config changes speed, never
    the grouping of the arithmetic.
    """

    name: str
    kernel: int
    block_m: int
    block_n: int
    block_k: int = 128

    @property
    def label(self) -> str:
        return f"{self.name}:{self.block_m}x{self.block_n}x{self.block_k}"

    @property
    def needs_dma(self) -> bool:
        """Runs only on LDS-DMA operands: K % 128 == 0, 16-byte aligned codes and
        K-group-major activation scales (other calls raise "unsupported")."""
        return self.kernel >= _lib.CONFIG_TILE256


GEMM_CONFIGS = (
    FP8GemmConfig("stream", _lib.CONFIG_STREAM, 64, 64),
    FP8GemmConfig("tile128", _lib.CONFIG_TILE128, 128, 128),
    FP8GemmConfig("tile256", _lib.CONFIG_TILE256, 256, 256),
    # One kernel variant each (tuning, and tests that reach every variant).
    FP8GemmConfig("dma128x64", _lib.CONFIG_DMA128_64, 128, 64),
    FP8GemmConfig("dma128x128", _lib.CONFIG_DMA128_128, 128, 128),
    FP8GemmConfig("dma128x160", _lib.CONFIG_DMA128_160, 128, 160),
    FP8GemmConfig("t256x128", _lib.CONFIG_T256_128, 256, 128),
    FP8GemmConfig("t256x160", _lib.CONFIG_T256_160, 256, 160),
    FP8GemmConfig("t256x192", _lib.CONFIG_T256_192, 256, 192),
    FP8GemmConfig("t256x224", _lib.CONFIG_T256_224, 256, 224),
    FP8GemmConfig("t256x256", _lib.CONFIG_T256_256, 256, 256),
    FP8GemmConfig("t192x128", _lib.CONFIG_T192_128, 192, 128),
    FP8GemmConfig("t192x160", _lib.CONFIG_T192_160, 192, 160),
    FP8GemmConfig("t192x192", _lib.CONFIG_T192_192, 192, 192),
    FP8GemmConfig("t192x224", _lib.CONFIG_T192_224, 192, 224),
    FP8GemmConfig("t192x256", _lib.CONFIG_T192_256, 192, 256),
    FP8GemmConfig("dma64x64", _lib.CONFIG_DMA64_64, 64, 64),
    FP8GemmConfig("dma64x128", _lib.CONFIG_DMA64_128, 64, 128),
)
# Alias under the reference's name.
SPLIT_GEMM_CONFIGS = GEMM_CONFIGS


def m_bucket(rows: int) -> int:
    """Ceiling power of two, capped at the last pre-tuned bucket (sm89_fp8.py:89-94)."""

    if rows < 0:
        raise ValueError("rows must be nonnegative")
    return min(1 << (max(1, rows) - 1).bit_length(), MAX_M_BUCKET)


def select_fp8_path(rows: int, path: str = "auto") -> str:
    """Resolve dispatch; the threshold is inclusive (sm89_fp8.py:97-104)."""

    if path not in {"auto", "fused", "split"}:
        raise ValueError(f"Unknown MI355X FP8 path: {path!r}")
    if rows < 0:
        raise ValueError("rows must be nonnegative")
    return ("split" if rows >= SPLIT_M_THRESHOLD else "fused") if path == "auto" else path


def pretune_row_buckets(max_tokens: int) -> tuple[int, ...]:
    """Every power-of-two bucket through the ceiling bucket (sm89_fp8.py:107-110)."""

    return tuple(1 << i for i in range(m_bucket(max(1, max_tokens)).bit_length()))


_ARCH_OK: dict[int, bool] = {}  # device index -> is gfx950 (device properties do not change)


def dispatch_name(rows: int, n: int, k: int, cus: int = 256) -> str:
    """The kernel the automatic dispatch runs for an ``rows x n x k`` GEMM on ``cus`` CUs
    (aligned operands, K % 128 == 0): ``"stream WxT"`` (the weight-streaming decode kernel,
    W weight rows per workgroup, T token rows per slice) or ``"tile RxC"`` (a prefill tile).
    Host-only: asks the library's planner, touches no device."""

    import ctypes

    kernel, r, c = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    _lib.check(_lib.load().mi355x_fp8_dispatch_choice(rows, n, k, cus, ctypes.byref(kernel), ctypes.byref(r),
                                                       ctypes.byref(c)))
    return f"{'stream' if kernel.value == _lib.CONFIG_STREAM else 'tile'} {r.value}x{c.value}"


def _device_index(device: torch.device | str | int | None) -> int:
    if device is None:
        return torch.cuda.current_device()
    if isinstance(device, int):
        return device
    device = torch.device(device)
    return device.index if device.index is not None else torch.cuda.current_device()


def mi355x_available(device: torch.device | str | int | None = None) -> bool:
    """Whether a gfx950 GPU is visible to torch (the reference's sm89_available)."""

    if not _ARCH_OK and not torch.cuda.is_available():
        return False
    index = _device_index(device)
    ok = _ARCH_OK.get(index)
    if ok is None:
        if not torch.cuda.is_available():
            return False
        props = torch.cuda.get_device_properties(index)
        ok = _ARCH_OK[index] = str(getattr(props, "gcnArchName", "")).split(":")[0] == "gfx950"
    return ok


def _supports_call(input, weight, weight_scale_inv, block_size, activation_scale) -> bool:
    """The accepted call set of sm89_fp8.py:123-147, on a gfx950 device."""

    return bool(
        input.is_cuda and weight.is_cuda and weight_scale_inv.is_cuda
        and input.device == weight.device == weight_scale_inv.device
        and mi355x_available(weight.device)
        and input.dtype in {torch.float16, torch.bfloat16}
        and weight.dtype == torch.float8_e4m3fn
        and weight_scale_inv.dtype == torch.float32
        and input.ndim >= 2 and weight.ndim == 2 and weight_scale_inv.ndim == 2
        and block_size is not None and tuple(block_size) == SUPPORTED_BLOCK_SIZE
        and activation_scale is None
        and input.shape[-1] == weight.shape[1]
        and tuple(weight_scale_inv.shape)
        == ((weight.shape[0] + 127) // 128, (weight.shape[1] + 127) // 128)
    )


def _dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return _lib.DTYPE_BF16
    if dtype == torch.float16:
        return _lib.DTYPE_F16
    raise TypeError(f"unsupported dtype {dtype}")


class _Workspace:
    """Per (device, stream) scratch byte buffer, grown on demand.

    Calls on one stream are ordered, so they may share it; different streams get
    different buffers.  Growing happens only on a larger shape than any seen before on
    that stream (``pretune_mi355x_fp8`` warms the largest), so steady-state calls and
    HIP-graph captures allocate nothing.
    """

    def __init__(self) -> None:
        self._buffers: dict[tuple[int, int], torch.Tensor] = {}

    def get(self, device: torch.device, nbytes: int, stream: int | None = None) -> torch.Tensor | None:
        if nbytes == 0:
            return None
        key = (_device_index(device), _stream_ptr(device) if stream is None else stream)
        buf = self._buffers.get(key)
        if buf is None or buf.numel() < nbytes:
            grown = max(nbytes, 0 if buf is None else 2 * buf.numel())
            buf = torch.empty(grown, dtype=torch.uint8, device=device)
            self._buffers[key] = buf
        return buf

    def clear(self) -> None:
        self._buffers.clear()


_workspace = _Workspace()


# torch's current HIP stream of a device as a raw handle; the private getter skips building a
# Stream object (a few microseconds per call on the eager path).
_current_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_ptr(device: torch.device) -> int:
    if _current_raw_stream is not None:
        return _current_raw_stream(_device_index(device))
    return torch.cuda.current_stream(device).cuda_stream


def quantize_mi355x_fp8_activation(input_2d: torch.Tensor, *, scale_layout: str = "row"
                                   ) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize a 2-D activation once: ``(q [M, K] e4m3fn, s [M, ceil(K/128)] fp32)``.

    Same contract and errors as quantize_sm89_fp8_activation (sm89_fp8.py:401-424); the
    input may have any strides, q is contiguous and the scales are raw.  With
    ``scale_layout="kgroup"`` the scales are stored K-group-major (the returned ``s`` is a
    strided [M, G] view of a [G, roundup(M, 64)] buffer, stride (1, roundup(M, 64))): the
    layout the prefill GEMM streams into LDS.  Values are identical in both layouts.
    """

    if input_2d.ndim != 2 or input_2d.dtype not in {torch.bfloat16, torch.float16}:
        raise ValueError("Expected a 2D bf16/fp16 activation")
    if scale_layout not in {"row", "kgroup"}:
        raise ValueError(f"Unknown scale layout: {scale_layout!r}")
    if not input_2d.is_cuda or not mi355x_available(input_2d.device):
        raise RuntimeError("Activation quantization requires an MI355X (gfx950) GPU")
    m, k = input_2d.shape
    if k == 0:
        raise ValueError("Activation width must be positive")
    groups_k = (k + 127) // 128
    quantized = torch.empty((m, k), device=input_2d.device, dtype=torch.float8_e4m3fn)
    if scale_layout == "row":
        scales = torch.empty((m, groups_k), device=input_2d.device, dtype=torch.float32)
        s_sm, s_sk = groups_k, 1
    else:
        mpad = max(64, -(-m // 64) * 64)
        scales = torch.empty((groups_k, mpad), device=input_2d.device, dtype=torch.float32)[:, :m].t()
        s_sm, s_sk = 1, mpad
    if m:
        _lib.check(_lib.load().mi355x_fp8_act_quant(
            input_2d.data_ptr(), _dtype_code(input_2d.dtype), m, k, input_2d.stride(0), input_2d.stride(1),
            quantized.data_ptr(), k, k, scales.data_ptr(), s_sm, s_sk, _stream_ptr(input_2d.device)))
    return quantized, scales


def _config_code(config: FP8GemmConfig | None) -> int:
    return _lib.CONFIG_AUTO if config is None else config.kernel


def _check_gemm_operands(activation: torch.Tensor, weight: torch.Tensor, output: torch.Tensor,
                         activation_scales: torch.Tensor, weight_scales: torch.Tensor) -> None:
    """Every shape, dtype, stride and device fact the C-ABI's kernels rely on but cannot
    see (it receives bare pointers); a violation raises ValueError before any launch."""

    tensors = (activation, weight, output, activation_scales, weight_scales)
    if any(t.ndim != 2 for t in tensors):
        raise ValueError("GEMM operands must be 2-D")
    if activation.dtype != torch.float8_e4m3fn or weight.dtype != torch.float8_e4m3fn:
        raise ValueError("activation and weight must be float8_e4m3fn")
    if activation_scales.dtype != torch.float32 or weight_scales.dtype != torch.float32:
        raise ValueError("activation and weight scales must be float32")
    if output.dtype not in {torch.bfloat16, torch.float16}:
        raise ValueError("output must be bfloat16 or float16")
    m, k = activation.shape
    n = weight.shape[0]
    kb, nb = (k + 127) // 128, (n + 127) // 128
    if weight.shape[1] != k:
        raise ValueError(f"weight K {weight.shape[1]} != activation K {k}")
    if tuple(output.shape) != (m, n):
        raise ValueError(f"output shape {tuple(output.shape)} != ({m}, {n})")
    if tuple(weight_scales.shape) != (nb, kb):
        raise ValueError(f"weight scales shape {tuple(weight_scales.shape)} != ({nb}, {kb})")
    if tuple(activation_scales.shape) != (m, kb):
        raise ValueError(f"activation scales shape {tuple(activation_scales.shape)} != ({m}, {kb})")
    for name, t in (("activation", activation), ("weight", weight), ("output", output)):
        if t.stride(-1) != 1 or (t.shape[0] > 1 and t.stride(0) < t.shape[1]):
            raise ValueError(f"{name} needs unit column stride and non-overlapping rows")
    if any(st < 0 for t in (activation_scales, weight_scales) for st in t.stride()):
        raise ValueError("scale strides must be nonnegative")
    if len({t.device for t in tensors}) != 1 or not activation.is_cuda:
        raise ValueError("GEMM operands must be on one GPU")


def launch_block_gemm(activation: torch.Tensor, weight: torch.Tensor, output: torch.Tensor,
                      activation_scales: torch.Tensor, weight_scales: torch.Tensor,
                      config: FP8GemmConfig | None = None) -> None:
    """GEMM on pre-quantized activations into ``output`` (the reference's
    _launch_split_gemm, sm89_fp8.py:427-441).  ``config`` forces a kernel."""

    _check_gemm_operands(activation, weight, output, activation_scales, weight_scales)
    m, k = activation.shape
    n = weight.shape[0]
    lib = _lib.load()
    code = _config_code(config)
    nbytes = lib.mi355x_fp8_block_gemm_workspace_bytes(m, n, k, code)
    stream = _stream_ptr(output.device)
    ws = _workspace.get(output.device, nbytes, stream)
    _lib.check(lib.mi355x_fp8_block_gemm(
        activation.data_ptr(), activation.stride(0), activation_scales.data_ptr(),
        activation_scales.stride(0), activation_scales.stride(1), weight.data_ptr(), weight.stride(0),
        weight_scales.data_ptr(), weight_scales.stride(0), weight_scales.stride(1), output.data_ptr(),
        _dtype_code(output.dtype), output.stride(0), m, n, k,
        None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), code, stream))


def mi355x_fp8_linear(
    input: torch.Tensor,
    weight: torch.Tensor,
    weight_scale_inv: torch.Tensor,
    block_size: list[int] | tuple[int, int] | None = None,
    bias: torch.Tensor | None = None,
    activation_scale: torch.Tensor | None = None,
    output_dtype: torch.dtype | None = None,
    allow_deepgemm: bool = True,
    *,
    path: str = "auto",
    gemm_config: FP8GemmConfig | None = None,
) -> torch.Tensor:
    """Transformers-compatible FP8 linear (the reference's sm89_fp8_linear,
    sm89_fp8.py:444-528).

    ``path`` accepts "auto", "fused" and "split" (all three run the quantizer + block
    GEMM); ``gemm_config`` requires ``path="split"`` and forces the GEMM kernel.
    ``allow_deepgemm`` is accepted and ignored, as in the reference's fast path.
    """

    select_fp8_path(0, path)  # reject typos first
    if gemm_config is not None and (path != "split" or gemm_config not in GEMM_CONFIGS):
        raise ValueError("gemm_config must be a listed GEMM config with path='split'")
    if not _supports_call(input, weight, weight_scale_inv, block_size, activation_scale):
        raise RuntimeError(
            "Unsupported MI355X FP8 call (needs gfx950 tensors, bf16/fp16 input, e4m3fn weight, "
            "fp32 [ceil(N/128), ceil(K/128)] scales, block_size (128, 128), no activation_scale); "
            "there is no fallback backend")
    if output_dtype is not None and output_dtype not in {torch.float16, torch.bfloat16}:
        raise TypeError("MI355X FP8 output must be float16 or bfloat16")

    k = int(input.shape[-1])
    m = int(input.numel() // k) if k else 0
    n = int(weight.shape[0])
    out_dtype = output_dtype or input.dtype
    output = torch.empty((m, n), device=input.device, dtype=out_dtype)
    select_fp8_path(m, path)
    if m == 0 or n == 0:
        result = output.reshape(*input.shape[:-1], n)
        return result if bias is None else result + bias
    if k == 0:
        raise ValueError("Activation width must be positive")
    input_2d = input.reshape(m, k)
    if input_2d.stride(-1) != 1:
        input_2d = input_2d.contiguous()
    weight_2d = weight if weight.stride(-1) == 1 else weight.contiguous()
    scales_2d = weight_scale_inv
    lib = _lib.load()
    code = _config_code(gemm_config)
    nbytes = lib.mi355x_fp8_linear_workspace_bytes(m, n, k, code)
    stream = _stream_ptr(input.device)
    ws = _workspace.get(input.device, nbytes, stream)
    _lib.check(lib.mi355x_fp8_linear(
        input_2d.data_ptr(), _dtype_code(input_2d.dtype), m, k, input_2d.stride(0), input_2d.stride(1),
        weight_2d.data_ptr(), weight_2d.stride(0), scales_2d.data_ptr(), scales_2d.stride(0),
        scales_2d.stride(1), n, output.data_ptr(), _dtype_code(out_dtype), output.stride(0),
        ws.data_ptr(), ws.numel(), code, stream))
    result = output.reshape(*input.shape[:-1], n)
    return result if bias is None else result + bias


# The name Transformers' FP8Linear calls.
fp8_linear = mi355x_fp8_linear


def _fp8_linear_shapes(model: Any) -> list[tuple[torch.Tensor, torch.Tensor, tuple[int, ...]]]:
    """``(weight, scales, block_size)`` of every module holding an e4m3fn weight with fp32 scales."""

    found = []
    for module in model.modules():
        weight = getattr(module, "weight", None)
        scales = getattr(module, "weight_scale_inv", None)
        if isinstance(weight, torch.Tensor) and weight.dtype == torch.float8_e4m3fn and isinstance(scales, torch.Tensor):
            found.append((weight, scales, tuple(getattr(module, "block_size", SUPPORTED_BLOCK_SIZE))))
    return found


def pretune_mi355x_fp8(model: Any, max_tokens: int = MAX_M_BUCKET) -> int:
    """Make every later FP8 linear call of ``model`` allocation-free (the role of the
    reference's pretune, sm89_fp8.py:531-558, which fills Triton's autotune cache).

    Nothing here is tuned: the kernel is a closed-form choice from (M, N, K).  What a
    call can still need is its workspace (the quantized activations and their scales),
    so this reserves the current stream's workspace once, at the size the largest
    shape needs at the ceiling bucket, and then runs each distinct (N, K) shape once
    per row bucket so that every kernel the dispatch can pick is loaded before a HIP
    graph is captured.  Returns the number of (shape, bucket) pairs warmed.
    """

    dtype = next(p.dtype for p in model.parameters() if p.dtype in {torch.bfloat16, torch.float16})
    return pretune_mi355x_fp8_shapes(_fp8_linear_shapes(model), dtype, max_tokens)


def pretune_mi355x_fp8_shapes(shapes: Any, dtype: torch.dtype, max_tokens: int = MAX_M_BUCKET) -> int:
    """``pretune_mi355x_fp8`` for explicit ``(weight, scales, block_size)`` triples."""

    by_shape: dict[tuple[int, int], tuple[torch.Tensor, torch.Tensor, tuple[int, ...]]] = {}
    for weight, scales, block in shapes:
        by_shape.setdefault((int(weight.shape[0]), int(weight.shape[1])), (weight, scales, tuple(block)))
    if not by_shape:
        return 0
    buckets = pretune_row_buckets(int(max_tokens))
    device = next(iter(by_shape.values()))[0].device
    lib = _lib.load()
    need = max(lib.mi355x_fp8_linear_workspace_bytes(buckets[-1], n, k, _lib.CONFIG_AUTO) for n, k in by_shape)
    _workspace.get(device, need)
    with torch.inference_mode():
        for weight, scales, block in by_shape.values():
            activation = torch.zeros((buckets[-1], weight.shape[1]), dtype=dtype, device=weight.device)
            for bucket in buckets:
                mi355x_fp8_linear(activation[:bucket], weight, scales, block_size=list(block))
    torch.cuda.synchronize()
    return len(by_shape) * len(buckets)


def install_mi355x_fp8_dispatch() -> dict[str, Any]:
    """Swap Transformers' ``finegrained_fp8.fp8_linear`` for this op (sm89_fp8.py:579-610)."""

    if not mi355x_available():
        arch = (str(torch.cuda.get_device_properties(torch.cuda.current_device()).gcnArchName)
                if torch.cuda.is_available() else None)
        raise RuntimeError(f"The custom FP8 kernel requires an AMD gfx950 (MI355X) GPU; detected arch={arch}")
    _lib.load()
    from transformers.integrations import finegrained_fp8

    global _original_fp8_linear
    if finegrained_fp8.fp8_linear is not mi355x_fp8_linear:
        _original_fp8_linear = finegrained_fp8.fp8_linear
        finegrained_fp8.fp8_linear = mi355x_fp8_linear
    return {
        "installed": True,
        "backend": "minillm_mi355x_hip_fp8",
        "arch_required": "gfx950",
        "block_size": [128, 128],
        "fused_operations": [
            "dynamic activation scaling",
            "FP8 E4M3 activation quantization",
            "block-scaled FP8 matrix multiplication",
        ],
        "fallback": None,
    }


def uninstall_mi355x_fp8_dispatch() -> None:
    """Restore the ``fp8_linear`` that ``install_mi355x_fp8_dispatch`` replaced."""

    global _original_fp8_linear
    if _original_fp8_linear is None:
        return
    from transformers.integrations import finegrained_fp8

    finegrained_fp8.fp8_linear = _original_fp8_linear
    _original_fp8_linear = None


def silu_mul_quant_mi355x_fp8(gate: torch.Tensor, up: torch.Tensor, *, scale_layout: str = "kgroup",
                              return_intermediate: bool = False):
    """``SiLU(gate) * up`` in bf16, quantized per row and 128-column group, in one kernel.

    The elementwise part is the reference's silu_mul (engine/kernels/fused.py:127-137,
    217-232: silu rounded to bf16, then a bf16 multiply); the quantization is the
    activation quantizer's (sm89_fp8.py:304-332).  ``gate`` and ``up`` are [..., I] bf16
    with the same row stride and unit column stride (e.g. the two column views of one
    merged gate_up output).  Returns ``(q, s)`` or, with ``return_intermediate``,
    ``(h, q, s)`` where h is the bf16 product (what the reference feeds to down_proj).
    """

    if gate.shape != up.shape or gate.dtype != torch.bfloat16 or up.dtype != torch.bfloat16:
        raise ValueError("gate and up must be bf16 tensors of one shape")
    if scale_layout not in {"row", "kgroup"}:
        raise ValueError(f"Unknown scale layout: {scale_layout!r}")
    if not gate.is_cuda or not mi355x_available(gate.device):
        raise RuntimeError("silu_mul_quant requires an MI355X (gfx950) GPU")
    i = int(gate.shape[-1])
    if i == 0:
        raise ValueError("Width must be positive")
    g2, u2 = gate.reshape(-1, i), up.reshape(-1, i)
    if g2.stride(-1) != 1 or u2.stride(-1) != 1 or g2.stride(0) != u2.stride(0):
        g2, u2 = g2.contiguous(), u2.contiguous()
    m = g2.shape[0]
    groups = (i + 127) // 128
    q = torch.empty((m, i), device=gate.device, dtype=torch.float8_e4m3fn)
    if scale_layout == "row":
        s = torch.empty((m, groups), device=gate.device, dtype=torch.float32)
        s_sm, s_sk = groups, 1
    else:
        mpad = max(64, -(-m // 64) * 64)
        s = torch.empty((groups, mpad), device=gate.device, dtype=torch.float32)[:, :m].t()
        s_sm, s_sk = 1, mpad
    h = torch.empty((m, i), device=gate.device, dtype=torch.bfloat16) if return_intermediate else None
    if m:
        _lib.check(_lib.load().mi355x_fp8_silu_mul_quant(
            g2.data_ptr(), u2.data_ptr(), _lib.DTYPE_BF16, m, i, g2.stride(0),
            None if h is None else h.data_ptr(), i, q.data_ptr(), i, i, s.data_ptr(), s_sm, s_sk,
            _stream_ptr(gate.device)))
    shape = tuple(gate.shape)
    q = q.reshape(shape)
    if h is not None:
        return h.reshape(shape), q, s
    return q, s


def _quant_outputs(m: int, k: int, device: torch.device, scale_layout: str):
    groups = (k + 127) // 128
    q = torch.empty((m, k), device=device, dtype=torch.float8_e4m3fn)
    if scale_layout == "row":
        s = torch.empty((m, groups), device=device, dtype=torch.float32)
        return q, s, groups, 1
    mpad = max(64, -(-m // 64) * 64)
    s = torch.empty((groups, mpad), device=device, dtype=torch.float32)[:, :m].t()
    return q, s, 1, mpad


def rmsnorm_quant_mi355x_fp8(x: torch.Tensor, weight: torch.Tensor, eps: float,
                             residual: torch.Tensor | None = None, *, scale_layout: str = "kgroup",
                             return_intermediate: bool = False):
    """Qwen3 RMSNorm (optionally after the residual add), quantized per row and 128-column
    group, in one kernel: the input side of the q/k/v and gate/up projections.

    The norm is the reference's rms_norm (engine/kernels/fused.py:89-124, 165-199):
    ``y = bf16(weight * bf16(x * rsqrt(mean(x^2) + eps)))``, with the row sum in PyTorch's
    reduction order and, with ``residual``, ``x`` replaced by ``bf16(x + residual)``.  The
    reciprocal square root is correctly rounded here (the reference's is libdevice's
    approximation), so y can differ from the reference in the last bf16 place.  The
    quantization is the activation quantizer's (sm89_fp8.py:304-332) applied to y.

    Returns ``(q, s)``, plus the residual sum ``bf16(x + residual)`` when ``residual`` is
    given; with ``return_intermediate`` the bf16 ``y`` comes first.
    """

    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("rmsnorm_quant takes bf16 activations and a bf16 norm weight")
    if scale_layout not in {"row", "kgroup"}:
        raise ValueError(f"Unknown scale layout: {scale_layout!r}")
    if not x.is_cuda or not mi355x_available(x.device):
        raise RuntimeError("rmsnorm_quant requires an MI355X (gfx950) GPU")
    k = int(x.shape[-1])
    if k % 4 or k < 128:
        raise ValueError("rms_norm reproduces PyTorch's vectorized reduction: width must be a multiple of 4, >= 128")
    if tuple(weight.shape) != (k,):
        raise ValueError("norm weight must have shape (width,)")
    x2 = x.reshape(-1, k)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    w1 = weight.contiguous()
    m = x2.shape[0]
    r2 = summed = None
    if residual is not None:
        if residual.shape != x.shape or residual.dtype != torch.bfloat16:
            raise ValueError("residual must be bf16 with the shape of x")
        r2 = residual.reshape(-1, k)
        if r2.stride(-1) != 1:
            r2 = r2.contiguous()
        summed = torch.empty((m, k), device=x.device, dtype=torch.bfloat16)
    q, s, s_sm, s_sk = _quant_outputs(m, k, x.device, scale_layout)
    y = torch.empty((m, k), device=x.device, dtype=torch.bfloat16) if return_intermediate else None
    if m:
        _lib.check(_lib.load().mi355x_fp8_rmsnorm_quant(
            x2.data_ptr(), _lib.DTYPE_BF16, m, k, x2.stride(0),
            None if r2 is None else r2.data_ptr(), 0 if r2 is None else r2.stride(0),
            None if summed is None else summed.data_ptr(), k, w1.data_ptr(), float(eps),
            None if y is None else y.data_ptr(), k, q.data_ptr(), k, k, s.data_ptr(), s_sm, s_sk,
            _stream_ptr(x.device)))
    shape = tuple(x.shape)
    out = [q.reshape(shape), s]
    if summed is not None:
        out.append(summed.reshape(shape))
    if y is not None:
        out.insert(0, y.reshape(shape))
    return tuple(out)


def rmsnorm_linear_mi355x_fp8(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, weight: torch.Tensor,
                              weight_scale_inv: torch.Tensor, residual: torch.Tensor | None = None,
                              output_dtype: torch.dtype | None = None):
    """``fp8_linear(rms_norm(x [+ residual]), weight)`` (the q/k/v or gate/up projection of a
    Qwen3 layer).  Returns the projection, plus the residual sum when ``residual`` is given.

    Up to 8 rows (bf16 in and out, K a multiple of 256 up to 2560) the norm, the activation
    quantizer and the GEMM run as one launch (the decode kernel recomputing the rows' norms);
    otherwise the norm and the quantizer run fused in one kernel and the GEMM in a second.
    Both give the same bits."""

    k = int(x.shape[-1])
    n = int(weight.shape[0])
    out_dtype = output_dtype or torch.bfloat16
    x2 = x.reshape(-1, k)
    if (out_dtype == torch.bfloat16 and x.dtype == torch.bfloat16 and norm_weight.dtype == torch.bfloat16
            and x2.shape[0] <= 8 and x2.stride(-1) == 1 and weight.dtype == torch.float8_e4m3fn
            and weight.stride(-1) == 1 and weight_scale_inv.dtype == torch.float32 and x.is_cuda
            and mi355x_available(x.device) and weight.device == x.device and weight_scale_inv.device == x.device
            and tuple(weight_scale_inv.shape) == (-(-n // 128), -(-k // 128)) and tuple(norm_weight.shape) == (k,)
            and (residual is None or (residual.shape == x.shape and residual.dtype == torch.bfloat16))):
        m = int(x2.shape[0])
        out = torch.empty((m, n), device=x.device, dtype=out_dtype)
        r2 = summed = None
        if residual is not None:
            r2 = residual.reshape(-1, k)
            if r2.stride(-1) != 1:
                r2 = r2.contiguous()
            summed = torch.empty((m, k), device=x.device, dtype=x.dtype)
        w1 = norm_weight.contiguous()
        lib = _lib.load()
        code = lib.mi355x_fp8_rmsnorm_linear(
            x2.data_ptr(), m, k, x2.stride(0), None if r2 is None else r2.data_ptr(), 0 if r2 is None else r2.stride(0),
            None if summed is None else summed.data_ptr(), k, w1.data_ptr(), float(eps), weight.data_ptr(),
            weight.stride(0), weight_scale_inv.data_ptr(), weight_scale_inv.stride(0), weight_scale_inv.stride(1),
            n, out.data_ptr(), out.stride(0), _stream_ptr(x.device))
        if code != _lib.ERR_UNSUPPORTED:
            _lib.check(code)
            out = out.reshape(*x.shape[:-1], n)
            return (out, summed.reshape(x.shape)) if residual is not None else out

    outs = rmsnorm_quant_mi355x_fp8(x, norm_weight, eps, residual)
    q, s = outs[0], outs[1]
    out = torch.empty((q.numel() // k, n), device=x.device, dtype=out_dtype)
    launch_block_gemm(q.reshape(-1, k), weight, out, s, weight_scale_inv)
    out = out.reshape(*x.shape[:-1], n)
    return (out, outs[2]) if residual is not None else out


def rmsnorm_gate_up_silu_mi355x_fp8(x: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                                    gate_up_weight: torch.Tensor, gate_up_scale: torch.Tensor,
                                    residual: torch.Tensor | None = None):
    """``silu_mul(*project_gate_up(rms_norm(x [+ residual])))``: the post-attention norm, the
    merged gate/up projection (weight rows: gate, then up) and SiLU(gate) * up, the input of
    the down projection.  Returns h [..., I] (bf16), plus the residual sum when ``residual`` is
    given.

    Up to 8 rows (bf16, K a multiple of 256 up to 2560) the three run as one launch, each
    workgroup owning matching gate and up weight rows; otherwise the norm-linear and the
    SiLU*up kernel run separately.  Both give the same bits: h = bf16(bf16(silu(g)) * u) on the
    projection's bf16 gate and up outputs, as ``silu_mul_quant_mi355x_fp8`` forms it."""

    k = int(x.shape[-1])
    n = int(gate_up_weight.shape[0])
    inter = n // 2
    x2 = x.reshape(-1, k)
    if (x.dtype == torch.bfloat16 and norm_weight.dtype == torch.bfloat16 and x2.shape[0] <= 8 and n % 2 == 0
            and x2.stride(-1) == 1 and gate_up_weight.dtype == torch.float8_e4m3fn and gate_up_weight.stride(-1) == 1
            and gate_up_scale.dtype == torch.float32 and x.is_cuda and mi355x_available(x.device)
            and gate_up_weight.device == x.device and gate_up_scale.device == x.device
            and tuple(gate_up_scale.shape) == (-(-n // 128), -(-k // 128)) and tuple(norm_weight.shape) == (k,)
            and (residual is None or (residual.shape == x.shape and residual.dtype == torch.bfloat16))):
        m = int(x2.shape[0])
        h = torch.empty((m, inter), device=x.device, dtype=torch.bfloat16)
        r2 = summed = None
        if residual is not None:
            r2 = residual.reshape(-1, k)
            if r2.stride(-1) != 1:
                r2 = r2.contiguous()
            summed = torch.empty((m, k), device=x.device, dtype=x.dtype)
        w1 = norm_weight.contiguous()
        code = _lib.load().mi355x_fp8_rmsnorm_gate_up_silu(
            x2.data_ptr(), m, k, x2.stride(0), None if r2 is None else r2.data_ptr(), 0 if r2 is None else r2.stride(0),
            None if summed is None else summed.data_ptr(), k, w1.data_ptr(), float(eps), gate_up_weight.data_ptr(),
            gate_up_weight.stride(0), gate_up_scale.data_ptr(), gate_up_scale.stride(0), gate_up_scale.stride(1),
            n, h.data_ptr(), h.stride(0), _stream_ptr(x.device))
        if code != _lib.ERR_UNSUPPORTED:
            _lib.check(code)
            h = h.reshape(*x.shape[:-1], inter)
            return (h, summed.reshape(x.shape)) if residual is not None else h

    outs = rmsnorm_linear_mi355x_fp8(x, norm_weight, eps, gate_up_weight, gate_up_scale, residual)
    gu = outs[0] if residual is not None else outs
    gu2 = gu.reshape(-1, n)
    h = silu_mul_quant_mi355x_fp8(gu2[:, :inter], gu2[:, inter:], return_intermediate=True)[0]
    h = h.reshape(*x.shape[:-1], inter)
    return (h, outs[1]) if residual is not None else h


def mlp_forward_mi355x_fp8(x: torch.Tensor, gate_up_weight: torch.Tensor, gate_up_scale: torch.Tensor,
                           down_weight: torch.Tensor, down_scale: torch.Tensor,
                           output_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Qwen3 MLP on FP8 weights: ``down(SiLU(gate) * up)`` with merged gate/up.

    The reference's _mlp_forward (engine/kernels/fused.py:280-283) runs merged gate_up ->
    silu_mul -> down_proj, quantizing the bf16 product again inside down_proj.  Here the
    SiLU-mul writes the quantized product directly (one kernel instead of silu_mul plus the
    down projection's quantizer); the codes are those the quantizer would give for the
    same bf16 product.
    """

    k = int(x.shape[-1])
    gate_up = mi355x_fp8_linear(x.reshape(-1, k), gate_up_weight, gate_up_scale, [128, 128])
    inter = gate_up.shape[-1] // 2
    q, s = silu_mul_quant_mi355x_fp8(gate_up[:, :inter], gate_up[:, inter:])
    out = torch.empty((q.shape[0], down_weight.shape[0]), device=x.device, dtype=output_dtype or x.dtype)
    if q.shape[0]:
        launch_block_gemm(q, down_weight if down_weight.stride(-1) == 1 else down_weight.contiguous(), out, s,
                          down_scale)
    return out.reshape(*x.shape[:-1], down_weight.shape[0])
