"""The no-allocation entry point mi355x_fp8_linear_noalloc, through the C-ABI.

It must give the bits of mi355x_fp8_linear (the workspace entry point) on the same inputs,
on two calls in a row (the second smaller, so stale scratch contents from the first call
would show), allocate no torch memory, and reject a call larger than its static scratch
before launching anything.
"""

import sys

import pytest
import torch

from minillm_amd import _lib
from minillm_amd import mi355x_fp8 as fp8
from minillm_amd.validation import ModelShape, bit_mismatch_details, bitwise_equal, make_activations, make_weights

pytestmark = pytest.mark.gpu


def _one_launch_form(m, k):
    """Whether mi355x_fp8_linear may run the call as one launch (the decode kernel quantizing
    its own K groups), which leaves the workspace, and so the scratch, untouched: that form
    needs at most 16 rows and K % 16 == 0 (launch_linear_stream)."""

    return m <= 16 and k % 16 == 0


def _noalloc(x, w, ws, out, config=_lib.CONFIG_AUTO):
    m, k = x.shape
    stream = torch.cuda.current_stream(x.device).cuda_stream
    return _lib.load().mi355x_fp8_linear_noalloc(
        x.data_ptr(), _lib.DTYPE_BF16 if x.dtype == torch.bfloat16 else _lib.DTYPE_F16, m, k, x.stride(0),
        x.stride(1), w.data_ptr(), w.stride(0), ws.data_ptr(), ws.stride(0), ws.stride(1), w.shape[0],
        out.data_ptr(), _lib.DTYPE_BF16 if out.dtype == torch.bfloat16 else _lib.DTYPE_F16, out.stride(0), config,
        stream)


# Every call takes the two-launch form (quantizer into the scratch, then the GEMM from it),
# the second with fewer rows than the first, so stale scratch rows would show.
@pytest.mark.parametrize("first,second", [((2048, 2560, 9728), (40, 2560, 9728)),
                                          ((536, 19456, 2560), (24, 6144, 2560)),
                                          ((300, 193, 259), (7, 129, 127)),
                                          ((64, 2560, 4096), (17, 2560, 4096))])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_noalloc_equals_workspace_entry_twice(gpu, first, second, dtype):
    print("CASE noalloc", first, second, dtype, flush=True, file=sys.stderr)
    lib = _lib.load()
    assert lib.mi355x_fp8_linear_noalloc_scratch_bytes() == _lib.NOALLOC_SCRATCH_BYTES
    cases = []
    for i, (m, n, k) in enumerate((first, second)):
        assert not _one_launch_form(m, k) and lib.mi355x_fp8_linear_workspace_bytes(m, n, k, 0) > 0
        x = make_activations(m, k, 30 + i, dtype).to(gpu)
        w, ws = make_weights(ModelShape("noalloc", n, k), 30 + i)
        cases.append((x, w.to(gpu), ws.to(gpu)))
    outs = [torch.full((x.shape[0], w.shape[0]), float("nan"), dtype=dtype, device=gpu) for x, w, _ in cases]
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated(gpu)
    for (x, w, ws), out in zip(cases, outs):
        _lib.check(_noalloc(x, w, ws, out))
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated(gpu) == before
    for (x, w, ws), out in zip(cases, outs):
        ref = fp8.mi355x_fp8_linear(x, w, ws, [128, 128])
        assert bitwise_equal(out, ref), bit_mismatch_details(out, ref)


def test_noalloc_rejects_calls_beyond_the_scratch(gpu):
    lib = _lib.load()
    m, k, n = 4096, 9728, 256  # q alone is 39.8 MB > 24 MiB
    assert lib.mi355x_fp8_linear_workspace_bytes(m, n, k, 0) > _lib.NOALLOC_SCRATCH_BYTES
    x = torch.zeros((m, k), dtype=torch.bfloat16, device=gpu)
    w = torch.zeros((n, k), dtype=torch.uint8, device=gpu).view(torch.float8_e4m3fn)
    ws = torch.ones((2, 76), dtype=torch.float32, device=gpu)
    out = torch.full((m, n), 7.0, dtype=torch.bfloat16, device=gpu)
    assert _noalloc(x, w, ws, out) == _lib.ERR_SCRATCH
    with pytest.raises(ValueError, match="scratch"):
        _lib.check(_lib.ERR_SCRATCH)
    torch.cuda.synchronize()
    assert (out == 7.0).all().item()  # nothing was launched


def test_noalloc_under_hip_graph_capture(gpu):
    """The no-allocation entry point captured in a HIP graph (the caller it exists for): every
    replay, with eager work and synchronisations between them, gives the eager result."""

    print("CASE noalloc graph", flush=True, file=sys.stderr)
    # 32 rows: the two-launch form, so the captured quantizer writes the scratch and the
    # captured GEMM reads it.
    assert not _one_launch_form(32, 2560)
    x = make_activations(32, 2560, 41).to(gpu)
    w, ws = make_weights(ModelShape("noalloc_graph", 6144, 2560), 41)
    w, ws = w.to(gpu), ws.to(gpu)
    ref = fp8.mi355x_fp8_linear(x, w, ws, [128, 128])
    out = torch.full_like(ref, float("nan"))
    stream = torch.cuda.Stream(gpu)
    with torch.cuda.stream(stream):
        _lib.check(_noalloc(x, w, ws, out))  # first call on the device outside capture
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            _lib.check(_noalloc(x, w, ws, out))
    for _ in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert bitwise_equal(out, ref), bit_mismatch_details(out, ref)
        # unrelated eager work between replays, through the same scratch
        other = torch.empty_like(ref)
        _lib.check(_noalloc(x[:17], w, ws, other[:17]))
        torch.cuda.synchronize()
        assert bitwise_equal(other[:17], ref[:17]), bit_mismatch_details(other[:17], ref[:17])


_FIRST_CALL_UNDER_CAPTURE = r"""
import sys
sys.path.insert(0, sys.argv[1])
import torch
from minillm_amd import _lib
from minillm_amd import mi355x_fp8 as fp8
from minillm_amd.validation import ModelShape, bitwise_equal, make_activations, make_weights
dev = torch.device("cuda:0")
lib = _lib.load()
x = make_activations(32, 2560, 43).to(dev)
w, ws = make_weights(ModelShape("noalloc_first", 6144, 2560), 43)
w, ws = w.to(dev), ws.to(dev)
ref = fp8.mi355x_fp8_linear(x, w, ws, [128, 128])
out = torch.full_like(ref, float("nan"))
stream = torch.cuda.Stream(dev)
lib.mi355x_fp8_linear_noalloc_scratch_bytes()  # the documented set-up call, outside capture
torch.cuda.synchronize()
with torch.cuda.stream(stream):
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        _lib.check(lib.mi355x_fp8_linear_noalloc(
            x.data_ptr(), _lib.DTYPE_BF16, 32, 2560, x.stride(0), 1, w.data_ptr(), w.stride(0), ws.data_ptr(),
            ws.stride(0), ws.stride(1), 6144, out.data_ptr(), _lib.DTYPE_BF16, out.stride(0), 0,
            stream.cuda_stream))
for _ in range(3):
    out.fill_(float("nan"))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert bitwise_equal(out, ref)
print("first-call-under-capture ok", flush=True)
"""


def test_noalloc_first_call_of_the_process_under_capture(gpu, tmp_path):
    """In a fresh process, after only the set-up call, the first no-allocation call is made
    under HIP-graph capture; the graph's replays give the workspace entry point's bits."""

    import os
    import subprocess

    print("CASE noalloc first call under capture (subprocess)", flush=True, file=sys.stderr)
    pkg = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "mini-inference-engine_amd")
    script = tmp_path / "first_call.py"
    script.write_text(_FIRST_CALL_UNDER_CAPTURE)
    proc = subprocess.run([sys.executable, str(script), pkg], capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "first-call-under-capture ok" in proc.stdout
