"""Pins the CPU oracle (oracle/fp8_oracle.c) against independent checks.

Nothing here re-types the oracle's formulas: each check compares it with a library
routine (torch's float8_e4m3fn / bfloat16 / float16 casts), a definition (the OCP e4m3fn
code table), the reference tests' invariants for special rows, exact power-of-two
scaling laws, an fp64 dense product with a rounding-error bound, or brute force on tiny
shapes.
"""

import numpy as np
import pytest
import torch

import oracle
from minillm_amd.validation import ModelShape, TAIL_SHAPES, make_activations, make_weights
from _helpers import bits16, codes, crafted_sumsq_rows, sumsq_eps_sweep


# ---------------------------------------------------------------------------- formats

def test_e4m3_encode_matches_torch_over_fp32_patterns():
    # Every exponent and the top 8 mantissa bits (which contain the e4m3 rounding bit and
    # the first sticky bits), crossed with low-bit patterns that decide ties and sticky.
    hi = np.arange(1 << 17, dtype=np.uint32) << 15
    lows = np.array([0, 1, 0x3FFF, 0x4000, 0x4001, 0x7FFF, 0x1234, 0x5A5A], dtype=np.uint32)
    f = (hi[:, None] | lows[None, :]).ravel().view(np.float32)
    f = f[np.isfinite(f) & (np.abs(f) < 464)]
    ours = oracle.f32_to_e4m3(f)
    ref = torch.from_numpy(f.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert f.size > 500_000
    assert np.array_equal(ours, ref)


def test_e4m3_encode_rounding_midpoints_and_saturation():
    # Exact midpoints between neighbouring codes round to the even code.
    values = oracle.e4m3_to_f32(np.arange(0x7E, dtype=np.uint8))  # positive finite codes
    mids = ((values[:-1].astype(np.float64) + values[1:]) / 2).astype(np.float32)
    got = oracle.f32_to_e4m3(mids)
    below, above = np.arange(0x7D), np.arange(1, 0x7E)
    expect = np.where(below % 2 == 0, below, above).astype(np.uint8)
    assert np.array_equal(got, expect)
    # |v| in (448, 464) rounds to 448; larger values saturate (satfinite) to 448.
    assert list(oracle.f32_to_e4m3(np.array([448.0, 463.9, 1e6, -500.0], np.float32))) == [0x7E, 0x7E, 0x7E, 0xFE]
    assert list(oracle.f32_to_e4m3(np.array([0.0, -0.0, 2.0 ** -10, -(2.0 ** -10) * 1.5], np.float32))) == [0, 0x80, 0, 0x81]


def test_e4m3_decode_table_is_the_ocp_definition():
    table = oracle.e4m3_to_f32(np.arange(256, dtype=np.uint8))
    ref = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    finite = ~np.isnan(ref)
    assert np.array_equal(np.isnan(table), np.isnan(ref))
    assert np.array_equal(table[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert table[0x7E] == 448.0 and table[0x01] == 2.0 ** -9 and table[0x08] == 2.0 ** -6


def test_bf16_and_f16_rounding_match_torch():
    rng = np.random.default_rng(0)
    f = (rng.standard_normal(200_000) * np.exp(rng.uniform(-30, 30, 200_000))).astype(np.float32)
    f = np.concatenate([f, np.array([65504.0, 65520.0, 1e9, -0.0, 2.0 ** -25, 5.96e-8], np.float32)])
    lib = oracle.lib()
    bf = np.array([lib.orc_f32_to_bf16(float(v)) for v in f[:20000]], dtype=np.uint16)
    assert np.array_equal(bf, torch.from_numpy(f[:20000].copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
    h = np.array([lib.orc_f32_to_f16(float(v)) for v in f[-20000:]], dtype=np.uint16)
    assert np.array_equal(h, torch.from_numpy(f[-20000:].copy()).to(torch.float16).view(torch.int16).numpy().view(np.uint16))


# ---------------------------------------------------------------------------- quantizer

def test_quantizer_reference_special_rows():
    """Invariants of the reference's tests (test_sm89_fp8_exact.py:55-63 and the special
    rows of sm89_fp8_validation.py:58-70)."""

    x = make_activations(7, 259, 42)
    q, s = oracle.act_quant(bits16(x))
    assert not s[1].any() and not q[1].any()                  # zero row: +0 scales, +0 codes
    assert (s[3] < 1e-12).all()                               # tiny row: scale below the clamp
    assert (q[5] == 0x80).all()                               # -0.0 row keeps the sign
    assert set(q[6].tolist()) == {0x7E, 0xFE} and (s[6] == 1.0).all()
    assert not q[4, :128].any() and s[4, 0] == 0              # zero group then a tiny group
    for row in range(7):                                      # row independence
        q1, s1 = oracle.act_quant(bits16(x[row:row + 1]))
        assert np.array_equal(q1, q[row:row + 1]) and np.array_equal(s1, s[row:row + 1])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("k", [1, 127, 128, 259, 2560])
def test_quantizer_closed_form_properties(dtype, k):
    x = make_activations(9, k, 7, dtype)
    q, s = oracle.act_quant(bits16(x), is_fp16=dtype == torch.float16)
    xf = x.float().numpy()
    g = (k + 127) // 128
    pad = np.zeros((9, g * 128), np.float32)
    pad[:, :k] = xf
    amax = np.abs(pad.reshape(9, g, 128)).max(-1)
    # The scale is amax / 448 rounded once to fp32 (numpy's float32 division is IEEE).
    assert np.array_equal(s, (amax / np.float32(448.0)).astype(np.float32))
    deq = oracle.e4m3_to_f32(q).reshape(9, k).astype(np.float64)
    den = np.maximum(s, np.float32(1e-12)).repeat(128, 1)[:, :k].astype(np.float64)
    t = xf / den
    # The element holding the group maximum lands on +-448 (or +-0 for a zero group) ...
    for m in range(9):
        for gi in range(g):
            seg = np.abs(t[m, gi * 128:(gi + 1) * 128])
            if s[m, gi] >= 1e-12 and seg.size:
                assert np.abs(deq[m, gi * 128 + seg.argmax()]) == 448.0
    # ... and every code is within half an e4m3 ulp of x / scale (relative 2^-4, or the
    # subnormal spacing 2^-10 absolute).
    err = np.abs(deq - t)
    bound = np.maximum(np.abs(t) * 2.0 ** -4, 2.0 ** -10) + 1e-12
    assert (err <= bound).all()


# ---------------------------------------------------------------------------- GEMM

def _dense_fp64(q, s, w, ws, k):
    a = oracle.e4m3_to_f32(q).astype(np.float64) * np.repeat(s, 128, 1)[:, :k]
    b = oracle.e4m3_to_f32(w).astype(np.float64) * np.repeat(np.repeat(ws, 128, 0), 128, 1)[:w.shape[0], :k]
    return a @ b.T, np.abs(a) @ np.abs(b).T


@pytest.mark.parametrize("shape", TAIL_SHAPES + (ModelShape("kv", 256, 2560),), ids=lambda s: s.name)
def test_gemm_against_fp64_with_rounding_bound(shape):
    x = make_activations(11, shape.k, 5)
    w, ws = make_weights(shape, 5)
    q, s = oracle.act_quant(bits16(x))
    out = oracle.block_gemm(q, s, codes(w), ws.numpy())
    got = torch.from_numpy(out.view(np.int16)).view(torch.bfloat16).float().numpy().astype(np.float64)
    exact, mag = _dense_fp64(q, s, codes(w), ws.numpy(), shape.k)
    groups = (shape.k + 127) // 128
    # fp32 rounding of G group sums, 2 scale products and G additions, then one bf16 rounding.
    bound = (3 * groups + 4) * 2.0 ** -24 * mag + 2.0 ** -8 * np.abs(exact) + 1e-30
    assert (np.abs(got - exact) <= bound).all()


def test_gemm_scaling_laws_pin_scale_indices():
    """Doubling one activation scale doubles exactly that output row; doubling one weight
    block scale doubles exactly those 128 output columns and only through that K group, so
    a transposed or mis-indexed scale fails."""

    shape = ModelShape("t", 300, 384)
    x = make_activations(6, shape.k, 9)
    w, ws = make_weights(shape, 9)
    q, s = oracle.act_quant(bits16(x))
    wc, wsn = codes(w), ws.numpy()
    base = oracle.block_gemm(q, s, wc, wsn).view(np.int16)
    s2 = s.copy()
    s2[3, :] *= 2
    out = oracle.block_gemm(q, s2, wc, wsn)
    b = torch.from_numpy(base).view(torch.bfloat16).float()
    o = torch.from_numpy(out.view(np.int16)).view(torch.bfloat16).float()
    assert torch.equal(o[3], 2 * b[3]) and torch.equal(o[[0, 1, 2, 4, 5]], b[[0, 1, 2, 4, 5]])
    ws2 = wsn.copy()
    ws2[1, :] *= 4  # weight block row 1 = output columns 128..255, every K group
    o2 = torch.from_numpy(oracle.block_gemm(q, s, wc, ws2).view(np.int16)).view(torch.bfloat16).float()
    assert torch.equal(o2[:, 128:256], 4 * b[:, 128:256])
    assert torch.equal(o2[:, :128], b[:, :128]) and torch.equal(o2[:, 256:], b[:, 256:])


def test_gemm_brute_force_tiny():
    """Pure-Python evaluation of the reference expression on a tiny tail shape."""

    shape = ModelShape("tiny", 5, 259)
    x = make_activations(3, shape.k, 17)
    w, ws = make_weights(shape, 17)
    q, s = oracle.act_quant(bits16(x))
    out = oracle.block_gemm(q, s, codes(w), ws.numpy())
    qv = oracle.e4m3_to_f32(q)
    wv = oracle.e4m3_to_f32(codes(w))
    f32 = np.float32
    for m in range(3):
        for n in range(shape.n):
            acc = f32(0)
            for kb in range(3):
                lo, hi = kb * 128, min(shape.k, kb * 128 + 128)
                dot = f32(sum(float(qv[m, k]) * float(wv[n, k]) for k in range(lo, hi)))
                acc = f32(acc + f32(f32(dot * s[m, kb]) * ws.numpy()[n // 128, kb]))
            expect = torch.tensor([float(acc)]).to(torch.bfloat16).view(torch.int16).item() & 0xFFFF
            assert int(out[m, n]) == expect, (m, n)


def test_linear_row_independence_and_fp16_output():
    shape = TAIL_SHAPES[2]
    x = make_activations(8, shape.k, 3)
    w, ws = make_weights(shape, 3)
    full = oracle.linear(bits16(x), codes(w), ws.numpy())
    for row in (0, 2, 7):
        assert np.array_equal(oracle.linear(bits16(x[row:row + 1]), codes(w), ws.numpy()), full[row:row + 1])
    h = oracle.linear(bits16(x), codes(w), ws.numpy(), out_fp16=True)
    hf = torch.from_numpy(h.view(np.int16)).view(torch.float16).float()
    bf = torch.from_numpy(full.view(np.int16)).view(torch.bfloat16).float()
    finite = torch.isfinite(hf)
    assert torch.allclose(hf[finite], bf[finite], rtol=2 ** -7, atol=1e-3)


def test_silu_mul_matches_torch_bf16_semantics():
    """The reference's silu_mul is PyTorch's bf16 F.silu(g) * u (fused.py:135-137):
    torch on CPU computes silu in fp32 and rounds to bf16, then multiplies in bf16."""

    gen = torch.Generator().manual_seed(3)
    g = (torch.randn(4096, generator=gen) * 4).to(torch.bfloat16)
    u = (torch.randn(4096, generator=gen) * 2).to(torch.bfloat16)
    g[:6] = torch.tensor([0.0, -0.0, 88.0, -88.0, 1e-30, -100.0]).to(torch.bfloat16)
    ours = oracle.silu_mul(bits16(g), bits16(u))
    ref = bits16(torch.nn.functional.silu(g) * u)
    ulps = np.abs(ours.astype(np.int32) - ref.astype(np.int32))
    assert ulps.max() <= 1 and (ulps == 0).mean() > 0.99


# ---- RMSNorm (reference engine/kernels/fused.py:89-124, 165-214) -------------------------

def test_rmsnorm_block_width_known_values():
    """The reference's _torch_reduce_block_width at the widths Qwen3 uses (worked by hand
    from its formula: dim0 = width / 4 vectors, 512-thread blocks, 32-wide warps)."""

    for rows, width, bw in [(1, 2560, 512), (2, 2560, 256), (4, 2560, 128), (8, 2560, 64), (16, 2560, 32),
                            (2048, 2560, 32), (1, 128, 32), (64, 128, 32), (1, 256, 64), (3, 1024, 256)]:
        assert oracle.rmsnorm_block_width(rows, width) == bw, (rows, width)


def _bf16_bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_rmsnorm_closed_forms():
    """Rows whose sum of squares is exact in any order: the result is then fixed by the
    formula alone (y = bf16(w * bf16(x * fl(1/sqrt(var + eps)))))."""

    eps = np.float32(1e-6)
    for width in (128, 2560):
        w = (torch.arange(width) % 7 * 0.25 + 0.5).to(torch.bfloat16)
        for c in (2.0, -0.5, 3.0):
            x = torch.full((3, width), c, dtype=torch.bfloat16)
            y, _ = oracle.rmsnorm(_bf16_bits(x), _bf16_bits(w), float(eps))
            ss = np.float32(c * c * width)                      # exact
            var = np.float32(ss * np.float32(np.float32(1.0) / np.float32(width)))
            inv = np.float32(1.0 / np.sqrt(np.float64(np.float32(var + eps))))
            normed = torch.tensor(np.float32(c) * inv, dtype=torch.float32).to(torch.bfloat16).float()
            expect = (w.float() * normed).to(torch.bfloat16)
            assert np.array_equal(y[0], _bf16_bits(expect)) and np.array_equal(y[2], y[0])
        # One non-zero element: ss = a^2 exactly.
        x = torch.zeros(1, width, dtype=torch.bfloat16)
        x[0, 5] = 12.0
        y, _ = oracle.rmsnorm(_bf16_bits(x), _bf16_bits(w), float(eps))
        var = np.float32(np.float32(144.0) * np.float32(np.float32(1.0) / np.float32(width)))
        inv = np.float32(1.0 / np.sqrt(np.float64(np.float32(var + eps))))
        normed = torch.tensor(np.float32(12.0) * inv).to(torch.bfloat16).float()
        assert y[0, 5] == _bf16_bits((w[5].float() * normed).to(torch.bfloat16).reshape(1))[0]
        assert (y[0, np.arange(width) != 5] & 0x7FFF).max() == 0   # zeros stay zero


def test_rmsnorm_summation_order_closed_forms():
    """The oracle's sum of squares on rows that make each part of the reference's order
    visible (see _helpers.crafted_sumsq_rows), at block widths 512, 256, 32 (rows 1, 2, 16 of 2560),
    256 (3 rows of 1024) and 32 (one row of 128)."""

    for rows, width in [(1, 2560), (2, 2560), (16, 2560), (3, 1024), (1, 128)]:
        bw = oracle.rmsnorm_block_width(rows, width)
        for name, x, expect in crafted_sumsq_rows(rows, width, bw):
            got = oracle.rmsnorm_sumsq(_bf16_bits(x))
            assert np.array_equal(got, np.full(rows, expect, np.float32)), (name, rows, width, got[0], expect)
        # The eps sweep the GPU test runs over these rows separates each closed-form sum from
        # the sums the plausible other orders give (see sumsq_eps_sweep).
        for name, x, expect in crafted_sumsq_rows(rows, width, bw):
            sumsq_eps_sweep(width, expect, name)
        # Sums that are exact in any order: the order cannot matter.
        x = torch.full((rows, width), 3.0, dtype=torch.bfloat16)
        assert np.array_equal(oracle.rmsnorm_sumsq(_bf16_bits(x)), np.full(rows, 9.0 * width, np.float32))


def test_rmsnorm_matches_torch_within_one_ulp_and_residual_sum_is_exact():
    """Against torch's CPU Qwen3RMSNorm (its own summation order): within one bf16 ulp, and
    bitwise almost everywhere; the residual add is bitwise torch's bf16 add."""

    gen = torch.Generator().manual_seed(5)
    eps = 1e-6
    for rows, width in [(1, 2560), (8, 2560), (33, 2560), (4, 4096), (16, 132)]:
        x = (torch.randn(rows, width, generator=gen) * 3).to(torch.bfloat16)
        r = (torch.randn(rows, width, generator=gen)).to(torch.bfloat16)
        w = (torch.rand(width, generator=gen) + 0.5).to(torch.bfloat16)
        y, summed = oracle.rmsnorm(_bf16_bits(x), _bf16_bits(w), eps, _bf16_bits(r))
        s_ref = x + r
        assert np.array_equal(summed, _bf16_bits(s_ref))
        h = s_ref.float()
        ref = w * (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)).to(torch.bfloat16)
        diff = np.abs(y.astype(np.int32) - _bf16_bits(ref).astype(np.int32))
        assert diff.max() <= 1 and (diff == 0).mean() > 0.99, (rows, width, diff.max(), (diff == 0).mean())
    with pytest.raises(ValueError):
        oracle.rmsnorm(np.zeros((2, 130), np.uint16), np.zeros(130, np.uint16), 1e-6)
