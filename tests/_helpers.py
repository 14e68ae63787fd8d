"""Shared test helpers: bridges between torch tensors and the numpy oracle."""

from __future__ import annotations

import numpy as np
import torch

import oracle


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def codes(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def oracle_quant(x: torch.Tensor):
    q, s = oracle.act_quant(bits16(x), is_fp16=x.dtype == torch.float16)
    return torch.from_numpy(q).view(torch.float8_e4m3fn), torch.from_numpy(s)


def oracle_linear(x: torch.Tensor, w: torch.Tensor, ws: torch.Tensor, out_dtype=None) -> torch.Tensor:
    out_dtype = out_dtype or x.dtype
    x2 = x.reshape(-1, x.shape[-1])
    out = oracle.linear(bits16(x2), codes(w), ws.detach().cpu().float().numpy(),
                        is_fp16=x.dtype == torch.float16, out_fp16=out_dtype == torch.float16)
    return torch.from_numpy(out.view(np.int16)).view(out_dtype).reshape(*x.shape[:-1], w.shape[0])


def oracle_gemm(q: torch.Tensor, a_s: torch.Tensor, w: torch.Tensor, ws: torch.Tensor, out_dtype=torch.bfloat16):
    out = oracle.block_gemm(codes(q), a_s.cpu().numpy(), codes(w), ws.cpu().float().numpy(),
                            out_fp16=out_dtype == torch.float16)
    return torch.from_numpy(out.view(np.int16)).view(out_dtype)


# Output tolerance of the block GEMM against the fp32 oracle: for every
# row, max |gpu - oracle| <= REL_TOL * max |oracle row|.  Infinities must match exactly.
REL_TOL = 1e-2


def assert_close_rows(actual: torch.Tensor, expected: torch.Tensor, rel: float = REL_TOL) -> dict:
    a = actual.detach().cpu().float().reshape(-1, actual.shape[-1])
    e = expected.detach().cpu().float().reshape(-1, expected.shape[-1])
    assert a.shape == e.shape
    inf = torch.isinf(e)
    assert torch.equal(torch.isinf(a), inf), "infinity positions differ"
    assert torch.equal(a[inf], e[inf]), "infinity signs differ"
    assert not torch.isnan(a).any(), "NaN in output"
    a = torch.where(inf, torch.zeros_like(a), a)
    e = torch.where(inf, torch.zeros_like(e), e)
    diff = (a - e).abs().amax(dim=1)
    scale = e.abs().amax(dim=1)
    bad = diff > rel * scale
    assert not bad.any(), (
        f"{int(bad.sum())} rows over tolerance; worst row {int((diff / scale.clamp_min(1e-30)).argmax())} "
        f"rel={float((diff / scale.clamp_min(1e-30)).max()):.3e}")
    exact = None
    if actual.dtype == expected.dtype and actual.element_size() == 2:
        exact = float((actual.detach().cpu().reshape(e.shape).view(torch.int16)
                       == expected.detach().cpu().reshape(e.shape).view(torch.int16)).float().mean())
    return {"max_rel": float((diff / scale.clamp_min(1e-30)).max()), "bit_identical_frac": exact}


# The GEMM folds each K group as acc = fma(partial, a_s * w_s, acc), one rounding of the
# scale product where the reference rounds (dot * a_s) * w_s twice; the oracle sums each
# group's dot exactly.  Both differences are fp32 roundings, so most bf16 outputs still
# match the oracle's bits; this is the floor the configuration tests hold that fraction to.
BIT_IDENTICAL_FLOOR = 0.95


def record_parity(name: str, stats: dict, floor: float = BIT_IDENTICAL_FLOOR) -> dict:
    """Prints the distance of a GEMM output from the oracle's bits (max row-relative error
    and the fraction of bf16 outputs bit-identical to the oracle's) as one PARITY line, and
    holds the fraction to ``floor``."""

    import sys

    frac = stats.get("bit_identical_frac")
    print(f"PARITY {name} max_rel={stats['max_rel']:.3e} bit_identical_frac="
          f"{'n/a' if frac is None else f'{frac:.5f}'}", flush=True, file=sys.stderr)
    if frac is not None:
        assert frac >= floor, f"{name}: only {frac:.4f} of the outputs equal the oracle's bits"
    return stats


def crafted_sumsq_rows(rows, width, bw):
    """Rows of 4096s (square 2^24) and +-1s whose fp32 sum of squares the reference's
    summation order fixes in closed form (engine/kernels/fused.py:95-115 and the tree of
    fused.py:61-75): thread t owns vectors t, t + bw, ...; element 4 v + q goes into its
    accumulator q; the four accumulators combine as ((a0 + a1) + a2) + a3; then the bw thread
    partials fold as s[t] += s[t + h] for h = bw/2, ..., 1.  Near 2^24 fp32 steps by 2, so
    2^24 + 1 rounds (to even) down to 2^24, 2^24 + 2 is exact and 2^24 + 3 rounds up to 2^24 + 4.

    * "tree": x[0] = 4096, x[4 t] = 1 for t = 1 .. bw-1 (one per thread).  The first fold adds
      thread bw/2's 1 to 2^24 and loses it; the later folds add 2, 4, ..., bw/2 exactly:
      2^24 + bw - 2.  Adding the ones one at a time (element order, or one running sum over
      the partials) loses all of them: 2^24.
    * "pairs": x[0] = 4096, x[4] = x[4 (1 + bw/2)] = 1.  Threads 1 and 1 + bw/2 meet in the
      first fold (2), which then reaches thread 0 whole: 2^24 + 2.  Folding neighbours
      first (t with t + 1) brings each 1 to 2^24 alone: 2^24.
    * "width": x[0] = 4096, x[4 (bw/2)] = x[4 (bw/2) + 1] = 1 (thread bw/2, accumulators 0
      and 1: partial 2): 2^24 + 2.  With bw/2 threads, vector bw/2 is thread 0's second
      vector and each 1 meets 2^24 alone: 2^24.
    * "combine" (when a thread owns two vectors): x[0] = 4096, x[1] = x[2] = x[3] = 1 and
      x[4 bw + 3] = 1, so a0 = 2^24, a1 = a2 = 1, a3 = 2: ((2^24 + 1) + 1) + 2 = 2^24 + 2.
      (a0 + a1) + (a2 + a3) and ((a3 + a2) + a1) + a0 give 2^24 + 4; one running sum per
      thread gives 2^24.
    """

    def row(entries):
        x = torch.zeros(rows, width, dtype=torch.bfloat16)
        for col, val in entries:
            x[:, col] = val
        return x

    b = 2.0 ** 24
    out = [("tree", row([(0, 4096.0)] + [(4 * t, 1.0) for t in range(1, bw)]), b + bw - 2),
           ("pairs", row([(0, 4096.0), (4, 1.0), (4 * (1 + bw // 2), -1.0)]), b + 2),
           ("width", row([(0, 4096.0), (4 * (bw // 2), 1.0), (4 * (bw // 2) + 1, 1.0)]), b + 2)]
    if width // 4 > bw:
        out.append(("combine", row([(0, 4096.0), (1, 1.0), (2, 1.0), (3, -1.0), (4 * bw + 3, 1.0)]), b + 2))
    return [(name, x, np.float32(v)) for name, x, v in out]


def _y0(sumsq, width, eps):
    """bf16 bits of y = bf16(1 * bf16(4096 * inv)) for a row whose sum of squares is sumsq, with
    inv = fl32(1 / sqrt(var + eps)) in double, var = fl32(sumsq * fl32(1 / width))."""

    var = np.float32(np.float32(sumsq) * np.float32(np.float32(1.0) / np.float32(width)))
    inv = np.float32(1.0 / np.sqrt(np.float64(np.float32(var + np.float32(eps)))))
    prod = np.float32(np.float32(4096.0) * inv)
    return int(torch.tensor(float(prod)).to(torch.bfloat16).view(torch.int16).item()) & 0xFFFF


def sumsq_eps_sweep(width, expect, name):
    """eps values around the one that puts 4096 * inv on the bf16 rounding midpoint 50.375,
    stepped by the fp32 spacing of var + eps there, such that for every plausible wrong order
    (sums 2^24, and 2^24 + 4 for the "combine" row) some eps in the sweep gives another y for
    the 4096 element than the closed-form sum does.  Asserts that and returns the sweep."""

    b = 2.0 ** 24
    wrong = [b] + ([b + 4] if name == "combine" else [])
    target = (4096.0 / 50.375) ** 2
    var = float(np.float32(np.float32(expect) * np.float32(np.float32(1.0) / np.float32(width))))
    ulp = float(np.spacing(np.float32(target)))
    eps = [float(np.float32(target - var + k * ulp / 2)) for k in range(-24, 25)]
    for alt in wrong:
        if np.float32(alt) == np.float32(expect):
            continue
        assert any(_y0(expect, width, e) != _y0(alt, width, e) for e in eps), (name, width, alt)
    return eps
