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
