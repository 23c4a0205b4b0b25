"""Shared test helpers: seeded masks and the dense-conv (torch fp64) check.

The dense check is independent of the oracle's gather formula: it scatters the
kept tokens into a zero-filled [B*T, C, H, W] grid, runs ``F.conv2d`` with
``padding=1`` (the reference's own dense ``2d_conv`` adapter path,
opentad/models/backbones/vit_sparse_adapter_poguise.py:372-412,484-490) and
gathers the kept cells back. Gradients come from torch autograd of the same
expression.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F


def random_mask(rng: np.random.Generator, B, T, H, W, keep: float) -> np.ndarray:
    """Keep cells uniformly at random; per frame exactly round(keep*H*W)."""
    m = np.zeros((B, T, H * W), dtype=np.uint8)
    k = int(round(keep * H * W))
    for b in range(B):
        for t in range(T):
            m[b, t, rng.permutation(H * W)[:k]] = 1
    return m.reshape(B, T, H, W)


def topk_mask(rng: np.random.Generator, B, T, H, W, keep: float) -> np.ndarray:
    """Per sample keep ceil(keep*T*H*W) cells by top-k of a U(0,1) score
    (keep-set rule of vit_sparse_adapter_poguise.py:763,785-787)."""
    n = T * H * W
    k = math.ceil(keep * n)
    score = rng.random((B, n))
    m = np.zeros((B, n), dtype=np.uint8)
    idx = np.argsort(-score, axis=1, kind="stable")[:, :k]
    np.put_along_axis(m, idx, 1, axis=1)
    return m.reshape(B, T, H, W)


def w_std(w: torch.Tensor) -> torch.Tensor:
    """(9, C_in, C_out) -> (C_out, C_in, 3, 3) with k = ky*3 + kx
    (sparse_conv_layer.py:150-156)."""
    nine, ci, co = w.shape
    return w.permute(2, 1, 0).reshape(co, ci, 3, 3)


def dense_reference(mask: np.ndarray, x: np.ndarray, w: np.ndarray, bias, go: np.ndarray,
                    depthwise: bool = False):
    """Dense fp64 conv on the zero-filled grid. Returns (y, gi, gw, gb) as numpy fp64.

    ``x``/``go`` rows are the kept cells in flattened B*T*H*W order; ``w`` is
    (9, C_in, C_out) or (9, C) for depthwise."""
    B, T, H, W = mask.shape
    flat = torch.from_numpy(np.flatnonzero(mask.reshape(-1)))
    C = x.shape[1]
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    grid = torch.zeros(B * T * H * W, C, dtype=torch.float64)
    grid = grid.index_copy(0, flat, xt)
    grid = grid.view(B * T, H, W, C).permute(0, 3, 1, 2)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    if depthwise:
        wk = wt.permute(1, 0).reshape(C, 1, 3, 3)
        groups = C
    else:
        wk = w_std(wt)
        groups = 1
    bt = torch.tensor(bias, dtype=torch.float64, requires_grad=True) if bias is not None else None
    y = F.conv2d(grid, wk, bt, padding=1, groups=groups)
    y = y.permute(0, 2, 3, 1).reshape(B * T * H * W, -1).index_select(0, flat)
    y.backward(torch.tensor(go, dtype=torch.float64))
    gb = bt.grad.numpy() if bt is not None else None
    return y.detach().numpy(), xt.grad.numpy(), wt.grad.numpy(), gb


def kaiming_weight(rng: np.random.Generator, ci: int, co: int) -> np.ndarray:
    """Kaiming-uniform(a=sqrt(5)) on a (C_out, C_in, 3, 3) tensor, re-laid out to
    (9, C_in, C_out) (sparse_conv_layer.py:145-161)."""
    fan_in = ci * 9
    bound = 1.0 / math.sqrt(fan_in)  # gain*sqrt(3/fan_in) with a=sqrt(5)
    t = rng.uniform(-bound, bound, size=(co, ci, 3, 3)).astype(np.float32)
    return np.ascontiguousarray(t.reshape(co, ci, 9).transpose(2, 1, 0))


def assert_rounded_once(got, exact, abs_sum, dt):
    """got (float16 / bfloat16 / float32) against the exact result (fp64):
    every element within one unit in the last place of the exact value
    rounded to got's dtype, plus an fp32 accumulation allowance of 2^-20 x
    the element's sum of absolute terms (abs_sum): a single rounding of an
    fp32 sum. Rounding after each of several contributions, as an atomic
    pass into the 16-bit output does, drifts by more."""
    import torch

    g = got.detach().cpu().double()
    ex = torch.from_numpy(np.ascontiguousarray(exact)).double()
    allow = torch.from_numpy(np.ascontiguousarray(abs_sum)).double() * 2.0 ** -20
    if dt in (torch.float32, torch.float64):
        bar = 1e-5 if dt == torch.float32 else 1e-12
        assert float((g - ex).abs().max()) <= bar * float(ex.abs().max())
        return
    mant = 10 if dt == torch.float16 else 7
    r = ex.to(dt).double()
    ulp = torch.ldexp(torch.ones_like(r), torch.frexp(r.abs().clamp_min(2.0 ** -14)).exponent - 1 - mant)
    bad = (g - r).abs() > ulp + allow
    if bad.any():
        idx = tuple(int(v) for v in bad.nonzero()[0])
        print("  off by more than one ulp:", int(bad.sum()), "first at", idx, "got", float(g[idx]), "exact",
              float(ex[idx]), "ulp", float(ulp[idx]), flush=True)
    assert not bad.any()
