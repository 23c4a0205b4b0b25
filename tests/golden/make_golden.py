"""Writes the golden fixtures under tests/golden/ (run from the repository root:
``python tests/golden/make_golden.py``).

The reference repository ships no golden vectors for SparseConv2D (its tests are
end-to-end scripts only), so these fixtures are derived from sources that do
not share code with the oracle or the HIP kernels:

* neighbor tables: a direct numpy restatement of the reference's own table
  procedures (get_initial_neighbor_indices, then the Block remap after each
  sorted top-k prune; opentad/models/backbones/vit_sparse_adapter_poguise.py
  :1623-1670 and :913-977), driven step by step;
* convolution outputs and gradients: torch float64 ``F.conv2d(padding=1)`` on
  the kept tokens scattered into a zero-filled dense grid, and its autograd
  (the reference's dense ``2d_conv`` adapter path,
  vit_sparse_adapter_poguise.py:372-412,484-490).

Inputs are multiples of 1/8 with small magnitude, exactly representable in
float16 and bfloat16, so every dtype sees the same inputs.
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))


def initial_table(h, w, T, B):
    """get_initial_neighbor_indices restated (numpy, int64)."""
    idx = np.arange(h * w).reshape(h, w)
    pad = np.full((h + 2, w + 2), -1, dtype=np.int64)
    pad[1:-1, 1:-1] = idx
    cols = [pad[1 + dy:1 + dy + h, 1 + dx:1 + dx + w].reshape(-1) for dy in (-1, 0, 1) for dx in (-1, 0, 1)]
    sp = np.stack(cols, 1)
    t = np.concatenate([np.where(sp >= 0, sp + f * h * w, -1) for f in range(T)], 0)
    return np.stack([np.where(t >= 0, t + b * T * h * w, -1) for b in range(B)], 0)


def remap(table, keep):
    """Block remap restated: keep rows, map old global -> new global."""
    B, n_prev, _ = table.shape
    n_new = keep.shape[1]
    kept = np.stack([table[b][keep[b]] for b in range(B)], 0)
    mapping = np.full(B * n_prev, -1, dtype=np.int64)
    for b in range(B):
        mapping[b * n_prev + keep[b]] = b * n_new + np.arange(n_new)
    return np.where(kept != -1, mapping[np.clip(kept, 0, None)], -1)


def eighths(rng, shape, lim=16):
    return (rng.integers(-lim, lim + 1, size=shape) / 8.0).astype(np.float32)


def dense(mask, x, w, b, go, depthwise=False):
    B, T, H, W = mask.shape
    flat = torch.from_numpy(np.flatnonzero(mask.reshape(-1)))
    C = x.shape[1]
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    grid = torch.zeros(B * T * H * W, C, dtype=torch.float64).index_copy(0, flat, xt)
    grid = grid.view(B * T, H, W, C).permute(0, 3, 1, 2)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    if depthwise:
        wk, groups = wt.permute(1, 0).reshape(C, 1, 3, 3), C
    else:
        co = w.shape[2]
        wk, groups = wt.permute(2, 1, 0).reshape(co, C, 3, 3), 1
    bt = torch.tensor(b, dtype=torch.float64, requires_grad=True)
    y = F.conv2d(grid, wk, bt, padding=1, groups=groups)
    y = y.permute(0, 2, 3, 1).reshape(B * T * H * W, -1).index_select(0, flat)
    y.backward(torch.tensor(go, dtype=torch.float64))
    return y.detach().numpy(), xt.grad.numpy(), wt.grad.numpy(), bt.grad.numpy()


def main():
    rng = np.random.default_rng(20261201)
    out = {}

    # 1. initial table of a 5x7 grid, 3 frames, 2 samples (global indices)
    out["table_initial"] = dict(h=np.int64(5), w=np.int64(7), T=np.int64(3), B=np.int64(2),
                                table=initial_table(5, 7, 3, 2).astype(np.int32))

    # 2. two sorted top-k prunes (keep 0.7 then 0.5) of a 2 x 4 x 6 x 6 grid
    B, T, H, W = 2, 4, 6, 6
    table = initial_table(H, W, T, B)
    mask = np.ones((B, T * H * W), dtype=bool)
    alive = np.tile(np.arange(T * H * W), (B, 1))
    keeps = []
    for r in (0.7, 0.5):
        n_prev = table.shape[1]
        k = math.ceil(r * n_prev)
        score = rng.random((B, n_prev))
        keep = np.sort(np.argsort(-score, axis=1, kind="stable")[:, :k], axis=1)
        keeps.append(keep)
        table = remap(table, keep)
        alive = np.take_along_axis(alive, keep, 1)
    final_mask = np.zeros((B, T * H * W), dtype=np.uint8)
    for b in range(B):
        final_mask[b, alive[b]] = 1
    out["table_pruned"] = dict(mask=final_mask.reshape(B, T, H, W), keep0=keeps[0], keep1=keeps[1],
                               table=table.astype(np.int32))

    # 3. full conv, 1 x 2 x 5 x 6 grid at 60 % keep, C_in 16 -> C_out 24
    B, T, H, W, ci, co = 1, 2, 5, 6, 16, 24
    m = np.zeros((B * T, H * W), dtype=np.uint8)
    for f in range(B * T):
        m[f, rng.permutation(H * W)[:18]] = 1
    m = m.reshape(B, T, H, W)
    n = int(m.sum())
    x, w, b, go = eighths(rng, (n, ci)), eighths(rng, (9, ci, co), 4), eighths(rng, co), eighths(rng, (n, co))
    y, gi, gw, gb = dense(m, x, w, b, go)
    out["conv"] = dict(mask=m, x=x, w=w, b=b, go=go, y=y, gi=gi, gw=gw, gb=gb)

    # 4. depthwise, same grid, C = 32
    c = 32
    x, w, b, go = eighths(rng, (n, c)), eighths(rng, (9, c), 4), eighths(rng, c), eighths(rng, (n, c))
    y, gi, gw, gb = dense(m, x, w, b, go, depthwise=True)
    out["depthwise"] = dict(mask=m, x=x, w=w, b=b, go=go, y=y, gi=gi, gw=gw, gb=gb)

    for name, arrays in out.items():
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **arrays)
        print("wrote", os.path.relpath(path, ROOT), {k: v.shape for k, v in arrays.items()})


if __name__ == "__main__":
    sys.exit(main())
