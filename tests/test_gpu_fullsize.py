"""SparseConv2D at the full benchmark sizes: config c2 at every keep rate
the benchmark sweeps (10 / 25 / 40 / 55 / 70 / 100 %), c4 at 10 / 25 / 55 %,
c5 ragged, and the depthwise c3 on uniform and on the benchmark's clustered
(Gaussian-blob) keep masks. Checked: the neighbor table bit-exact against
the oracle's closed form, forward and backward-input on a seeded 2048-row
subsample against the fp64 oracle (run on the compacted sub-problem those
rows need), and the weight / bias gradients (sums over every row) against an
fp64 gather + matmul of the same expression, sum_i x[src(i,k)]^T go[i], at
full size.

The row count N decides the launch shape of the gathered GEMMs (row
fragments per workgroup, 64-column tiles for few rows) and the split plan of
the backward-weight pass, so the keep sweep runs every instantiation the
benchmark times at these shapes. Each case prints the errors it measured.

The oracle's scalar C loops are what the small-size tests pin; at these sizes
they would take minutes, hence the compacted sub-problems and the matmul form
of the row sums."""

from __future__ import annotations

import sys

import numpy as np
import pytest

from tests.helpers import kaiming_weight, topk_mask

pytestmark = pytest.mark.gpu

TOL = {"float16": 1e-2, "bfloat16": 1e-2}  # max-scaled error bars of the north star


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _ragged_mask(rng, B, T, H, W, lo=0.05, hi=0.15):
    """Per frame round(U(lo, hi) * H * W) random cells (config c5)."""
    m = np.zeros((B, T, H * W), np.uint8)
    for b in range(B):
        for t in range(T):
            k = int(round(rng.uniform(lo, hi) * H * W))
            m[b, t, rng.permutation(H * W)[:k]] = 1
    return m.reshape(B, T, H, W)


def _sub_fwd(oracle, x, t, w, rows):
    """oracle.fwd for `rows` only: the rows their entries gather, compacted."""
    ent = t[rows]
    need = np.unique(ent[ent >= 0])
    pos = np.full(x.shape[0], -1, np.int64)
    pos[need] = np.arange(need.size)
    n = max(need.size, rows.size)
    xc = np.zeros((n, x.shape[1]), np.float32)
    xc[: need.size] = x[need]
    tc = np.full((n, 9), -1, np.int32)
    tc[: rows.size] = np.where(ent >= 0, pos[np.maximum(ent, 0)], -1)
    return oracle.fwd(xc, tc, w)[: rows.size]


def _sub_bwd_in(oracle, go, t, w, rows):
    """oracle.bwd_in for output rows `rows` only: the entries that point into
    them, with their source rows compacted."""
    inrows = np.zeros(go.shape[0], bool)
    inrows[rows] = True
    pos = np.full(go.shape[0], -1, np.int64)
    pos[rows] = np.arange(rows.size)
    hit = (t >= 0) & inrows[np.maximum(t, 0)]
    src = np.nonzero(hit.any(axis=1))[0]
    n = max(src.size, rows.size)
    goc = np.zeros((n, go.shape[1]), np.float32)
    goc[: src.size] = go[src]
    tc = np.full((n, 9), -1, np.int32)
    tc[: src.size] = np.where(hit[src], pos[np.maximum(t[src], 0)], -1)
    return oracle.bwd_in(goc, tc, w)[: rows.size]


def _gw_fp64(go, x, t):
    gw = np.empty((9, x.shape[1], go.shape[1]))
    g64 = go.astype(np.float64)
    for k in range(9):
        xk = np.where((t[:, k] >= 0)[:, None], x[np.maximum(t[:, k], 0)], 0.0).astype(np.float64)
        gw[k] = xk.T @ g64
    return gw


def _run(dev, oracle, mask, c, dname, seed):
    import torch

    import eccv26_tad_amd as sv

    ops = sv.ops
    dt = {"float16": torch.float16, "bfloat16": torch.bfloat16}[dname]
    rng = np.random.default_rng(seed)
    table = sv.build_neighbor_table(torch.from_numpy(mask).to(dev))
    ref_t = oracle.build_table(mask)
    assert table.shape == ref_t.shape and np.array_equal(table.cpu().numpy(), ref_t)
    t = ref_t
    n = t.shape[0]
    _say("  n =", n)

    def rounded(a):
        return torch.from_numpy(a).to(dt).float().numpy()

    x = rounded(rng.standard_normal((n, c)).astype(np.float32))
    w = rounded(kaiming_weight(rng, c, c))
    b = rounded((rng.random(c).astype(np.float32) - 0.5) * 0.2)
    go = rounded(rng.standard_normal((n, c)).astype(np.float32))
    X, W, Bb, G = (torch.from_numpy(a).to(dev, dt) for a in (x, w, b, go))
    pf, pb = ops.pack_weight(W, True, True)
    y = ops.fwd_packed(X, table, W, pf, Bb, 0, 1).float().cpu().numpy()
    gi, gw, gb = ops.bwd_packed(G, X, table, W, pb, c, 0, True)
    gi, gw, gb = (a.float().cpu().numpy() for a in (gi, gw, gb))
    tol = TOL[dname]
    rows = np.sort(rng.choice(n, size=min(2048, n), replace=False))
    errs = {
        "y": oracle.rel_err(y[rows], _sub_fwd(oracle, x, t, w, rows) + b),
        "grad_x": oracle.rel_err(gi[rows], _sub_bwd_in(oracle, go, t, w, rows)),
        "grad_w": oracle.rel_err(gw, _gw_fp64(go, x, t)),
        "grad_b": oracle.rel_err(gb, go.astype(np.float64).sum(0)),
    }
    _say("  max-scaled errors:", {k: f"{v:.2e}" for k, v in errs.items()}, f"(bar {tol:g})")
    for k, v in errs.items():
        assert v <= tol, (k, v)


def test_c2_full_size(dev, oracle):
    """c2: B2 x T80 x 14x14, C=192 fp16, 55 % top-k keep (N = 17248)."""
    _say("c2 full size")
    mask = topk_mask(np.random.default_rng(1002), 2, 80, 14, 14, 0.55)
    _run(dev, oracle, mask, 192, "float16", 2002)


# N = 3136 / 7840 / 12544 / 21952 / 31360: the 64-column tiles of three row
# fragments (10 %, 25 %), four and six row fragments per full-width tile
# (40 %, 70 %) and eight (100 %) in the forward and backward-input GEMMs
@pytest.mark.parametrize("keep", [0.10, 0.25, 0.40, 0.70, 1.00])
def test_c2_full_size_keep_sweep(dev, oracle, keep):
    """c2 at the other keep rates of the benchmark sweep."""
    _say(f"c2 full size, keep {keep}")
    mask = topk_mask(np.random.default_rng(1102 + int(keep * 100)), 2, 80, 14, 14, keep)
    _run(dev, oracle, mask, 192, "float16", 2102 + int(keep * 100))


def test_c4_full_size(dev, oracle):
    """c4: B2 x T96 x 16x16, C=256 bf16, 25 % top-k keep (N = 12288)."""
    _say("c4 full size")
    mask = topk_mask(np.random.default_rng(1004), 2, 96, 16, 16, 0.25)
    _run(dev, oracle, mask, 256, "bfloat16", 2004)


def test_c5_full_size_ragged(dev, oracle):
    """c5: B4 x T128 x 16x16, C=512 bf16, ragged per-frame keeps of 5-15 %
    (global table, tokens_per_batch = 0)."""
    _say("c5 full size")
    mask = _ragged_mask(np.random.default_rng(1005), 4, 128, 16, 16)
    _run(dev, oracle, mask, 512, "bfloat16", 2005)


def test_c4_full_size_keep010(dev, oracle):
    """c4 at 10 % keep (N = 4916): 128-column tiles of three row fragments."""
    _say("c4 full size 10 %")
    mask = topk_mask(np.random.default_rng(1024), 2, 96, 16, 16, 0.10)
    _run(dev, oracle, mask, 256, "bfloat16", 2024)


def test_c4_full_size_keep055(dev, oracle):
    """c4 at 55 % keep (N = 27034): the gathered GEMMs run four row fragments
    per workgroup in two even rounds (no single round fits)."""
    _say("c4 full size 55 %")
    mask = topk_mask(np.random.default_rng(1014), 2, 96, 16, 16, 0.55)
    _run(dev, oracle, mask, 256, "bfloat16", 2014)


def _dw_run(dev, oracle, mask, rng):
    import torch

    import opentad_sparse_ops as ops

    t = oracle.build_table(mask)
    n, c = t.shape[0], 192
    dt = torch.float16
    x = torch.from_numpy(rng.standard_normal((n, c)).astype(np.float32)).to(dt)
    w = torch.from_numpy((rng.standard_normal((9, c)) * 0.3).astype(np.float32)).to(dt)
    b = torch.from_numpy((rng.standard_normal(c) * 0.1).astype(np.float32)).to(dt)
    go = torch.from_numpy(rng.standard_normal((n, c)).astype(np.float32)).to(dt)
    xn, wn, bn, gn = (a.float().numpy() for a in (x, w, b, go))
    T = torch.from_numpy(t).to(dev)
    y = ops.dw_fwd(x.to(dev), T, w.to(dev), b.to(dev), 0)
    gi, gw, gb = ops.dw_bwd(go.to(dev), x.to(dev), T, w.to(dev), 0, True)
    tol = TOL["float16"]
    _say("  n =", n, "hit rate", f"{float((t >= 0).mean()):.3f}")
    errs = {
        "y": oracle.rel_err(y.cpu().double().numpy(), oracle.dw_fwd(xn, t, wn, bn)),
        "grad_x": oracle.rel_err(gi.cpu().double().numpy(), oracle.dw_bwd_in(gn, t, wn)),
        "grad_w": oracle.rel_err(gw.cpu().double().numpy(), oracle.dw_bwd_w(gn, xn, t)),
        "grad_b": oracle.rel_err(gb.cpu().double().numpy(), oracle.bias_grad(gn)),
    }
    _say("  max-scaled errors:", {k: f"{v:.2e}" for k, v in errs.items()}, f"(bar {tol:g})")
    for k, v in errs.items():
        assert v <= tol, (k, v)


def test_c3_depthwise_full_size(dev, oracle):
    """c3: depthwise C=192 fp16 on B2 x T80 x 14x14 at 55 % keep: forward and
    the one-pass backward (input, weight, bias gradients) against the fp64
    oracle at full size."""
    _say("c3 depthwise full size")
    rng = np.random.default_rng(1003)
    mask = topk_mask(rng, 2, 80, 14, 14, 0.55)
    _dw_run(dev, oracle, mask, rng)


@pytest.mark.parametrize("keep", [0.10, 0.55])
def test_c3_depthwise_blob_masks(dev, oracle, keep):
    """c3 on the clustered keep masks the benchmark times (bench.blob_mask:
    two drifting Gaussian blobs per frame, top-k per sample): high neighbor
    hit rates, long runs of kept rows."""
    from bench import blob_mask

    _say(f"c3 depthwise, blob masks, keep {keep}")
    mask = blob_mask(keep).numpy()
    _dw_run(dev, oracle, mask, np.random.default_rng(1203 + int(keep * 100)))
