"""Backward ops on tables that carry the builders' symmetric record.

A table built from a keep mask is symmetric: every entry (i, k) -> j has its
partner (j, 8-k) -> i. The builders record that on the tensor they return,
and the autograd functions then call the backward ops with symmetric=True
(SVTAD_TABLE_SYMMETRIC in the C ABI): the backward-input kernels load no
partners and no pass for entries without one runs. Checked here:

* on builder tables, symmetric=True gives results bit-identical to the
  checked calls on every backward path: the one-launch and the two-launch
  full backward (c2 shape at 10 % and 55 % keep, global and per-sample
  indices), backward-input alone, its gathered GEMM alone, the depthwise
  one-pass backward and backward-input (vectorized and scalar kernels,
  every dtype), and the float32 paths that ignore the flag;
* the symmetric results against the fp64 oracle at the north-star bar;
* the record on the builders' tables and the global conversion only (remap
  and prune give none), through the modules, and that an in-place change
  drops it; a remap with a repeated keep index (one-way entries) gives the
  oracle's gradients.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest

from tests.helpers import kaiming_weight, topk_mask

pytestmark = pytest.mark.gpu

TOL = 1e-2  # max-scaled error bar of the north star (f16 / bf16)


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _dt(name):
    import torch

    return {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32,
            "float64": torch.float64}[name]


def _table(dev, keep, seed, grid=(2, 80, 14, 14)):
    import torch

    import eccv26_tad_amd as sv

    rng = np.random.default_rng(seed)
    mask = topk_mask(rng, *grid, keep)
    t = sv.build_neighbor_table(torch.from_numpy(mask).to(dev))
    assert sv.is_symmetric_table(t)
    return t, rng


def _eq(a, b, what):
    import torch

    assert a.shape == b.shape, what
    if not torch.equal(a, b):
        d = (a.double() - b.double()).abs()
        raise AssertionError(f"{what}: {int((d > 0).sum())} elements differ, max {float(d.max()):.3e}")


@pytest.mark.parametrize("keep,dname,per_sample", [
    (0.1, "float16", False),   # the one-launch backward
    (0.1, "bfloat16", True),
    (0.55, "float16", False),  # two launches: gathered GEMM, then backward-weight + reduction
    (0.55, "bfloat16", True),
    (0.25, "float32", False),  # no packed layout: the flag is accepted and ignored
])
def test_conv_backward_symmetric_is_bit_identical(dev, oracle, keep, dname, per_sample):
    import torch

    t, rng = _table(dev, keep, 11)
    n, c = t.shape[0], 192
    _say(f"conv symmetric vs checked: keep {keep} {dname} per_sample {per_sample}, n = {n}")
    dt = _dt(dname)
    tab, tpb = t, 0
    if per_sample:  # equal kept counts per sample (topk masks): per-sample indices
        tpb = n // 2
        tab = torch.where(t >= 0, t % tpb, t)
    x = torch.from_numpy(rng.standard_normal((n, c)).astype(np.float32)).to(dev, dt)
    w = torch.from_numpy(kaiming_weight(rng, c, c)).to(dev, dt)
    go = torch.from_numpy(rng.standard_normal((n, c)).astype(np.float32)).to(dev, dt)
    ops = __import__("eccv26_tad_amd").ops
    _, pb = ops.pack_weight(w, True, True)
    sym = ops.bwd_packed(go, x, tab, w, pb, c, tpb, True, symmetric=True)
    chk = ops.bwd_packed(go, x, tab, w, pb, c, tpb, True)
    for a, b, nm in zip(sym, chk, ("grad_in", "grad_w", "grad_b")):
        _eq(a, b, f"bwd_packed {nm}")
    gi_s = ops.bwd_in_packed(go, tab, w, pb, n, c, tpb, symmetric=True)
    _eq(gi_s, ops.bwd_in_packed(go, tab, w, pb, n, c, tpb), "bwd_in_packed")
    _eq(gi_s, sym[0], "bwd_in_packed vs bwd_packed")
    if pb.numel():
        _eq(ops.bwd_in_gemm(go, tab, pb, c, tpb, symmetric=True), ops.bwd_in_gemm(go, tab, pb, c, tpb),
            "bwd_in_gemm")
    torch.cuda.synchronize()
    # against the fp64 oracle (backward-input of the global table)
    gi_ref = oracle.bwd_in(go.double().cpu().numpy(), t.cpu().numpy(), w.double().cpu().numpy())
    err = np.abs(sym[0].double().cpu().numpy() - gi_ref).max() / max(np.abs(gi_ref).max(), 1e-30)
    _say(f"  grad_in max-scaled error {err:.2e}")
    assert err <= (TOL if dt in (torch.float16, torch.bfloat16) else 1e-5)


@pytest.mark.parametrize("dname,c,keep", [
    ("float16", 192, 0.55),   # vectorized one-pass kernels
    ("float16", 192, 0.1),
    ("bfloat16", 64, 0.25),
    ("float32", 24, 0.4),
    ("float64", 8, 0.4),
    ("float16", 4, 0.55),     # c / 8 not whole: the scalar kernels
])
def test_depthwise_backward_symmetric_is_bit_identical(dev, oracle, dname, c, keep):
    import torch

    ops = __import__("eccv26_tad_amd").ops
    t, rng = _table(dev, keep, 5)
    n = t.shape[0]
    _say(f"depthwise symmetric vs checked: {dname} C = {c} keep {keep}, n = {n}")
    dt = _dt(dname)
    x = torch.from_numpy(rng.standard_normal((n, c))).to(dev, dt)
    w = torch.from_numpy(rng.uniform(-1, 1, (9, c)) / 3).to(dev, dt)
    go = torch.from_numpy(rng.standard_normal((n, c))).to(dev, dt)
    sym = ops.dw_bwd(go, x, t, w, 0, True, symmetric=True)
    chk = ops.dw_bwd(go, x, t, w, 0, True)
    for a, b, nm in zip(sym, chk, ("grad_in", "grad_w", "grad_b")):
        _eq(a, b, f"dw_bwd {nm}")
    gi_s = ops.dw_bwd_in(go, t, w, 0, symmetric=True)
    _eq(gi_s, ops.dw_bwd_in(go, t, w, 0), "dw_bwd_in")
    torch.cuda.synchronize()
    gi_ref = oracle.dw_bwd_in(go.double().cpu().numpy(), t.cpu().numpy(), w.double().cpu().numpy())
    err = np.abs(gi_s.double().cpu().numpy() - gi_ref).max() / max(np.abs(gi_ref).max(), 1e-30)
    _say(f"  grad_in max-scaled error {err:.2e}")
    assert err <= (TOL if dt in (torch.float16, torch.bfloat16) else 1e-5)


def test_record_on_builders_only(dev):
    import torch

    import eccv26_tad_amd as sv

    rng = np.random.default_rng(3)
    mask = torch.from_numpy(topk_mask(rng, 2, 4, 6, 6, 0.5)).to(dev)
    n = int(mask.sum())
    for t in (sv.build_neighbor_table(mask), sv.build_neighbor_table(mask, n=n),
              sv.build_neighbor_table(mask, batched=True), sv.build_neighbor_table(mask, dtype=torch.int64),
              sv.get_initial_neighbor_indices(6, 6, 4, dev, 2)):
        assert sv.is_symmetric_table(t)
        # the recorded tables really are symmetric: the transpose equals the flipped table
        tt, coll = sv.transpose_neighbor_table(t)
        assert coll == 0
        _eq(tt, t.reshape(-1, 9).flip(1).to(torch.int32), "transposed table vs column-flipped table")
    grid = sv.get_initial_neighbor_indices(6, 6, 4, dev, 2)  # [2, 144, 9] global
    g = sv.global_neighbor_table(grid, 144)
    assert sv.is_symmetric_table(g)
    # remap and prune give no record (their keep indices are not checked)
    keep = torch.stack([torch.randperm(144, generator=torch.Generator().manual_seed(s))[:72] for s in (0, 1)])
    keep = keep.to(dev)
    t2 = sv.remap_neighbor_table(grid, keep)
    x = torch.randn(2, 1 + 144, 16, device=dev)
    _, _, t3 = sv.prune_tokens(x, keep, neighbor_indices=grid, num_key_tokens=1)
    assert not sv.is_symmetric_table(t2) and not sv.is_symmetric_table(t3)
    _eq(t2, t3, "prune_tokens table vs remap_neighbor_table")
    grid[0, 0, 0] = -1  # an in-place change drops the record (and the view's base's)
    assert not sv.is_symmetric_table(grid)
    assert not sv.is_symmetric_table(grid.clone())


@pytest.mark.parametrize("depthwise", [False, True])
def test_repeated_keep_index_gradients(dev, oracle, depthwise):
    """A keep set that repeats an index (not what topk gives) leaves a remapped
    table whose copied row has no partners; its gradients still match the
    oracle (the remap carries no symmetric record, so the backward checks)."""
    import torch

    import eccv26_tad_amd as sv

    rng = np.random.default_rng(21)
    grid = sv.get_initial_neighbor_indices(8, 8, 3, dev, 1)  # [1, 192, 9]
    keep = torch.from_numpy(rng.permutation(192)[:96]).to(dev)
    keep[10] = keep[11]  # a repeated index
    t = sv.remap_neighbor_table(grid, keep.view(1, -1))
    assert not sv.is_symmetric_table(t)
    tn = t.reshape(-1, 9).cpu().numpy()
    tt, coll = sv.transpose_neighbor_table(t)
    assert coll > 0 or not torch.equal(tt, t.reshape(-1, 9).flip(1))  # really one-way entries
    n, c = 96, 64
    _say(f"repeated keep index: depthwise {depthwise}, n = {n}")
    torch.manual_seed(0)
    m = (sv.SparseDepthwiseConv2d(c) if depthwise else sv.SparseConv2d(c, c)).to(dev).half()
    x = torch.from_numpy(rng.standard_normal((n, c)).astype(np.float32)).to(dev, torch.float16).requires_grad_(True)
    y = m(x, t)
    go = torch.from_numpy(rng.standard_normal((n, c)).astype(np.float32)).to(dev, torch.float16)
    y.backward(go)
    torch.cuda.synchronize()
    w = m.weight.detach().double().cpu().numpy()
    g = go.double().cpu().numpy()
    # module weights are (9, C) / (9, C_in, C_out), the oracle's layouts
    gi_ref = oracle.dw_bwd_in(g, tn, w) if depthwise else oracle.bwd_in(g, tn, w)
    err = np.abs(x.grad.double().cpu().numpy() - gi_ref).max() / max(np.abs(gi_ref).max(), 1e-30)
    _say(f"  grad_in max-scaled error {err:.2e}")
    assert err <= TOL


@pytest.mark.parametrize("depthwise", [False, True])
def test_modules_use_the_record(dev, depthwise):
    import torch

    import eccv26_tad_amd as sv

    t, rng = _table(dev, 0.25, 9)
    n, c = t.shape[0], 192
    _say(f"module with a recorded table vs an unrecorded copy: depthwise {depthwise}, n = {n}")
    torch.manual_seed(0)
    m = (sv.SparseDepthwiseConv2d(c) if depthwise else sv.SparseConv2d(c, c)).to(dev).half()
    x0 = torch.from_numpy(rng.standard_normal((n, c)).astype(np.float32)).to(dev, torch.float16)
    grads = []
    for tab in (t, t.clone()):
        assert sv.is_symmetric_table(tab) == (tab is t)
        m.zero_grad()
        x = x0.clone().requires_grad_(True)
        y = m(x, tab)
        y.float().square().sum().backward()
        grads.append((y.detach(), x.grad, m.weight.grad.clone(), m.bias.grad.clone()))
    for a, b, nm in zip(grads[0], grads[1], ("out", "grad_in", "grad_w", "grad_b")):
        _eq(a, b, nm)
