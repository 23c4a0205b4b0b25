"""Neighbor tables without a host synchronisation, against the CPU oracle
(bit-exact, integer work):

* build_neighbor_table(mask, n=...) (one launch, svtad_table_build) for
  uniform, ragged, empty and single-cell masks, frames up to 128x128, grids
  with several frames per workgroup, int32 and int64 entries, a row count
  above the mask's (trailing -1 rows) and below it (leading rows only), and a
  mask past the one-launch limit (scan + fill, still without a sync);
* get_initial_neighbor_indices (svtad_table_grid, the closed form) against the
  reference procedure's restatement;
* the tokens_per_batch heuristic on the device (global_neighbor_table,
  svtad_table_to_global) against the reference rule applied on the host, and
  SparseConv2d / SparseDepthwiseConv2d / SparseConvAdapter with per-sample
  (local) tables bit for bit against the global table;
* none of the sync-free calls synchronise (torch's sync debug mode raises on a
  device -> host copy);
* the OPENTAD_DEBUG_SPARSE validation after a prune step.
"""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import random_mask, topk_mask

pytestmark = pytest.mark.gpu


def _ragged(rng, B, T, H, W):
    m = np.zeros((B, T, H * W), np.uint8)
    for b in range(B):
        for t in range(T):
            k = int(rng.integers(0, H * W + 1))
            m[b, t, rng.permutation(H * W)[:k]] = 1
    return m.reshape(B, T, H, W)


CASES = [
    ("uniform c2 55%", lambda r: topk_mask(r, 2, 80, 14, 14, 0.55)),
    ("uniform 10%", lambda r: random_mask(r, 2, 80, 14, 14, 0.1)),
    ("ragged c5 grid", lambda r: _ragged(r, 4, 128, 16, 16)),  # 512 frames: 2 frames per workgroup
    ("empty", lambda r: np.zeros((2, 3, 5, 6), np.uint8)),
    ("full", lambda r: np.ones((1, 4, 7, 9), np.uint8)),
    ("single cell", lambda r: np.ones((3, 5, 1, 1), np.uint8)),
    ("128x128 frames", lambda r: random_mask(r, 1, 3, 128, 128, 0.3)),
    ("odd frames", lambda r: random_mask(r, 2, 7, 33, 17, 0.5)),
]


@pytest.mark.parametrize("name,make", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("index_dtype", ["int32", "int64"])
def test_build_with_known_count(dev, oracle, name, make, index_dtype):
    import torch

    from eccv26_tad_amd import build_neighbor_table

    rng = np.random.default_rng(abs(hash(name)) % 10000)
    mask = make(rng)
    ref = oracle.build_table(mask)
    n = ref.shape[0]
    dt = getattr(torch, index_dtype)
    print("table_build", name, mask.shape, "n", n, index_dtype, flush=True)
    m = torch.from_numpy(mask).to(dev)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        got = build_neighbor_table(m, n=n, dtype=dt)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    assert got.dtype == dt and got.shape == (n, 9)
    np.testing.assert_array_equal(got.cpu().numpy(), ref)
    # a larger row count: trailing rows are -1; a smaller one: the first rows
    more = build_neighbor_table(m, n=n + 5, dtype=dt).cpu().numpy()
    np.testing.assert_array_equal(more[:n], ref)
    assert (more[n:] == -1).all()
    if n > 3:
        np.testing.assert_array_equal(build_neighbor_table(m, n=n - 3, dtype=dt).cpu().numpy(), ref[: n - 3])


def test_build_with_known_count_large_mask(dev, oracle):
    """A mask past the one-launch limit (4 MiB) takes the scan + fill launches,
    sized by the caller's count instead of a read-back."""
    import torch

    from eccv26_tad_amd import build_neighbor_table

    rng = np.random.default_rng(77)
    mask = random_mask(rng, 1, 300, 128, 128, 0.02)
    assert mask.size > (4 << 20)
    ref = oracle.build_table(mask)
    n = ref.shape[0]
    m = torch.from_numpy(mask).to(dev)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        got = build_neighbor_table(m, n=n)
        more = build_neighbor_table(m, n=n + 2, dtype=torch.int64)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    np.testing.assert_array_equal(got.cpu().numpy(), ref)
    np.testing.assert_array_equal(more.cpu().numpy()[:n], ref)
    assert (more.cpu().numpy()[n:] == -1).all()


@pytest.mark.parametrize("h,w,T,B", [(14, 14, 80, 2), (16, 16, 96, 2), (5, 7, 3, 2), (1, 1, 4, 1), (128, 128, 1, 1)])
@pytest.mark.parametrize("index_dtype", ["int32", "int64"])
def test_initial_table_closed_form(dev, oracle, h, w, T, B, index_dtype):
    import torch

    from eccv26_tad_amd import get_initial_neighbor_indices

    dt = getattr(torch, index_dtype)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        got = get_initial_neighbor_indices(h, w, T, dev, B, dtype=dt)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    assert got.dtype == dt and got.shape == (B, T * h * w, 9)
    np.testing.assert_array_equal(got.cpu().numpy(), oracle.ref_initial_table(h, w, T, B))


def _host_rule(table, N):
    """The reference wrapper's rule (sparse_conv_layer.py:170-177), on the host:
    tokens_per_batch = N when max < N, then source = entry + (i // N) * N."""
    t = table.reshape(-1, 9).astype(np.int64)
    if t.size and t.max() < N:
        off = (np.arange(t.shape[0]) // N * N)[:, None]
        t = np.where(t >= 0, t + off, t)
    return np.where(t < 0, -1, t).astype(np.int32)


@pytest.mark.parametrize("local", [True, False])
@pytest.mark.parametrize("index_dtype", ["int32", "int64"])
def test_global_table_on_device(dev, oracle, local, index_dtype):
    import torch

    from eccv26_tad_amd import global_neighbor_table

    rng = np.random.default_rng(5)
    B, N = 3, 60
    mask = np.zeros((B, 2 * 7 * 9), np.uint8)
    for b in range(B):
        mask[b, rng.permutation(126)[:N]] = 1
    t = oracle.build_table(mask.reshape(B, 2, 7, 9)).reshape(B, N, 9)
    if local:
        t = np.where(t >= 0, t - (np.arange(B) * N)[:, None, None], t)
    tt = torch.from_numpy(t).to(dev).to(getattr(torch, index_dtype))
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        got = global_neighbor_table(tt, N)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    assert got.dtype == torch.int32 and got.shape == (B * N, 9)
    np.testing.assert_array_equal(got.cpu().numpy(), _host_rule(t, N))
    np.testing.assert_array_equal(got.cpu().numpy(), oracle.build_table(mask.reshape(B, 2, 7, 9)))
    empty = global_neighbor_table(torch.empty(0, 9, dtype=torch.int32, device=dev), N)
    assert empty.shape == (0, 9)


def test_modules_with_local_tables_do_not_sync(dev, oracle):
    """SparseConv2d, SparseDepthwiseConv2d and SparseConvAdapter with per-sample
    tables and tokens_per_batch=None: forward and backward without a host
    synchronisation, outputs and gradients identical to the global table's."""
    import torch

    from eccv26_tad_amd import SparseConv2d, SparseConvAdapter, SparseDepthwiseConv2d

    rng = np.random.default_rng(8)
    B, T, H, W, N = 2, 3, 7, 9, 90
    mask = np.zeros((B, T * H * W), np.uint8)
    for b in range(B):
        mask[b, np.sort(rng.permutation(T * H * W)[:N])] = 1
    t = oracle.build_table(mask.reshape(B, T, H, W)).reshape(B, N, 9)
    local = np.where(t >= 0, t - (np.arange(B) * N)[:, None, None], t)
    idx = torch.from_numpy(np.stack([np.flatnonzero(mask[b]) for b in range(B)])).to(dev)
    torch.manual_seed(0)
    convs = [SparseConv2d(64, 64).to(dev).half(), SparseDepthwiseConv2d(64).to(dev).half()]
    adapter = SparseConvAdapter(256, 0.25).to(dev).half()
    with torch.no_grad():
        adapter.up_proj.weight.normal_(0, 0.05)
    x = torch.randn(B, N, 64, device=dev, dtype=torch.float16)
    xa = torch.randn(B, N + 1, 256, device=dev, dtype=torch.float16)

    def run(mod, inp, tab):
        xi = inp.detach().clone().requires_grad_(True)
        if isinstance(mod, SparseConvAdapter):
            y = mod(xi, H, W, idx, T * H * W, tab, tokens_per_batch=None)
        else:
            y = mod(xi, tab)
        y.backward(torch.ones_like(y))
        return [y.detach(), xi.grad] + [p.grad.clone() for p in mod.parameters()]

    for mod, inp in [(convs[0], x), (convs[1], x), (adapter, xa)]:
        ref = run(mod, inp, torch.from_numpy(t).to(dev))
        mod.zero_grad()
        tab = torch.from_numpy(local).to(dev).long()
        torch.cuda.synchronize()
        torch.cuda.set_sync_debug_mode("error")
        try:
            got = run(mod, inp, tab)
        finally:
            torch.cuda.set_sync_debug_mode(0)
        mod.zero_grad()
        for a, b in zip(got, ref):
            assert torch.equal(a, b), type(mod).__name__


def test_debug_sparse_validation(dev, oracle):
    """With the OPENTAD_DEBUG_SPARSE switch on, every prune step validates its
    table (a valid prune passes); validate_neighbor_table raises on a stale
    token count and on an out-of-range entry, with the reference's messages."""
    import torch

    import eccv26_tad_amd as sv
    from eccv26_tad_amd import neighbor

    B, T, H, W = 2, 4, 6, 6
    n = T * H * W
    table = sv.get_initial_neighbor_indices(H, W, T, dev, B)
    keep = torch.sort(torch.randperm(n, generator=torch.Generator().manual_seed(3))[: n // 2]).values
    keep = keep.repeat(B, 1).to(dev)
    x = torch.randn(B, 1 + n, 32, device=dev, dtype=torch.float16)
    calls = []
    orig = neighbor.validate_neighbor_table
    neighbor.validate_neighbor_table = lambda t, num, where="": (calls.append(where), orig(t, num, where))[1]
    try:
        sv.set_debug_sparse(True)
        _, _, t_new = sv.prune_tokens(x, keep, None, table, 1)
        sv.remap_neighbor_table(table, keep)
    finally:
        sv.set_debug_sparse(False)
        neighbor.validate_neighbor_table = orig
    assert calls == ["prune_tokens", "remap_neighbor_table"]
    with pytest.raises(RuntimeError, match="out of sync"):
        sv.validate_neighbor_table(t_new, n // 2 + 1, "test")
    bad = t_new.clone()
    bad[1, 3, 2] = B * (n // 2)
    with pytest.raises(RuntimeError, match="out of bounds"):
        sv.validate_neighbor_table(bad, n // 2, "test")
