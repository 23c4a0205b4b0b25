"""Pins the CPU oracle (oracle/sv_oracle.*) with checks independent of its formulas.

* Table: the closed form against a numpy restatement of the reference's own
  build (pad/shift/stack + offsets) and its remap after sorted top-k prunes,
  plus the structural invariants (self at k=4, symmetry, borders, bounds).
* Convolution: the gather formulas against torch ``conv2d`` / autograd on a
  zero-filled dense grid (fp64), isolated tokens against ``x @ W[4] + b``.
* Sensitivity: plausible mistakes planted in (a copy of) the oracle's inputs
  must fail these checks.
"""
import numpy as np
import pytest

from tests.helpers import dense_reference, kaiming_weight, random_mask, topk_mask


SHAPES = [(1, 1, 1, 1), (1, 1, 3, 4), (1, 2, 5, 7), (2, 3, 14, 14), (2, 2, 16, 16)]


@pytest.mark.parametrize("shape", SHAPES)
def test_full_mask_table_equals_reference_build(oracle, shape):
    B, T, H, W = shape
    got = oracle.build_table(np.ones(shape, np.uint8))
    ref = oracle.ref_initial_table(H, W, T, B).reshape(-1, 9)
    np.testing.assert_array_equal(got, ref)


def test_reference_build_known_answer(oracle):
    # 2x2 grid, one frame: hand-written table (k = (dy+1)*3 + (dx+1)).
    ref = oracle.ref_initial_table(2, 2, 1, 1)[0]
    expect = np.array([
        [-1, -1, -1, -1, 0, 1, -1, 2, 3],
        [-1, -1, -1, 0, 1, -1, 2, 3, -1],
        [-1, 0, 1, -1, 2, 3, -1, -1, -1],
        [0, 1, -1, 2, 3, -1, -1, -1, -1],
    ], dtype=np.int32)
    np.testing.assert_array_equal(ref, expect)
    np.testing.assert_array_equal(oracle.build_table(np.ones((1, 1, 2, 2), np.uint8)), expect)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_prune_chain_equals_closed_form(oracle, seed):
    """Reference procedure: initial table, then several sorted top-k prunes with
    the Block remap; must equal the closed form built from the final mask."""
    rng = np.random.default_rng(seed)
    B, T, H, W = 2, 3, 6, 5
    n = T * H * W
    table = oracle.ref_initial_table(H, W, T, B)
    alive = np.tile(np.arange(n), (B, 1))  # original cell of each current token
    for keep_rate in (0.8, 0.6, 0.3):
        n_prev = table.shape[1]
        k = int(np.ceil(keep_rate * n_prev))
        idx = oracle.ref_topk_sorted(rng.random((B, n_prev)), k)
        new_np = oracle.ref_remap(table, idx)
        new_c = oracle.remap_table(table, idx)
        np.testing.assert_array_equal(new_c, new_np)
        table = new_np
        alive = np.take_along_axis(alive, idx, axis=1)
        mask = np.zeros((B, n), np.uint8)
        np.put_along_axis(mask, alive, 1, axis=1)
        closed = oracle.build_table(mask.reshape(B, T, H, W))
        np.testing.assert_array_equal(table.reshape(-1, 9), closed)


def test_remap_unsorted_keep_matches_numpy(oracle):
    rng = np.random.default_rng(5)
    table = oracle.ref_initial_table(4, 4, 2, 2)
    idx = np.stack([rng.permutation(32)[:11] for _ in range(2)])
    np.testing.assert_array_equal(oracle.remap_table(table, idx), oracle.ref_remap(table, idx))


@pytest.mark.parametrize("keep", [0.0, 0.1, 0.5, 1.0])
def test_table_invariants(oracle, keep):
    rng = np.random.default_rng(7)
    B, T, H, W = 2, 4, 7, 9
    mask = random_mask(rng, B, T, H, W, keep)
    t = oracle.build_table(mask)
    n = t.shape[0]
    assert n == int(mask.sum())
    assert t.shape == (n, 9) and t.dtype == np.int32
    if n == 0:
        return
    np.testing.assert_array_equal(t[:, 4], np.arange(n))
    assert t.max() < n and t.min() >= -1
    for k in range(9):
        v = t[:, k] >= 0
        j = t[v, k]
        np.testing.assert_array_equal(t[j, 8 - k], np.nonzero(v)[0])
    # border cells have -1 toward the outside
    cells = np.flatnonzero(mask.reshape(-1))
    y = (cells % (H * W)) // W
    x = cells % W
    for k in range(9):
        dy, dx = k // 3 - 1, k % 3 - 1
        outside = (y + dy < 0) | (y + dy >= H) | (x + dx < 0) | (x + dx >= W)
        assert np.all(t[outside, k] == -1)


def _case(seed, B=2, T=2, H=5, W=6, ci=8, co=12, keep=0.6, bias=True):
    rng = np.random.default_rng(seed)
    mask = random_mask(rng, B, T, H, W, keep)
    n = int(mask.sum())
    x = rng.standard_normal((n, ci)).astype(np.float32)
    w = kaiming_weight(rng, ci, co)
    b = rng.uniform(-0.3, 0.3, co).astype(np.float32) if bias else None
    go = rng.standard_normal((n, co)).astype(np.float32)
    return mask, x, w, b, go


@pytest.mark.parametrize("seed,bias", [(0, True), (1, False), (2, True)])
def test_conv_matches_dense_conv2d(oracle, seed, bias):
    mask, x, w, b, go = _case(seed, bias=bias)
    t = oracle.build_table(mask)
    y_ref, gi_ref, gw_ref, gb_ref = dense_reference(mask, x, w, b, go)
    np.testing.assert_allclose(oracle.fwd(x, t, w, b), y_ref, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oracle.bwd_in(go, t, w), gi_ref, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oracle.bwd_w(go, x, t), gw_ref, rtol=1e-12, atol=1e-12)
    if bias:
        np.testing.assert_allclose(oracle.bias_grad(go), gb_ref, rtol=1e-12, atol=1e-12)


def test_full_keep_is_dense_conv(oracle):
    mask, x, w, b, go = _case(3, keep=1.0)
    t = oracle.build_table(mask)
    y_ref, gi_ref, gw_ref, _ = dense_reference(mask, x, w, b, go)
    np.testing.assert_allclose(oracle.fwd(x, t, w, b), y_ref, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oracle.bwd_w(go, x, t), gw_ref, rtol=1e-12, atol=1e-12)


def test_isolated_tokens_reduce_to_center_tap(oracle):
    rng = np.random.default_rng(4)
    mask = np.zeros((1, 2, 6, 6), np.uint8)
    mask[:, :, ::2, ::2] = 1  # no two kept cells are 8-adjacent
    n = int(mask.sum())
    x = rng.standard_normal((n, 8)).astype(np.float32)
    w = kaiming_weight(rng, 8, 4)
    b = rng.standard_normal(4).astype(np.float32)
    t = oracle.build_table(mask)
    assert np.all(t[:, [0, 1, 2, 3, 5, 6, 7, 8]] == -1)
    ref = x.astype(np.float64) @ w[4].astype(np.float64) + b
    np.testing.assert_allclose(oracle.fwd(x, t, w, b), ref, rtol=1e-12, atol=1e-12)


def test_local_indices_with_tokens_per_batch(oracle):
    """Local per-batch indices + tokens_per_batch equal global indices + 0,
    with tokens_per_batch not a multiple of 32 (the per-row offset rule)."""
    rng = np.random.default_rng(9)
    B, T, H, W = 3, 1, 7, 7
    mask = np.zeros((B, T * H * W), np.uint8)
    nb = 37
    for b in range(B):
        mask[b, rng.permutation(T * H * W)[:nb]] = 1
    mask = mask.reshape(B, T, H, W)
    t = oracle.build_table(mask)
    local = t.copy()
    for b in range(B):
        blk = local[b * nb:(b + 1) * nb]
        blk[blk >= 0] -= b * nb
    x = rng.standard_normal((B * nb, 8)).astype(np.float32)
    w = kaiming_weight(rng, 8, 8)
    go = rng.standard_normal((B * nb, 8)).astype(np.float32)
    np.testing.assert_array_equal(oracle.fwd(x, local, w, None, nb), oracle.fwd(x, t, w, None, 0))
    np.testing.assert_array_equal(oracle.bwd_in(go, local, w, nb), oracle.bwd_in(go, t, w, 0))
    np.testing.assert_array_equal(oracle.bwd_w(go, x, local, nb), oracle.bwd_w(go, x, t, 0))


def test_depthwise_matches_grouped_conv2d(oracle):
    rng = np.random.default_rng(11)
    mask = random_mask(rng, 2, 2, 6, 5, 0.5)
    n, c = int(mask.sum()), 6
    x = rng.standard_normal((n, c)).astype(np.float32)
    w = rng.standard_normal((9, c)).astype(np.float32)
    b = rng.standard_normal(c).astype(np.float32)
    go = rng.standard_normal((n, c)).astype(np.float32)
    t = oracle.build_table(mask)
    y_ref, gi_ref, gw_ref, _ = dense_reference(mask, x, w, b, go, depthwise=True)
    np.testing.assert_allclose(oracle.dw_fwd(x, t, w, b), y_ref, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oracle.dw_bwd_in(go, t, w), gi_ref, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oracle.dw_bwd_w(go, x, t), gw_ref, rtol=1e-12, atol=1e-12)


def test_fp32_port_matches_fp64(oracle):
    mask, x, w, b, go = _case(12, B=1, T=8, H=14, W=14, ci=48, co=48, keep=0.5)
    t = oracle.build_table(mask)
    port = oracle.Fp32Port(x.shape[0], 48, 48)
    y = port.fwd(x, t, w, b).copy()
    gi, gw = port.bwd(go, x, t, w)
    assert oracle.rel_err(y, oracle.fwd(x, t, w, b)) < 1e-5
    assert oracle.rel_err(gi, oracle.bwd_in(go, t, w)) < 1e-5
    assert oracle.rel_err(gw, oracle.bwd_w(go, x, t)) < 1e-5


def test_out_of_range_entries_are_missing(oracle):
    x = np.ones((2, 4), np.float32)
    w = np.ones((9, 4, 4), np.float32)
    t = np.full((2, 9), -1, np.int32)
    t[0, 4], t[1, 4] = 0, 1
    t[0, 0] = 7        # beyond N: treated as missing
    t[1, 1] = -5       # negative non-sentinel: treated as missing
    y = oracle.fwd(x, t, w)
    np.testing.assert_array_equal(y, np.full((2, 4), 4.0))


# ---------------------------------------------------------------------------
# sensitivity: planted mistakes must be caught by the dense check
# ---------------------------------------------------------------------------

def test_planted_offset_flip_is_caught(oracle):
    mask, x, w, b, go = _case(21)
    t = oracle.build_table(mask)
    y_ref = dense_reference(mask, x, w, b, go)[0]
    flipped = np.ascontiguousarray(w[::-1])          # k <-> 8-k mistake
    assert not np.allclose(oracle.fwd(x, t, flipped, b), y_ref, rtol=1e-6, atol=1e-6)
    swapped = np.ascontiguousarray(w.reshape(3, 3, *w.shape[1:]).transpose(1, 0, 2, 3).reshape(w.shape))
    assert not np.allclose(oracle.fwd(x, t, swapped, b), y_ref, rtol=1e-6, atol=1e-6)  # ky/kx swap


def test_planted_table_mistakes_are_caught(oracle):
    mask, x, w, b, go = _case(22)
    t = oracle.build_table(mask)
    y_ref, gi_ref, _, _ = dense_reference(mask, x, w, b, go)
    t_bad = t.copy()
    t_bad[:, [0, 8]] = t_bad[:, [8, 0]]                # transposed offsets
    assert not np.allclose(oracle.fwd(x, t_bad, w, b), y_ref, rtol=1e-6, atol=1e-6)
    # a bwd_in that gathers with W[k] instead of W[8-k] (symmetric-table shortcut done wrong)
    gi_wrong = oracle.bwd_in(go, t[:, ::-1].copy(), w)
    assert not np.allclose(gi_wrong, gi_ref, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("seed", [0, 1])
def test_prune_step_equals_row_loop_and_closed_form(oracle, seed):
    """ref_prune_step against a plain per-row loop (x rows, index bookkeeping)
    and, for its table, against the closed form of the pruned mask."""
    rng = np.random.default_rng(seed)
    B, T, H, W, S, C = 2, 2, 5, 4, 1, 3
    n = T * H * W
    table = oracle.ref_initial_table(H, W, T, B)
    x = rng.standard_normal((B, S + n, C)).astype(np.float32)
    last = np.stack([rng.permutation(1000)[:n] for _ in range(B)]).astype(np.int64)
    k = int(np.ceil(0.6 * n))
    idx = oracle.ref_topk_sorted(rng.random((B, n)), k)
    x_new, idx_new, t_new = oracle.ref_prune_step(x, idx, last, table, S)
    for b in range(B):
        np.testing.assert_array_equal(x_new[b, :S], x[b, :S])
        for j in range(k):
            np.testing.assert_array_equal(x_new[b, S + j], x[b, S + idx[b, j]])
            assert idx_new[b, j] == last[b, idx[b, j]]
    mask = np.zeros((B, n), np.uint8)
    np.put_along_axis(mask, idx, 1, axis=1)
    np.testing.assert_array_equal(t_new.reshape(-1, 9), oracle.build_table(mask.reshape(B, T, H, W)))
    # without the optional parts
    x2, i2, t2 = oracle.ref_prune_step(x, idx, None, None, S)
    np.testing.assert_array_equal(x2, x_new)
    assert i2 is None and t2 is None


@pytest.mark.parametrize("dname", ["float16", "bfloat16"])
def test_rounded_once_check_rejects_per_contribution_rounding(oracle, dname):
    """The GPU tests' single-rounding check (helpers.assert_rounded_once),
    pinned on the CPU: backward-input of a random asymmetric table whose rows
    receive several contributions, summed in fp32 and rounded once, passes;
    the same sums rounded to the 16-bit dtype after every contribution (what
    an atomic pass into the output does) fail."""
    import torch

    from tests.helpers import assert_rounded_once, kaiming_weight

    dt = getattr(torch, dname)
    rng = np.random.default_rng(13)
    n, ci, co = 150, 32, 24
    t = rng.integers(-1, n, size=(n, 9)).astype(np.int32)
    t[rng.random((n, 9)) < 0.3] = -1

    def rd(a):
        return torch.from_numpy(a).to(dt).float().numpy()

    w = rd(kaiming_weight(rng, ci, co))
    go = rd(rng.standard_normal((n, co)).astype(np.float32))
    exact = oracle.bwd_in(go, t, w)
    abs_sum = oracle.bwd_in(np.abs(go), t, np.abs(w))
    contribs = [[] for _ in range(n)]
    for i in range(n):
        for k in range(9):
            j = int(t[i, k])
            if 0 <= j < n:
                contribs[j].append(go[i].astype(np.float32) @ w[k].T.astype(np.float32))
    once = torch.zeros((n, ci), dtype=dt)
    each = torch.zeros((n, ci), dtype=dt)
    for j in range(n):
        acc = np.zeros(ci, np.float32)
        for c in contribs[j]:
            acc = (acc + c).astype(np.float32)
            each[j] = (each[j].float() + torch.from_numpy(c)).to(dt)
        once[j] = torch.from_numpy(acc).to(dt)
    assert_rounded_once(once, exact, abs_sum, dt)
    with pytest.raises(AssertionError):
        assert_rounded_once(each, exact, abs_sum, dt)
