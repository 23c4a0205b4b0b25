"""GPU parity of the fused prune step (prune_tokens, svtad_prune_step) against
the oracle's restatement of the Block prune step (vit_sparse_adapter_poguise.py
:899-977). Integer and copy work: every output is compared bit-exactly."""

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _case(rng, oracle, B, T, H, W, S, C, keep, sorted_keep=True):
    n = T * H * W
    table = oracle.ref_initial_table(H, W, T, B)
    x = rng.standard_normal((B, S + n, C)).astype(np.float32)
    last = np.stack([rng.permutation(4 * n)[:n] for _ in range(B)]).astype(np.int64)
    k = int(np.ceil(keep * n))
    if sorted_keep:
        idx = oracle.ref_topk_sorted(rng.random((B, n)), k)
    else:
        idx = np.stack([rng.permutation(n)[:k] for _ in range(B)]).astype(np.int64)
    return x, last, table, idx


@pytest.mark.parametrize("dname", ["float16", "float32", "bfloat16"])
@pytest.mark.parametrize("S,C", [(1, 768), (0, 192), (2, 3), (1, 6)])
def test_prune_matches_oracle(dev, oracle, dname, S, C):
    """Row widths of 16-byte, 4-byte and odd-byte chunks; with and without key
    tokens."""
    import torch

    import eccv26_tad_amd as sv

    _say("prune", dname, S, C)
    rng = np.random.default_rng(C + S)
    x, last, table, idx = _case(rng, oracle, 2, 3, 7, 6, S, C, 0.55)
    dt = getattr(torch, dname)
    X = torch.from_numpy(x).to(dev, dt)
    xr = X.cpu().float().numpy()  # the values as rounded to dt
    x_ref, i_ref, t_ref = oracle.ref_prune_step(xr, idx, last, table, S)
    xn, ix, tn = sv.prune_tokens(X, torch.from_numpy(idx).to(dev), torch.from_numpy(last).to(dev),
                                 torch.from_numpy(table).to(dev), S)
    assert xn.dtype == dt and xn.shape == x_ref.shape
    assert torch.equal(xn.cpu(), torch.from_numpy(x_ref).to(dt))
    np.testing.assert_array_equal(ix.cpu().numpy(), i_ref)
    np.testing.assert_array_equal(tn.cpu().numpy(), t_ref)


def test_prune_unsorted_keep_and_optional_parts(dev, oracle):
    import torch

    import eccv26_tad_amd as sv

    rng = np.random.default_rng(7)
    x, last, table, idx = _case(rng, oracle, 3, 2, 5, 5, 1, 40, 0.3, sorted_keep=False)
    X = torch.from_numpy(x).to(dev)
    I = torch.from_numpy(idx).to(dev)
    x_ref, i_ref, t_ref = oracle.ref_prune_step(x, idx, last, table, 1)
    xn, ix, tn = sv.prune_tokens(X, I, torch.from_numpy(last).to(dev), torch.from_numpy(table).to(dev), 1)
    np.testing.assert_array_equal(xn.cpu().numpy(), x_ref)
    np.testing.assert_array_equal(ix.cpu().numpy(), i_ref)
    np.testing.assert_array_equal(tn.cpu().numpy(), t_ref)
    # no bookkeeping, no table (the reference skips the table when it is None)
    xn2, ix2, tn2 = sv.prune_tokens(X, I, None, None, 1)
    assert ix2 is None and tn2 is None
    np.testing.assert_array_equal(xn2.cpu().numpy(), x_ref)
    # int64 table in, int64 out (InternVideo's tables are int64)
    _, _, tn3 = sv.prune_tokens(X, I, None, torch.from_numpy(table).to(dev).long(), 1)
    assert tn3.dtype == torch.int64
    np.testing.assert_array_equal(tn3.cpu().numpy(), t_ref)


def test_prune_edges(dev, oracle):
    """Keep everything (identity), keep nothing, and a chain of prunes that must
    end at the closed-form table of the surviving cells."""
    import torch

    import eccv26_tad_amd as sv

    rng = np.random.default_rng(3)
    B, T, H, W = 2, 2, 6, 6
    n = T * H * W
    x, last, table, _ = _case(rng, oracle, B, T, H, W, 1, 16, 1.0)
    X, L, Tb = (torch.from_numpy(a).to(dev) for a in (x, last, table))
    full = torch.arange(n, device=dev).repeat(B, 1)
    xn, ix, tn = sv.prune_tokens(X, full, L, Tb, 1)
    assert torch.equal(xn, X) and torch.equal(ix, L) and torch.equal(tn, Tb)
    xn, ix, tn = sv.prune_tokens(X, full[:, :0], L, Tb, 1)
    assert xn.shape == (B, 1, 16) and ix.shape == (B, 0) and tn.shape == (B, 0, 9)
    assert torch.equal(xn, X[:, :1])
    # chain: three sorted top-k prunes, then compare with the closed form
    alive = np.tile(np.arange(n), (B, 1))
    t_cur, x_cur = Tb, X
    for keep in (0.7, 0.5, 0.3):
        n_prev = t_cur.shape[1]
        k = int(np.ceil(keep * n_prev))
        idx = oracle.ref_topk_sorted(rng.random((B, n_prev)), k)
        x_cur, _, t_cur = sv.prune_tokens(x_cur, torch.from_numpy(idx).to(dev), None, t_cur, 1)
        alive = np.take_along_axis(alive, idx, axis=1)
    mask = np.zeros((B, n), np.uint8)
    np.put_along_axis(mask, alive, 1, axis=1)
    np.testing.assert_array_equal(t_cur.cpu().numpy().reshape(-1, 9),
                                  oracle.build_table(mask.reshape(B, T, H, W)))


def test_prune_full_size(dev, oracle):
    """The ViT-B token tensor of config 2: B2 x (1 + 80*14*14) x 768 fp16 at 55 %
    keep, bit-exact against the oracle."""
    import torch

    import eccv26_tad_amd as sv

    _say("prune full size")
    rng = np.random.default_rng(11)
    B, T, H, W, S, C = 2, 80, 14, 14, 1, 768
    n = T * H * W
    table = oracle.ref_initial_table(H, W, T, B)
    idx = oracle.ref_topk_sorted(rng.random((B, n)), int(np.ceil(0.55 * n)))
    X = torch.randn(B, S + n, C, device=dev, dtype=torch.float16)
    L = torch.arange(n, device=dev, dtype=torch.long).repeat(B, 1)
    xn, ix, tn = sv.prune_tokens(X, torch.from_numpy(idx).to(dev), L, torch.from_numpy(table).to(dev), S)
    x_ref, i_ref, t_ref = oracle.ref_prune_step(X.cpu().numpy(), idx, L.cpu().numpy(), table, S)
    assert np.array_equal(xn.cpu().numpy(), x_ref)
    np.testing.assert_array_equal(ix.cpu().numpy(), i_ref)
    np.testing.assert_array_equal(tn.cpu().numpy(), t_ref)
