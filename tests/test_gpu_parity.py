"""GPU parity: the HIP kernels (through opentad_sparse_ops / the C ABI) against
the CPU oracle on the same seeded inputs.

Bar: bit-exact for the neighbor tables (integer work); max-scaled error
max|got-ref|/max|ref| <= 1e-5 for fp32, <= 1e-2 for fp16/bf16, <= 1e-12 for
fp64, against the fp64 oracle fed the same (rounded) inputs.
"""
import math
import sys

import numpy as np
import pytest

from tests.helpers import assert_rounded_once as _assert_rounded_once
from tests.helpers import kaiming_weight, random_mask, topk_mask

pytestmark = pytest.mark.gpu

TOL = {"float32": 1e-5, "float16": 1e-2, "bfloat16": 1e-2, "float64": 1e-12}


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _err_ok(oracle, got, ref, tol, what):
    """Max-scaled error of got against ref, printed, and whether it meets tol."""
    e = oracle.rel_err(got, ref)
    _say(f"  {what}: max-scaled error {e:.2e} (bar {tol:.0e})")
    return e <= tol


def _t(a, dev, dtype):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(dtype)


def _np32(t):
    return t.detach().float().cpu().numpy()


def _dt(name):
    import torch

    return getattr(torch, name)


# ---------------------------------------------------------------------------
# neighbor tables (bit-exact)
# ---------------------------------------------------------------------------

TABLE_SHAPES = [(1, 1, 1, 1), (1, 1, 3, 4), (2, 3, 14, 14), (2, 80, 14, 14), (4, 8, 16, 16),
                (1, 2, 33, 17), (1, 1, 128, 128)]


@pytest.mark.parametrize("shape", TABLE_SHAPES)
@pytest.mark.parametrize("keep", [0.0, 0.1, 0.55, 1.0])
def test_build_table_bit_exact(dev, oracle, shape, keep):
    import opentad_sparse_ops as ops
    import torch

    _say("build_table", shape, keep)
    rng = np.random.default_rng(hash((shape, keep)) & 0xffff)
    mask = random_mask(rng, *shape, keep)
    got = ops.build_neighbor_table(torch.from_numpy(mask).to(dev)).cpu().numpy()
    np.testing.assert_array_equal(got, oracle.build_table(mask))


def test_build_table_bool_mask_and_initial(dev, oracle):
    import torch

    from eccv26_tad_amd import build_neighbor_table, get_initial_neighbor_indices

    m = torch.ones(2, 3, 5, 7, dtype=torch.bool, device=dev)
    np.testing.assert_array_equal(build_neighbor_table(m).cpu().numpy(),
                                  oracle.ref_initial_table(5, 7, 3, 2).reshape(-1, 9))
    init = get_initial_neighbor_indices(5, 7, 3, dev, 2, dtype=torch.int64)
    assert init.dtype == torch.int64 and init.shape == (2, 105, 9)
    np.testing.assert_array_equal(init.cpu().numpy(), oracle.ref_initial_table(5, 7, 3, 2))


@pytest.mark.parametrize("sorted_keep", [True, False])
def test_remap_bit_exact(dev, oracle, sorted_keep):
    import torch

    from eccv26_tad_amd import remap_neighbor_table

    rng = np.random.default_rng(3)
    B, T, H, W = 2, 16, 14, 14
    table = oracle.ref_initial_table(H, W, T, B)
    for keep_rate in (0.7, 0.5):
        n_prev = table.shape[1]
        k = math.ceil(keep_rate * n_prev)
        if sorted_keep:
            idx = oracle.ref_topk_sorted(rng.random((B, n_prev)), k)
        else:
            idx = np.stack([rng.permutation(n_prev)[:k] for _ in range(B)])
        got = remap_neighbor_table(torch.from_numpy(table).to(dev), torch.from_numpy(idx).to(dev))
        ref = oracle.ref_remap(table, idx)
        np.testing.assert_array_equal(got.cpu().numpy(), ref)
        table = ref


def test_remap_int64_table(dev, oracle):
    import torch

    from eccv26_tad_amd import remap_neighbor_table

    table = oracle.ref_initial_table(6, 6, 2, 2).astype(np.int64)
    idx = oracle.ref_topk_sorted(np.random.default_rng(1).random((2, 72)), 30)
    got = remap_neighbor_table(torch.from_numpy(table).to(dev), torch.from_numpy(idx).to(dev))
    assert got.dtype == torch.int64
    np.testing.assert_array_equal(got.cpu().numpy(), oracle.ref_remap(table, idx))


def test_transpose_table(dev, oracle):
    import torch

    from eccv26_tad_amd import transpose_neighbor_table

    mask = random_mask(np.random.default_rng(2), 2, 4, 14, 14, 0.4)
    t = oracle.build_table(mask)
    tt, coll = transpose_neighbor_table(torch.from_numpy(t).to(dev))
    assert coll == 0
    np.testing.assert_array_equal(tt.cpu().numpy(), t[:, ::-1])
    dup = np.full((3, 9), -1, np.int32)
    dup[:, 4] = [0, 0, 0]  # three entries map to (0, 4)
    tt, coll = transpose_neighbor_table(torch.from_numpy(dup).to(dev))
    assert coll == 2 and tt.cpu().numpy()[0, 4] in (0, 1, 2)


def test_validate_table(dev, oracle):
    import torch

    from eccv26_tad_amd import validate_neighbor_table

    t = oracle.ref_initial_table(4, 4, 2, 2)
    tt = torch.from_numpy(t).to(dev)
    validate_neighbor_table(tt, 32)
    with pytest.raises(RuntimeError, match="second dim"):
        validate_neighbor_table(tt, 31)
    bad = t.copy()
    bad[1, 3, 2] = 64
    with pytest.raises(RuntimeError, match="out of bounds"):
        validate_neighbor_table(torch.from_numpy(bad).to(dev), 32)


# ---------------------------------------------------------------------------
# convolution: forward / bwd_in / bwd_w / bias grad
# ---------------------------------------------------------------------------

def _conv_case(seed, shape, keep, ci, co, dtype, bias=True, clustered=False):
    rng = np.random.default_rng(seed)
    mask = topk_mask(rng, *shape, keep) if not clustered else random_mask(rng, *shape, keep)
    n = int(mask.sum())
    x = rng.standard_normal((n, ci)).astype(np.float32)
    w = kaiming_weight(rng, ci, co)
    b = rng.uniform(-0.5, 0.5, co).astype(np.float32) if bias else None
    go = rng.standard_normal((n, co)).astype(np.float32)
    return mask, x, w, b, go


def _rounded(a, dt):
    """Inputs rounded to the test dtype, back in fp32 (what the GPU sees)."""
    import torch

    return torch.from_numpy(a).to(dt).to(torch.float32).numpy()


CONV_CASES = [
    # (shape B,T,H,W), keep, C_in, C_out, dtype
    ((1, 8, 14, 14), 0.5, 48, 48, "float32"),      # config 1
    ((1, 8, 14, 14), 0.5, 48, 48, "float64"),
    ((2, 4, 14, 14), 0.3, 64, 64, "float16"),
    ((2, 4, 14, 14), 0.55, 192, 192, "float16"),   # config 2 channels
    ((2, 4, 14, 14), 0.55, 192, 192, "bfloat16"),
    ((2, 3, 16, 16), 0.25, 256, 256, "bfloat16"),  # config 4 channels
    ((1, 2, 16, 16), 0.1, 512, 512, "bfloat16"),   # config 5 channels
    ((1, 3, 7, 9), 0.6, 12, 20, "float32"),        # C_in % 8 != 0, odd C_out
    ((1, 3, 7, 9), 0.6, 20, 36, "float16"),
    ((2, 2, 14, 14), 1.0, 128, 96, "float16"),
    ((2, 16, 14, 14), 0.55, 192, 192, "float16"),  # many row tiles and row splits
    ((1, 4, 16, 16), 0.4, 256, 128, "bfloat16"),
    ((1, 8, 14, 14), 0.5, 48, 48, "float16"),      # config-1 channels on the matrix cores
    ((1, 3, 9, 11), 0.7, 40, 24, "float16"),       # widths that are not tile multiples
    ((1, 8, 16, 16), 0.5, 512, 512, "bfloat16"),   # backward-weight wider than one co-resident grid
]


@pytest.mark.parametrize("case", CONV_CASES, ids=lambda c: f"{c[0]}-{c[1]}-{c[2]}x{c[3]}-{c[4]}")
def test_conv_fwd_bwd_vs_oracle(dev, oracle, case):
    import opentad_sparse_ops as ops

    shape, keep, ci, co, dname = case
    _say("conv", case)
    dt = _dt(dname)
    mask, x, w, b, go = _conv_case(7, shape, keep, ci, co, dname)
    x, w, b, go = (_rounded(a, dt) for a in (x, w, b, go))
    t = oracle.build_table(mask)
    X, W, Bb, G = (_t(a, dev, dt) for a in (x, w, b, go))
    T = _t(t, dev, _dt("int32"))
    tol = TOL[dname]
    y = ops.implicit_gemm_fwd_v2(X, T, W, Bb, 0)
    assert _err_ok(oracle, _np32(y) if dname != "float64" else y.cpu().numpy(), oracle.fwd(x, t, w, b), tol, "y")
    y0 = ops.fwd(X, T, W, co, 0)
    assert _err_ok(oracle, y0.cpu().double().numpy(), oracle.fwd(x, t, w), tol, "y0")
    gi = ops.bwd_in(G, T, W, x.shape[0], ci, 0)
    assert gi.dtype == dt and gi.shape == (x.shape[0], ci)
    assert _err_ok(oracle, gi.cpu().double().numpy(), oracle.bwd_in(go, t, w), tol, "gi")
    gw, gb = ops.bwd_w_bias(G, X, T, ci, 0, True)
    assert gw.dtype == dt and gw.shape == (9, ci, co)
    assert _err_ok(oracle, gw.cpu().double().numpy(), oracle.bwd_w(go, x, t), tol, "gw")
    assert _err_ok(oracle, gb.cpu().double().numpy(), oracle.bias_grad(go), tol, "gb")
    gw2 = ops.bwd_w(G, X, T, ci, 0)
    assert _err_ok(oracle, gw2.cpu().double().numpy(), oracle.bwd_w(go, x, t), tol, "gw2")


@pytest.mark.parametrize("dname", ["float32", "float16"])
def test_local_indices_tokens_per_batch(dev, oracle, dname):
    """Local indices with tokens_per_batch = 37 (not a multiple of 32, B = 3)."""
    import opentad_sparse_ops as ops

    dt = _dt(dname)
    rng = np.random.default_rng(9)
    B, nb = 3, 37
    mask = np.zeros((B, 49), np.uint8)
    for b in range(B):
        mask[b, rng.permutation(49)[:nb]] = 1
    mask = mask.reshape(B, 1, 7, 7)
    t = oracle.build_table(mask)
    local = t.copy()
    for b in range(B):
        blk = local[b * nb:(b + 1) * nb]
        blk[blk >= 0] -= b * nb
    ci = co = 16
    x = _rounded(rng.standard_normal((B * nb, ci)).astype(np.float32), dt)
    w = _rounded(kaiming_weight(rng, ci, co), dt)
    go = _rounded(rng.standard_normal((B * nb, co)).astype(np.float32), dt)
    X, W, G = (_t(a, dev, dt) for a in (x, w, go))
    L = _t(local, dev, _dt("int32"))
    tol = TOL[dname]
    assert _err_ok(oracle, _np32(ops.fwd(X, L, W, co, nb)), oracle.fwd(x, t, w), tol, "fwd")
    assert _err_ok(oracle, _np32(ops.bwd_in(G, L, W, B * nb, ci, nb)), oracle.bwd_in(go, t, w), tol, "bwd_in")
    assert _err_ok(oracle, _np32(ops.bwd_w(G, X, L, ci, nb)), oracle.bwd_w(go, x, t), tol, "bwd_w")


@pytest.mark.parametrize("dname", ["float32", "float16", "bfloat16"])
def test_asymmetric_table_orphans(dev, oracle, dname):
    """Tables that are not transposition-symmetric (duplicates, one-way links,
    out-of-range entries) go through the orphan pass of bwd_in."""
    import opentad_sparse_ops as ops

    dt = _dt(dname)
    rng = np.random.default_rng(13)
    n, ci, co = 150, 32, 24
    t = rng.integers(-1, n, size=(n, 9)).astype(np.int32)
    t[rng.random((n, 9)) < 0.3] = -1
    t[5, 2] = n + 40   # out of range -> missing
    t[6, 3] = -7       # negative non-sentinel -> missing
    x = _rounded(rng.standard_normal((n, ci)).astype(np.float32), dt)
    w = _rounded(kaiming_weight(rng, ci, co), dt)
    go = _rounded(rng.standard_normal((n, co)).astype(np.float32), dt)
    X, W, G = (_t(a, dev, dt) for a in (x, w, go))
    T = _t(t, dev, _dt("int32"))
    tol = TOL[dname]
    import torch

    assert _err_ok(oracle, _np32(ops.fwd(X, T, W, co, 0)), oracle.fwd(x, t, w), tol, "fwd")
    gi = ops.bwd_in(G, T, W, n, ci, 0)
    assert _err_ok(oracle, _np32(gi), oracle.bwd_in(go, t, w), tol, "bwd_in")
    assert _err_ok(oracle, _np32(ops.bwd_w(G, X, T, ci, 0)), oracle.bwd_w(go, x, t), tol, "bwd_w")
    # rows reached by one-way entries are recomputed in fp32 in a fixed
    # order and rounded once: two runs agree bit for bit, and every element
    # is the correctly rounded exact value or one of its two neighbors
    assert torch.equal(gi, ops.bwd_in(G, T, W, n, ci, 0))
    _assert_rounded_once(gi, oracle.bwd_in(go, t, w), oracle.bwd_in(np.abs(go), t, np.abs(w)), dt)


def _one_way_entries(t):
    """Entries (i, k) -> j of a global table whose partner (j, 8-k) -> i is absent."""
    n = t.shape[0]
    cnt = 0
    for i in range(n):
        for k in range(9):
            j = int(t[i, k])
            if 0 <= j < n and int(t[j, 8 - k]) != i:
                cnt += 1
    return cnt


@pytest.mark.parametrize("dname", ["float16", "bfloat16"])
@pytest.mark.parametrize("c", [64, 192])
def test_orphan_flag_wide_path(dev, oracle, c, dname):
    """On the matrix-core path the orphan pass only works when the
    backward-input kernel flags an entry without its symmetric partner. One
    packed weight is reused across symmetric, asymmetric and symmetric tables
    (a set flag may only cost time), then repacked (clears the flag); the
    per-call op keeps the flag in its workspace. Every result is checked
    against the oracle."""
    import opentad_sparse_ops as ops

    _say("orphan-flag", c, dname)
    dt = _dt(dname)
    rng = np.random.default_rng(29)
    mask, x, w, b, go = _conv_case(31, (1, 4, 12, 12), 0.6, c, c, dname)
    sym = oracle.build_table(mask)
    n = sym.shape[0]
    asym = sym.copy()
    # one-way links: entries whose partner (j, 8-k) -> i is absent
    rows = rng.choice(n, size=12, replace=False)
    for q, i in enumerate(rows):
        asym[i, q % 9] = int(rng.integers(0, n))
    X, W, G = (_t(a, dev, dt) for a in (x, w, go))
    Ts, Ta = _t(sym, dev, _dt("int32")), _t(asym, dev, _dt("int32"))
    tol = TOL[dname]
    ref_s, ref_a = oracle.bwd_in(go, sym, w), oracle.bwd_in(go, asym, w)
    assert oracle.rel_err(ref_a, ref_s) > 10 * tol  # the one-way links matter
    _, pb = ops.pack_weight(W, False, True)
    assert pb.numel() > 0
    for T, ref in ((Ts, ref_s), (Ta, ref_a), (Ts, ref_s), (Ta, ref_a)):
        assert _err_ok(oracle, _np32(ops.bwd_in_packed(G, T, W, pb, n, c, 0)), ref, tol, "bwd_in_packed")
    _, pb2 = ops.pack_weight(W, False, True)
    for T, ref in ((Ta, ref_a), (Ts, ref_s)):
        assert _err_ok(oracle, _np32(ops.bwd_in_packed(G, T, W, pb2, n, c, 0)), ref, tol, "bwd_in_packed")
        assert _err_ok(oracle, _np32(ops.bwd_in(G, T, W, n, c, 0)), ref, tol, "bwd_in")
    # the rows reached by one-way links: one rounding, the same bits on every
    # run, through each path (packed, per-call, and the combined backward
    # whose reduction runs the pass)
    import torch

    a1 = ops.bwd_in_packed(G, Ta, W, pb2, n, c, 0)
    assert torch.equal(a1, ops.bwd_in_packed(G, Ta, W, pb2, n, c, 0))
    assert torch.equal(a1, ops.bwd_in(G, Ta, W, n, c, 0))
    gi, _, _ = ops.bwd_packed(G, X, Ta, W, pb2, c, 0, True)
    assert torch.equal(gi, a1)
    go_r, w_r = _rounded(go, dt), _rounded(w, dt)  # what the GPU computed with
    _assert_rounded_once(a1, oracle.bwd_in(go_r, asym, w_r), oracle.bwd_in(np.abs(go_r), asym, np.abs(w_r)), dt)


@pytest.mark.parametrize("ci,co,dname", [(192, 192, "float16"), (64, 64, "bfloat16"),
                                         (48, 64, "float16"), (128, 96, "bfloat16")])
def test_bwd_packed_matches(dev, oracle, ci, co, dname, monkeypatch):
    """bwd_packed (the autograd backward in one call) gives what bwd_in_packed +
    bwd_w_bias give: bit-identical on symmetric tables in its two-launch form
    (same kernels, no atomics); its one-launch form at 192 channels gives
    grad_x bit for bit and sums the weight and bias gradients in another
    order (fewer splits, the center offset in four parts). Within tolerance of
    the oracle when one-way links send work to the orphan pass (inside the
    reduction for the large-tile shapes, a pass of its own for 48 -> 64;
    128 -> 96 has no packed backward-input layout and falls back to the two
    calls)."""
    import opentad_sparse_ops as ops
    import torch

    _say("bwd_packed", ci, co, dname)
    dt = _dt(dname)
    mask, x, w, b, go = _conv_case(37, (1, 6, 14, 14), 0.5, ci, co, dname)
    sym = oracle.build_table(mask)
    n = sym.shape[0]
    X, W, G = (_t(a, dev, dt) for a in (x, w, go))
    Ts = _t(sym, dev, _dt("int32"))
    _, pb = ops.pack_weight(W, False, True)
    assert (pb.numel() > 0) == (co in (64, 128, 192, 256, 512))
    gi2 = ops.bwd_in_packed(G, Ts, W, pb, n, ci, 0)
    gw2, gb2 = ops.bwd_w_bias(G, X, Ts, ci, 0, True)
    monkeypatch.setenv("SVTAD_BWD_FUSED", "off")
    gi, gw, gb = ops.bwd_packed(G, X, Ts, W, pb, ci, 0, True)
    assert torch.equal(gi, gi2) and torch.equal(gw, gw2) and torch.equal(gb, gb2)
    _, gw3, gb3 = ops.bwd_packed(G, X, Ts, W, pb, ci, 0, False)
    assert torch.equal(gw3, gw2) and gb3.numel() == 0
    monkeypatch.delenv("SVTAD_BWD_FUSED")
    gi, gw, gb = ops.bwd_packed(G, X, Ts, W, pb, ci, 0, True)  # one launch where it applies
    assert torch.equal(gi, gi2)
    for a, r in ((gw, gw2), (gb, gb2)):
        d = (a.double() - r.double()).abs().max() / r.double().abs().max().clamp_min(1e-30)
        assert float(d) <= 4e-3, float(d)
    rng = np.random.default_rng(41)
    asym = sym.copy()
    for q, i in enumerate(rng.choice(n, size=10, replace=False)):
        asym[i, q % 9] = int(rng.integers(0, n))
    Ta = _t(asym, dev, _dt("int32"))
    tol = TOL[dname]
    gi, gw, gb = ops.bwd_packed(G, X, Ta, W, pb, ci, 0, True)
    assert _err_ok(oracle, _np32(gi), oracle.bwd_in(go, asym, w), tol, "gi")
    assert _err_ok(oracle, _np32(gw), oracle.bwd_w(go, x, asym), tol, "gw")
    assert _err_ok(oracle, _np32(gb), go.astype(np.float64).sum(0), tol, "gb")


@pytest.mark.parametrize("c,dname", [(192, "float16"), (64, "bfloat16")])
def test_far_symmetric_table_slice_fallback(dev, oracle, c, dname):
    """A symmetric table whose neighbors are random rows anywhere in [0, n):
    the row windows of the tiles do not fit in LDS, so the gathered GEMMs take
    their per-offset slice path (a table from a mask takes the window path).
    fwd, bwd_in (no orphans: every link has its partner) and bwd_w against the
    oracle."""
    import opentad_sparse_ops as ops

    _say("far-table", c, dname)
    dt = _dt(dname)
    rng = np.random.default_rng(53)
    n = 3000
    t = np.full((n, 9), -1, np.int32)
    t[:, 4] = np.arange(n)
    for k in range(4):  # offset k pairs with 8 - k
        perm = rng.permutation(n)
        a, b = perm[: n // 2], perm[n // 2: 2 * (n // 2)]
        keep = rng.random(a.shape[0]) < 0.8
        t[a[keep], k] = b[keep]
        t[b[keep], 8 - k] = a[keep]
    assert all((t[t[:, k][t[:, k] >= 0], 8 - k] == np.nonzero(t[:, k] >= 0)[0]).all() for k in range(9))
    x = _rounded(rng.standard_normal((n, c)).astype(np.float32), dt)
    w = _rounded(kaiming_weight(rng, c, c), dt)
    go = _rounded(rng.standard_normal((n, c)).astype(np.float32), dt)
    X, W, G = (_t(a_, dev, dt) for a_ in (x, w, go))
    T = _t(t, dev, _dt("int32"))
    tol = TOL[dname]
    assert _err_ok(oracle, _np32(ops.fwd(X, T, W, c, 0)), oracle.fwd(x, t, w), tol, "fwd")
    assert _err_ok(oracle, _np32(ops.bwd_in(G, T, W, n, c, 0)), oracle.bwd_in(go, t, w), tol, "bwd_in")
    pf, pb = ops.pack_weight(W, True, True)
    gi, gw, gb = ops.bwd_packed(G, X, T, W, pb, c, 0, True)
    assert _err_ok(oracle, _np32(gi), oracle.bwd_in(go, t, w), tol, "gi")
    assert _err_ok(oracle, _np32(gw), oracle.bwd_w(go, x, t), tol, "gw")
    assert _err_ok(oracle, _np32(ops.fwd_packed(X, T, W, pf, None, 0, 0)), oracle.fwd(x, t, w), tol, "fwd_packed")


def test_empty_and_isolated(dev, oracle):
    import opentad_sparse_ops as ops
    import torch

    W = torch.randn(9, 16, 8, device=dev)
    y = ops.fwd(torch.empty(0, 16, device=dev), torch.empty(0, 9, dtype=torch.int32, device=dev), W, 8, 0)
    assert y.shape == (0, 8)
    gw, gb = ops.bwd_w_bias(torch.empty(0, 8, device=dev), torch.empty(0, 16, device=dev),
                            torch.empty(0, 9, dtype=torch.int32, device=dev), 16, 0, True)
    assert float(gw.abs().max()) == 0.0 and float(gb.abs().max()) == 0.0
    mask = np.zeros((1, 2, 6, 6), np.uint8)
    mask[:, :, ::2, ::2] = 1
    t = oracle.build_table(mask)
    x = np.random.default_rng(0).standard_normal((t.shape[0], 16)).astype(np.float32)
    y = ops.fwd(_t(x, dev, torch.float32), _t(t, dev, torch.int32), W, 8, 0)
    ref = x.astype(np.float64) @ W[4].double().cpu().numpy()
    assert oracle.rel_err(_np32(y), ref) <= 1e-5


def test_chunked_api_matches(dev, oracle):
    import opentad_sparse_ops as ops
    import torch

    mask, x, w, b, go = _conv_case(17, (1, 4, 14, 14), 0.5, 128, 128, "float16")
    t = oracle.build_table(mask)
    X, W, Bb = (_t(a, dev, torch.float16) for a in (x, w, b))
    T = _t(t, dev, torch.int32)
    y1 = ops.implicit_gemm_fwd_v2(X, T, W, Bb, 0)
    y2 = ops.implicit_gemm_fwd_v2_chunked(X, T, W, Bb, 0, 4096)
    y3 = ops.implicit_gemm_fwd_v2_chunked(X, T, W, torch.Tensor(), 0, 100)
    assert torch.equal(y1, y2)
    y4 = ops.fwd(X, T, W, 128, 0)
    assert torch.equal(y3, y4)


# ---------------------------------------------------------------------------
# autograd wrapper (drop-in SparseConv2d)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("ci,dname,autocast", [(48, "float32", False), (192, "float32", True),
                                                (64, "float32", True), (256, "bfloat16", False)])
def test_sparse_conv2d_module(dev, oracle, ci, dname, autocast):
    import torch

    from eccv26_tad_amd import SparseConv2d, build_neighbor_table

    torch.manual_seed(0)
    rng = np.random.default_rng(21)
    B, T, H, W = 2, 4, 14, 14
    mask = topk_mask(rng, B, T, H, W, 0.4)
    table = build_neighbor_table(torch.from_numpy(mask).to(dev), batched=True)  # global, [B, N, 9]
    nb = table.shape[1]
    dt = _dt(dname)
    m = SparseConv2d(ci, ci).to(dev).to(dt)
    x = torch.randn(B, nb, ci, device=dev, dtype=dt, requires_grad=True)
    go = torch.randn(B, nb, ci, device=dev, dtype=dt)
    with torch.autocast("cuda", dtype=torch.float16, enabled=autocast):
        y = m(x, table)
    y.backward(go)
    run_dt = torch.float16 if autocast else dt
    xr = x.detach().to(run_dt).float().cpu().numpy().reshape(-1, ci)
    wr = m.weight.detach().to(run_dt).float().cpu().numpy()
    br = m.bias.detach().to(run_dt).float().cpu().numpy()
    gr = go.to(run_dt).float().cpu().numpy().reshape(-1, ci)
    t = table.reshape(-1, 9).cpu().numpy()
    tol = TOL["float16" if autocast else dname]
    assert y.dtype == run_dt
    assert _err_ok(oracle, _np32(y).reshape(-1, ci), oracle.fwd(xr, t, wr, br), tol, "y")
    assert _err_ok(oracle, _np32(x.grad).reshape(-1, ci), oracle.bwd_in(gr, t, wr), tol, "x grad")
    assert m.weight.grad.dtype == m.weight.dtype
    assert _err_ok(oracle, _np32(m.weight.grad), oracle.bwd_w(gr, xr, t), tol, "m weight grad")
    assert _err_ok(oracle, _np32(m.bias.grad), oracle.bias_grad(gr), tol, "m bias grad")


def test_module_local_table_heuristic(dev, oracle):
    """A [B, N, 9] table of local indices makes the wrapper pass tokens_per_batch = N."""
    import torch

    from eccv26_tad_amd import SparseConv2d

    rng = np.random.default_rng(4)
    B, T, H, W = 3, 1, 9, 9
    mask = np.zeros((B, 81), np.uint8)
    for b in range(B):
        mask[b, rng.permutation(81)[:30]] = 1
    t = oracle.build_table(mask.reshape(B, T, H, W))
    local = t.reshape(B, 30, 9).copy()
    for b in range(B):
        blk = local[b]
        blk[blk >= 0] -= b * 30
    m = SparseConv2d(16, 16).to(dev)
    x = torch.randn(B, 30, 16, device=dev)
    y_local = m(x, torch.from_numpy(local).to(dev))
    y_global = m(x, torch.from_numpy(t.reshape(B, 30, 9)).to(dev))
    assert torch.allclose(y_local, y_global, rtol=0, atol=0)


@pytest.mark.parametrize("dname", ["float16", "bfloat16"])
def test_module_packed_weight_cache(dev, oracle, dname, monkeypatch):
    """The module's packed-weight cache: a forward on an unchanged weight
    (inference, a checkpointed recompute) packs nothing and gives the same bits
    as a module that packs on every call; an in-place weight update, a new
    dtype under autocast or invalidate() repack, and the results follow the
    oracle."""
    import torch
    import torch.utils.checkpoint as ckpt

    import eccv26_tad_amd.sparse_conv_layer as scl
    from eccv26_tad_amd import SparseConv2d, build_neighbor_table

    calls = []
    real_pack = scl._ops.pack_weight

    def counting_pack(*a):
        calls.append(a[1:])
        return real_pack(*a)

    monkeypatch.setattr(scl._ops, "pack_weight", counting_pack)
    torch.manual_seed(3)
    rng = np.random.default_rng(17)
    dt = _dt(dname)
    mask = topk_mask(rng, 2, 4, 14, 14, 0.55)
    table = build_neighbor_table(torch.from_numpy(mask).to(dev), batched=True)
    nb, c = table.shape[1], 192
    m = SparseConv2d(c, c).to(dev).to(dt)
    ref = SparseConv2d(c, c).to(dev).to(dt)
    ref.packed_weight_cache = None
    ref.load_state_dict(m.state_dict())
    x = torch.randn(2, nb, c, device=dev, dtype=dt)
    go = torch.randn(2, nb, c, device=dev, dtype=dt)
    t = table.reshape(-1, 9).cpu().numpy()

    def oracle_ok(y, w, what):
        xr, wr, br = (_np32(a) for a in (x.reshape(-1, c), w, m.bias))
        return _err_ok(oracle, _np32(y).reshape(-1, c), oracle.fwd(xr, t, wr, br), TOL[dname], what)

    # inference: one pack (forward layout only) for three forwards
    with torch.no_grad():
        calls.clear()
        ys = [m(x, table) for _ in range(3)]
        assert calls == [(True, False)]
        y_ref = ref(x, table)
    for y in ys:
        assert torch.equal(y, y_ref)
    assert oracle_ok(ys[0], m.weight, "inference")

    # an in-place update bumps the version counter: repack, new result
    with torch.no_grad():
        m.weight.mul_(0.5)
        ref.weight.mul_(0.5)
        calls.clear()
        y2 = m(x, table)
        assert len(calls) == 1
        assert torch.equal(y2, ref(x, table))
        assert not torch.equal(y2, ys[0])
    assert oracle_ok(y2, m.weight, "after weight update")

    # training step with activation checkpointing: the recompute reuses the
    # layouts the first forward packed (both, as x needs a gradient)
    xg = x.clone().requires_grad_(True)
    xr_ = x.clone().requires_grad_(True)
    calls.clear()
    y = ckpt.checkpoint(m, xg, table, use_reentrant=False)
    y.backward(go)
    assert calls == [(True, True)]
    yr = ref(xr_, table)
    yr.backward(go)
    assert torch.equal(y, yr)
    assert torch.equal(xg.grad, xr_.grad)
    assert torch.equal(m.weight.grad, ref.weight.grad)
    assert torch.equal(m.bias.grad, ref.bias.grad)

    # a write through .data is not seen by the version counter; invalidate() repacks
    with torch.no_grad():
        m.weight.data.mul_(2.0)
        m.packed_weight_cache.invalidate()
        calls.clear()
        y3 = m(x, table)
        assert len(calls) == 1
    assert oracle_ok(y3, m.weight, "after invalidate")

    # autocast to the other half type packs that dtype's layout
    other = torch.bfloat16 if dt == torch.float16 else torch.float16
    m32 = SparseConv2d(c, c).to(dev)
    x32 = x.float()
    with torch.no_grad(), torch.autocast("cuda", dtype=dt):
        calls.clear()
        a = m32(x32, table)
        b = m32(x32, table)
        assert len(calls) == 1 and torch.equal(a, b)
    with torch.no_grad(), torch.autocast("cuda", dtype=other):
        calls.clear()
        o = m32(x32, table)
        assert len(calls) == 1 and o.dtype == other


# ---------------------------------------------------------------------------
# depthwise
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dname", ["float32", "float16", "bfloat16", "float64"])
def test_depthwise_vs_oracle(dev, oracle, dname):
    import opentad_sparse_ops as ops

    dt = _dt(dname)
    rng = np.random.default_rng(31)
    mask = topk_mask(rng, 2, 4, 14, 14, 0.55)
    n, c = int(mask.sum()), 192
    t = oracle.build_table(mask)
    x = _rounded(rng.standard_normal((n, c)).astype(np.float32), dt)
    w = _rounded(rng.standard_normal((9, c)).astype(np.float32) * 0.3, dt)
    b = _rounded(rng.standard_normal(c).astype(np.float32), dt)
    go = _rounded(rng.standard_normal((n, c)).astype(np.float32), dt)
    X, W, Bb, G = (_t(a, dev, dt) for a in (x, w, b, go))
    T = _t(t, dev, _dt("int32"))
    tol = TOL[dname]
    y = ops.dw_fwd(X, T, W, Bb, 0)
    assert _err_ok(oracle, y.cpu().double().numpy(), oracle.dw_fwd(x, t, w, b), tol, "y")
    gi = ops.dw_bwd_in(G, T, W, 0)
    assert _err_ok(oracle, gi.cpu().double().numpy(), oracle.dw_bwd_in(go, t, w), tol, "gi")
    gw, gb = ops.dw_bwd_w(G, X, T, 0, True)
    assert _err_ok(oracle, gw.cpu().double().numpy(), oracle.dw_bwd_w(go, x, t), tol, "gw")
    assert _err_ok(oracle, gb.cpu().double().numpy(), oracle.bias_grad(go), tol, "gb")


def test_depthwise_module_grad(dev, oracle):
    import torch

    from eccv26_tad_amd import SparseDepthwiseConv2d

    rng = np.random.default_rng(5)
    mask = random_mask(rng, 1, 3, 8, 8, 0.5)
    t = oracle.build_table(mask)
    n = t.shape[0]
    m = SparseDepthwiseConv2d(24).to(dev)
    x = torch.randn(n, 24, device=dev, requires_grad=True)
    y = m(x, torch.from_numpy(t).to(dev))
    go = torch.randn_like(y)
    y.backward(go)
    w = m.weight.detach().cpu().numpy()
    xn, gn = x.detach().cpu().numpy(), go.cpu().numpy()
    assert oracle.rel_err(_np32(y), oracle.dw_fwd(xn, t, w, m.bias.detach().cpu().numpy())) <= 1e-5
    assert oracle.rel_err(_np32(x.grad), oracle.dw_bwd_in(gn, t, w)) <= 1e-5
    assert oracle.rel_err(_np32(m.weight.grad), oracle.dw_bwd_w(gn, xn, t)) <= 1e-5


@pytest.mark.parametrize("dname,c,tpb", [("float16", 192, 0), ("bfloat16", 64, 0), ("float32", 24, 0),
                                          ("float64", 8, 0), ("float16", 192, 1)])
def test_depthwise_one_pass_backward(dev, oracle, dname, c, tpb):
    """dw_bwd (one pass over the rows + one reduction) against dw_bwd_in +
    dw_bwd_w on mask-built tables, global and per-sample (tokens_per_batch)
    indices: weight and bias gradients bit for bit (same row lanes, same
    order); the input gradient bit for bit except float16, where the two
    kernels' compiled multiply-adds leave a few elements 1 ulp apart; and the
    oracle on a table with asymmetric entries (the reduction's orphan
    pass)."""
    import torch

    import opentad_sparse_ops as ops

    dt = _dt(dname)
    rng = np.random.default_rng(c + tpb)
    B, Tn = 2, 5
    mask = topk_mask(rng, B, Tn, 14, 14, 0.55)
    t = oracle.build_table(mask)
    n = t.shape[0]
    x = _rounded(rng.standard_normal((n, c)).astype(np.float32), dt)
    w = _rounded(rng.standard_normal((9, c)).astype(np.float32) * 0.3, dt)
    go = _rounded(rng.standard_normal((n, c)).astype(np.float32), dt)
    X, W, G = (_t(a, dev, dt) for a in (x, w, go))
    tab, tpb_v = t, 0
    if tpb:  # per-sample indices: equal kept counts per sample
        tpb_v = n // B
        tab = t.copy()
        tab[tab >= 0] %= tpb_v
    T = _t(tab, dev, _dt("int32"))
    _say("dw one-pass", dname, c, tpb_v)
    gi, gw, gb = ops.dw_bwd(G, X, T, W, tpb_v, True)
    gi2 = ops.dw_bwd_in(G, T, W, tpb_v)
    gw2, gb2 = ops.dw_bwd_w(G, X, T, tpb_v, True)
    assert torch.equal(gw, gw2) and torch.equal(gb, gb2)
    if dt == torch.float16:
        # the compiler's choice of fp16 multiply-add instructions differs
        # between the two kernels: a few elements 1 ulp apart
        d = (gi.double() - gi2.double()).abs()
        assert float(d.max()) <= 2e-3 * float(gi2.double().abs().max())
        assert int(torch.count_nonzero(d)) <= gi.numel() // 1000
    else:
        assert torch.equal(gi, gi2)
    gi3, gw3, gb3 = ops.dw_bwd(G, X, T, W, tpb_v, False)
    assert gb3.numel() == 0 and torch.equal(gi3, gi) and torch.equal(gw3, gw2)
    tol = TOL[dname]
    assert _err_ok(oracle, gi.cpu().double().numpy(), oracle.dw_bwd_in(go, t, w), tol, "gi")
    assert _err_ok(oracle, gw.cpu().double().numpy(), oracle.dw_bwd_w(go, x, t), tol, "gw")
    # asymmetric entries: every 7th row points one entry at a random row
    asym = t.copy()
    for i in range(0, n, 7):
        asym[i, int(rng.integers(0, 9))] = int(rng.integers(0, n))
    Ta = _t(asym, dev, _dt("int32"))
    gia, gwa, gba = ops.dw_bwd(G, X, Ta, W, 0, True)
    assert _err_ok(oracle, gia.cpu().double().numpy(), oracle.dw_bwd_in(go, asym, w), tol, "gia")
    assert _err_ok(oracle, gwa.cpu().double().numpy(), oracle.dw_bwd_w(go, x, asym), tol, "gwa")
    assert _err_ok(oracle, gba.cpu().double().numpy(), oracle.bias_grad(go), tol, "gba")
    # the rows reached by the one-way entries: one rounding, the same bits
    # on every run and through the separate backward-input call
    n_oneway = _one_way_entries(asym)
    _say(f"  {n_oneway} one-way entries")
    assert 0 < n_oneway <= 2048
    assert torch.equal(gia, ops.dw_bwd(G, X, Ta, W, 0, True)[0])
    _assert_rounded_once(gia, oracle.dw_bwd_in(go, asym, w), oracle.dw_bwd_in(np.abs(go), asym, np.abs(w)), dt)
    # a symmetric table again after the asymmetric one (flag words rewritten)
    gi4, _, _ = ops.dw_bwd(G, X, T, W, tpb_v, True)
    assert torch.equal(gi4, gi)


@pytest.mark.parametrize("dname,c", [("float32", 192), ("float32", 8), ("bfloat16", 64)])
def test_depthwise_one_pass_backward_row_chunks(dev, dname, c):
    """Splits longer than one LDS chunk of rows (141,120 rows, 552 per split):
    the one-pass backward still equals the two separate calls bit for bit."""
    import torch

    import eccv26_tad_amd as sv
    import opentad_sparse_ops as ops

    dt = _dt(dname)
    g = torch.Generator().manual_seed(c)
    mask = torch.ones(1, 720, 14, 14, dtype=torch.uint8)
    mask.view(-1)[torch.randperm(mask.numel(), generator=g)[:40]] = 0  # a few holes
    T = sv.build_neighbor_table(mask.to(dev))
    n = T.shape[0]
    _say("dw one-pass chunks", dname, c, n)
    x = torch.randn(n, c, generator=g).to(dev, dt)
    go = torch.randn(n, c, generator=g).to(dev, dt)
    w = (torch.randn(9, c, generator=g) * 0.3).to(dev, dt)
    gi, gw, gb = ops.dw_bwd(go, x, T, w, 0, True)
    gi2 = ops.dw_bwd_in(go, T, w, 0)
    gw2, gb2 = ops.dw_bwd_w(go, x, T, 0, True)
    assert torch.equal(gi, gi2) and torch.equal(gw, gw2) and torch.equal(gb, gb2)


# ---------------------------------------------------------------------------
# determinism
# ---------------------------------------------------------------------------

BW_TR_CASES = [
    # (shape B,T,H,W), keep, C_in, C_out, dtype: the tile configurations of
    # the transposed-read backward-weight kernel (192 x 192, 128 x 256,
    # 128 x 128 tiles), several tiles per split, empty and short splits
    ((2, 8, 14, 14), 0.55, 192, 192, "float16"),
    ((2, 8, 14, 14), 0.1, 192, 192, "bfloat16"),
    ((1, 4, 16, 16), 0.5, 256, 256, "bfloat16"),
    ((1, 4, 16, 16), 0.4, 128, 128, "float16"),
    ((1, 3, 14, 14), 0.7, 384, 384, "float16"),
    ((1, 1, 5, 7), 0.3, 192, 192, "float16"),
]


@pytest.mark.skip(reason="the transposed-read backward-weight kernel (loads straight into LDS, "
                         "ds_read_b64_tr_b16 fragments) made a GPU memory fault on its first case; "
                         "no cause was found on the CPU, so the kernel was taken out and this "
                         "comparison does not run")
@pytest.mark.parametrize("case", BW_TR_CASES, ids=lambda c: f"{c[0]}-{c[1]}-{c[2]}x{c[3]}-{c[4]}")
def test_bw_transposed_read_kernel_matches_staging_kernel(dev, oracle, case, monkeypatch):
    """The backward-weight partials from LDS transposing reads (default) and
    from the staging-wave kernel (SVTAD_BW_TR=0) take the same MFMA inputs in
    the same order: bit-identical weight gradients. The bias is summed
    differently (an MFMA against ones vs dot2 row groups): both against the
    oracle."""
    import torch

    import opentad_sparse_ops as ops

    shape, keep, ci, co, dname = case
    dt = _dt(dname)
    mask, x, w, b, go = _conv_case(41, shape, keep, ci, co, dt)
    t = oracle.build_table(mask)
    x, go = _rounded(x, dt), _rounded(go, dt)
    X, G, T = _t(x, dev, dt), _t(go, dev, dt), torch.from_numpy(t).to(dev)
    _say(f"bw kernels {case} n={x.shape[0]}")
    monkeypatch.delenv("SVTAD_BW_TR", raising=False)
    gw_tr, gb_tr = ops.bwd_w_bias(G, X, T, ci, 0, True)
    torch.cuda.synchronize()
    monkeypatch.setenv("SVTAD_BW_TR", "0")
    gw_st, gb_st = ops.bwd_w_bias(G, X, T, ci, 0, True)
    torch.cuda.synchronize()
    monkeypatch.delenv("SVTAD_BW_TR")
    assert torch.equal(gw_tr, gw_st)
    tol = TOL[dname]
    assert _err_ok(oracle, _np32(gw_tr), oracle.bwd_w(go, x, t), tol, "gw")
    assert _err_ok(oracle, _np32(gb_tr), oracle.bias_grad(go), tol, "gb (transposed reads)")
    assert _err_ok(oracle, _np32(gb_st), oracle.bias_grad(go), tol, "gb (staging waves)")
    # the linear layers' weight gradient runs the same kernel with one offset
    rows = torch.from_numpy(np.random.default_rng(5).integers(0, x.shape[0], x.shape[0]).astype(np.int32)).to(dev)
    wg_tr = ops.linear_wgrad(G, rows, X)
    monkeypatch.setenv("SVTAD_BW_TR", "0")
    wg_st = ops.linear_wgrad(G, rows, X)
    monkeypatch.delenv("SVTAD_BW_TR")
    assert torch.equal(wg_tr, wg_st)


def test_backward_is_deterministic(dev, oracle):
    import opentad_sparse_ops as ops
    import torch

    mask, x, w, b, go = _conv_case(41, (2, 8, 14, 14), 0.5, 192, 192, "float16")
    t = oracle.build_table(mask)
    X, W, G = (_t(a, dev, torch.float16) for a in (x, w, go))
    T = _t(t, dev, torch.int32)
    a1 = ops.bwd_in(G, T, W, x.shape[0], 192, 0)
    a2 = ops.bwd_in(G, T, W, x.shape[0], 192, 0)
    w1 = ops.bwd_w(G, X, T, 192, 0)
    w2 = ops.bwd_w(G, X, T, 192, 0)
    assert torch.equal(a1, a2) and torch.equal(w1, w2)


@pytest.mark.parametrize("ci,co,dname", [(192, 192, "float16"), (256, 256, "bfloat16"), (128, 96, "float16")])
def test_packed_entry_points_match(dev, oracle, ci, co, dname):
    """pack_weight + fwd_packed / bwd_in_packed (the autograd path) give exactly
    what fwd_bias / bwd_in give (same kernels, same order)."""
    import opentad_sparse_ops as ops
    import torch

    _say("packed", ci, co, dname)
    dt = _dt(dname)
    mask, x, w, b, go = _conv_case(11, (2, 6, 14, 14), 0.55, ci, co, dname)
    t = oracle.build_table(mask)
    X, W, Bb, G = (_t(a, dev, dt) for a in (x, w, b, go))
    T = _t(t, dev, _dt("int32"))
    pf, pb = ops.pack_weight(W, True, True)
    # a layout exists for reduction widths 64/128/192/256/512; C_out = 96 has
    # none for backward-input (empty tensor -> the per-call path)
    assert pf.numel() > 0 and (pb.numel() > 0) == (co in (64, 128, 192, 256, 512))
    for mode in (0, 1, 2):
        assert torch.equal(ops.fwd_packed(X, T, W, pf, Bb, 0, mode), ops.fwd_bias(X, T, W, Bb, 0, mode))
    assert torch.equal(ops.bwd_in_packed(G, T, W, pb, x.shape[0], ci, 0), ops.bwd_in(G, T, W, x.shape[0], ci, 0))
    # empty packed tensors fall back to the per-call path
    empty = torch.empty(0, dtype=torch.uint8, device=dev)
    assert torch.equal(ops.fwd_packed(X, T, W, empty, Bb, 0, 1), ops.fwd_bias(X, T, W, Bb, 0, 1))
    f32 = W.float()
    pf32, pb32 = ops.pack_weight(f32, True, True)
    assert pf32.numel() == 0 and pb32.numel() == 0
