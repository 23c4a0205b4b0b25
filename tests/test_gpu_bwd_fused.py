"""The one-launch backward (backward-input tiles and backward-weight partials
in one grid, then the ordered reduction) at the full c2 shape, C = 192, and
at config 4's, C = 256.

svtad_bwd_packed takes it where both grids together fit one workgroup per
CU (10 %, 25 % and 40 % keep at c2, 10 % at c4, with fewer row splits where
needed);
SVTAD_BWD_FUSED=off turns it off and "<gfm>x<gfn>[:<splits>]" forces a tile
shape and split count. Checked:

* forced tiles with the two-launch path's row tile: grad_x bit-identical
  (same row tiles, same offsets per wave set). The one-launch backward
  splits the center offset in four units per split, not two, and takes
  fewer splits, so the weight and bias gradients sum in another order;
* the automatic choice (which may take fewer splits), other row tiles and
  forced split counts: within one rounding of the two-launch path, and every
  result against the fp64 oracle at the north-star bar;
* an asymmetric table (orphan entries: the flag set inside the launch, the
  orphan pass in the reduction) against the oracle;
* a forced shape outside the instantiated ones is rejected before any launch.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest

from tests.helpers import kaiming_weight, topk_mask
from tests.test_gpu_fullsize import _gw_fp64, _sub_bwd_in

pytestmark = pytest.mark.gpu

TOL = 1e-2  # max-scaled error bar of the north star (f16 / bf16)


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _problem(dev, oracle, keep, dname, seed, drop=0.0, per_sample=False, c=192, grid=(2, 80, 14, 14)):
    """Config 2's grid and width by default; config 4 is c=256, grid
    (2, 96, 16, 16)."""
    import torch

    import eccv26_tad_amd as sv

    dt = {"float16": torch.float16, "bfloat16": torch.bfloat16}[dname]
    rng = np.random.default_rng(seed)
    mask = topk_mask(rng, *grid, keep)
    t = oracle.build_table(mask)
    if drop > 0:  # one side of some symmetric pairs removed: orphan entries
        off = (t >= 0) & (rng.random(t.shape) < drop)
        off[:, 4] = False
        t = np.where(off, -1, t).astype(np.int32)
    n = t.shape[0]
    tab, tpb = t, 0
    if per_sample:  # per-sample indices (tokens_per_batch): equal kept counts per sample
        tpb = n // 2
        tab = t.copy()
        tab[tab >= 0] %= tpb

    def rounded(a):
        return torch.from_numpy(a).to(dt).float().numpy()

    x = rounded(rng.standard_normal((n, c)).astype(np.float32))
    w = rounded(kaiming_weight(rng, c, c))
    go = rounded(rng.standard_normal((n, c)).astype(np.float32))
    X, W, G = (torch.from_numpy(a).to(dev, dt) for a in (x, w, go))
    T = torch.from_numpy(tab).to(dev)
    return sv.ops, dict(x=x, w=w, go=go, t=t, X=X, W=W, G=G, T=T, n=n, c=c, rng=rng, tpb=tpb)


def _bwd(ops, P, monkeypatch, mode):
    import torch

    if mode is None:
        monkeypatch.delenv("SVTAD_BWD_FUSED", raising=False)
    else:
        monkeypatch.setenv("SVTAD_BWD_FUSED", mode)
    _, pb = ops.pack_weight(P["W"], False, True)
    gi, gw, gb = ops.bwd_packed(P["G"], P["X"], P["T"], P["W"], pb, P["c"], P["tpb"], True)
    torch.cuda.synchronize()
    monkeypatch.delenv("SVTAD_BWD_FUSED", raising=False)
    return [a.float().cpu().numpy() for a in (gi, gw, gb)]


def _oracle_errs(oracle, P, res):
    gi, gw, gb = res
    rows = np.sort(P["rng"].choice(P["n"], size=min(2048, P["n"]), replace=False))
    return {
        "grad_x": oracle.rel_err(gi[rows], _sub_bwd_in(oracle, P["go"], P["t"], P["w"], rows)),
        "grad_w": oracle.rel_err(gw, _gw_fp64(P["go"], P["x"], P["t"])),
        "grad_b": oracle.rel_err(gb, P["go"].astype(np.float64).sum(0)),
    }


def _scaled(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


# Tile shapes with the row tile of the two-launch backward-input at that N
# (three row fragments below 40 % keep, four at 40 %) give grad_x bit for
# bit. Every mode's weight and bias gradients (other splits, the center in
# four parts) and the other shapes' grad_x sum in another order.
@pytest.mark.parametrize("keep,dname,same,other", [
    (0.10, "float16", ("3x1", "3x3"), (None, "4x3", "3x3:4")),
    (0.25, "float16", ("3x1", "3x3"), (None, "4x3", "3x3:4")),
    (0.10, "bfloat16", ("3x1", "3x3"), (None, "4x3", "3x3:4")),
    (0.40, "float16", ("4x3",), (None, "3x3", "4x3:5")),
])
def test_fused_matches_two_launch(dev, oracle, monkeypatch, keep, dname, same, other):
    ops, P = _problem(dev, oracle, keep, dname, 3100 + int(keep * 100))
    _say(f"fused backward, keep {keep} {dname}, n = {P['n']}")
    ref = _bwd(ops, P, monkeypatch, "off")
    for mode in same:
        got = _bwd(ops, P, monkeypatch, mode)
        assert np.array_equal(got[0], ref[0]), (mode, "grad_x", _scaled(got[0], ref[0]))
    _say(f"  {', '.join(same)}: grad_x bit-identical to the two-launch path")
    for mode in (*same, *other):
        got = _bwd(ops, P, monkeypatch, mode)
        d = {k: _scaled(a, b) for k, a, b in zip(("grad_x", "grad_w", "grad_b"), got, ref)}
        e = _oracle_errs(oracle, P, got)
        _say(f"  {mode or 'automatic'}: vs two-launch", {k: f"{v:.2e}" for k, v in d.items()},
             "vs oracle", {k: f"{v:.2e}" for k, v in e.items()}, f"(bar {TOL:g})")
        for k, v in d.items():
            assert v <= 4e-3, (mode, k, v)
        for k, v in e.items():
            assert v <= TOL, (mode, k, v)
    e = _oracle_errs(oracle, P, ref)
    _say("  two-launch vs oracle", {k: f"{v:.2e}" for k, v in e.items()})
    for k, v in e.items():
        assert v <= TOL, (k, v)


@pytest.mark.parametrize("keep", [0.10, 0.25])
def test_fused_per_sample_table(dev, oracle, monkeypatch, keep):
    """Per-sample neighbor indices (tokens_per_batch = n / B): the one-launch
    backward's grad_x equals the two-launch path's bit for bit with the same
    tile, its weight and bias gradients within one rounding, and every result
    the oracle's (on the global form of the same table)."""
    ops, P = _problem(dev, oracle, keep, "float16", 3500 + int(keep * 100), per_sample=True)
    _say(f"fused backward, per-sample table, keep {keep}, n = {P['n']}, tpb = {P['tpb']}")
    ref = _bwd(ops, P, monkeypatch, "off")
    got = _bwd(ops, P, monkeypatch, "3x1")
    assert np.array_equal(got[0], ref[0]), _scaled(got[0], ref[0])
    for name, a, b in zip(("grad_w", "grad_b"), got[1:], ref[1:]):
        assert _scaled(a, b) <= 4e-3, (name, _scaled(a, b))
    got = _bwd(ops, P, monkeypatch, None)
    e = _oracle_errs(oracle, P, got)
    _say("  automatic vs oracle", {k: f"{v:.2e}" for k, v in e.items()}, f"(bar {TOL:g})")
    for k, v in e.items():
        assert v <= TOL, (k, v)


def test_fused_config4(dev, oracle, monkeypatch):
    """Config 4 at 10 % keep (C = 256 bf16, N = 4916): 128-column tiles of
    three row fragments beside 128 x 256 backward-weight units, the center
    offset in four units per split. The backward-input tiles are the two
    launches' (grad_x bit for bit); the weight and bias gradients sum over
    other splits and parts. The automatic choice takes 2 splits."""
    ops, P = _problem(dev, oracle, 0.10, "bfloat16", 3600, c=256, grid=(2, 96, 16, 16))
    _say(f"fused backward, config 4, n = {P['n']}")
    ref = _bwd(ops, P, monkeypatch, "off")
    for mode in (None, "3x2", "3x2:3"):
        got = _bwd(ops, P, monkeypatch, mode)
        d = {k: _scaled(a, b) for k, a, b in zip(("grad_x", "grad_w", "grad_b"), got, ref)}
        e = _oracle_errs(oracle, P, got)
        _say(f"  {mode or 'automatic'}: vs two-launch", {k: f"{v:.2e}" for k, v in d.items()},
             "vs oracle", {k: f"{v:.2e}" for k, v in e.items()}, f"(bar {TOL:g})")
        assert np.array_equal(got[0], ref[0]), mode
        for k, v in d.items():
            assert v <= 4e-3, (mode, k, v)
        for k, v in e.items():
            assert v <= TOL, (mode, k, v)


def test_fused_orphans(dev, oracle, monkeypatch):
    """An asymmetric table at 10 % keep: the orphan entries reach grad_x
    through the flag set in the one-launch backward."""
    ops, P = _problem(dev, oracle, 0.10, "float16", 3300, drop=0.2)
    _say(f"fused backward, asymmetric table, n = {P['n']}")
    ref = _bwd(ops, P, monkeypatch, "off")
    for mode in (None, "3x1"):
        got = _bwd(ops, P, monkeypatch, mode)
        e = _oracle_errs(oracle, P, got)
        d = _scaled(got[0], ref[0])
        _say(f"  {mode or 'automatic'}: grad_x vs two-launch {d:.2e}, vs oracle",
             {k: f"{v:.2e}" for k, v in e.items()}, f"(bar {TOL:g})")
        assert d <= 4e-3, (mode, d)
        # other splits and the center in four parts: another summation order
        assert _scaled(got[1], ref[1]) <= 4e-3 and _scaled(got[2], ref[2]) <= 4e-3, mode
        for k, v in e.items():
            assert v <= TOL, (mode, k, v)


def test_fused_without_bias(dev, oracle, monkeypatch):
    """with_bias=False (no bias partials, no bias reduction): the same input
    and weight gradients as with the bias, bit for bit, and no bias output."""
    import torch

    ops, P = _problem(dev, oracle, 0.10, "float16", 3700)
    monkeypatch.delenv("SVTAD_BWD_FUSED", raising=False)
    _, pb = ops.pack_weight(P["W"], False, True)
    gi, gw, gb = ops.bwd_packed(P["G"], P["X"], P["T"], P["W"], pb, P["c"], 0, True)
    gi2, gw2, gb2 = ops.bwd_packed(P["G"], P["X"], P["T"], P["W"], pb, P["c"], 0, False)
    torch.cuda.synchronize()
    assert gb2.numel() == 0 and gb.numel() == P["c"]
    assert torch.equal(gi, gi2) and torch.equal(gw, gw2)


def test_fused_step_in_hip_graph(dev, oracle, monkeypatch):
    """The training step at 10 % keep (pack, forward, one-launch backward,
    reduction) captured in a HIP graph: every replay, with eager work and
    synchronisations between them, equals the eager step bit for bit."""
    import torch

    ops, P = _problem(dev, oracle, 0.10, "float16", 3800)
    monkeypatch.delenv("SVTAD_BWD_FUSED", raising=False)
    c = P["c"]
    b = torch.linspace(-0.1, 0.1, c, device=dev).half()

    def step():
        pf, pb = ops.pack_weight(P["W"], True, True)
        y = ops.fwd_packed(P["X"], P["T"], P["W"], pf, b, 0, 1)
        gi, gw, gb = ops.bwd_packed(P["G"], P["X"], P["T"], P["W"], pb, c, 0, True)
        return y, gi, gw, gb

    ref = [a.clone() for a in step()]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = step()
    for r in range(3):
        g.replay()
        torch.cuda.synchronize()
        for a, e in zip(out, ref):
            assert torch.equal(a, e), r
        step()  # eager work between replays
        torch.cuda.synchronize()
    _say("  three graph replays equal the eager step")


def test_fused_bad_forced_shape(dev, oracle, monkeypatch):
    ops, P = _problem(dev, oracle, 0.10, "float16", 3400)
    with pytest.raises(RuntimeError, match="SVTAD_BWD_FUSED"):
        _bwd(ops, P, monkeypatch, "5x3")
