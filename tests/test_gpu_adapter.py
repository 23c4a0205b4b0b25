"""The fused sparse-conv adapter against an independent float32 restatement
of the reference adapter (``tests/adapter_ref.py``: the chain of
vit_sparse_adapter_poguise.py:288-362,511-653 in PyTorch float32 ops, its
convolution on the dense ``2d_conv`` path, which the CPU oracle pins) on the
same rounded weights and inputs: output and every gradient (x, down_proj,
up_proj, gamma, the sparse conv's weight and bias, and the attention /
heatmap parameters of those variants).

The bar does not depend on the draw. Every case runs on five seeds, and for
every draw the module also runs the reference's own unfused chain in the same
precision (``reference_forward``: the op order of vit_sparse_adapter_poguise.py
with PyTorch's float16 / bfloat16 ops, or its autocast casts), measured
against the same float32 restatement (max-scaled errors; a scalar gain's
gradient against the sum of its absolute terms). For every quantity:

* the mean of the fused path's five errors is at most ``max(1e-2, 1.5 x``
  the mean of the chain's``)``;
* each fused error is at most ``max(1e-2, 2 x`` the chain's largest``)``.

One draw's chain error is not a stable yardstick: where the bfloat16
attention ops dominate (LayerNorm, softmax and their gradients, which both
paths run as the same PyTorch ops) it moves by about 2x from draw to draw,
and so does the fused path's on the same quantity. The mean over five draws
is stable; the per-draw ceiling catches a single bad draw. Both errors are
printed for every draw.

Shapes: the ViT-B adapter (embed 768, hidden 256 after the reference's
power-of-two rounding) on B2 x T80 x 14x14 at 55 % keep with one CLS token,
a small case with no special token, every ``use_attn`` variant (1, 2, 3, 4)
and the heatmap injection on the same grid and on a resized heatmap grid; in
float16 and bfloat16 modules, and under ``torch.autocast(bfloat16)`` with
float32 parameters, the way the reference trains and tests
(opentad/cores/train_engine.py:672, opentad/cores/test_engine.py:63).
"""
from __future__ import annotations

import contextlib

import numpy as np
import pytest
import torch

from tests.adapter_ref import adapter_fp32, gain_scales
from tests.helpers import topk_mask

pytestmark = pytest.mark.gpu

SEEDS = (0, 1, 2, 3, 4)


def _err(got, ref):
    got, ref = got.double(), ref.double()
    return float((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30))


def _setup(dev, dt, B, T, H, W, keep, embed, mlp_ratio, S, seed, **variant):
    import eccv26_tad_amd as sv

    rng = np.random.default_rng(seed)
    mask = topk_mask(rng, B, T, H, W, keep)
    flat = mask.reshape(B, -1)
    idx = torch.from_numpy(np.stack([np.flatnonzero(flat[b]) for b in range(B)])).to(dev)
    table = sv.build_neighbor_table(torch.from_numpy(mask).to(dev)).view(B, -1, 9)
    g = torch.Generator().manual_seed(seed)
    torch.manual_seed(seed)  # the module's own initialisation draws from the global generator
    mod = sv.SparseConvAdapter(embed, mlp_ratio, **variant)
    with torch.no_grad():
        # non-trivial values where the init leaves zeros or ones (up_proj,
        # gamma, the gates, the attention MLP's last layer, the biases)
        for name, p in mod.named_parameters():
            if name in ("gamma", "attn_gamma"):
                p.fill_(0.75)
            elif name == "heatmap_gate":
                p.fill_(0.6)
            elif name.startswith("up_proj") or name.startswith("attn_mlp.3") or name.endswith("bias"):
                p.copy_(torch.randn(p.shape, generator=g) * (0.05 if p.dim() > 1 else 0.1))
            elif "norm" in name and name.endswith("weight"):
                p.copy_(1.0 + torch.randn(p.shape, generator=g) * 0.1)
    mod = mod.to(dev, dt)
    N = S + idx.shape[1]
    x = torch.randn(B, N, embed, generator=g).to(dev, dt)
    go = torch.randn(B, N, embed, generator=g).to(dev, dt)
    return mod, idx, table, x, go


def _fp32_reference(mod, idx, table, x, go, H, W, T):
    """adapter_fp32's output, x gradient, parameter gradients and gain scales
    for the module's (rounded) parameters and the given x and go."""
    xr = x.detach().float().requires_grad_(True)
    gains = {}
    yr, P = adapter_fp32(mod, xr, H, W, idx, T * H * W, gains)
    yr.backward(go.detach().float())
    return yr.detach(), xr.grad, P, gain_scales(gains)


def _errors(y, gx, mod, ref):
    """Max-scaled errors of an output, its x gradient and the module's
    parameter gradients (``.grad``) against ``_fp32_reference``'s."""
    yr, gxr, P, scales = ref
    errs = {"y": _err(y, yr), "x": _err(gx, gxr)}
    for name, p in mod.named_parameters():
        if P[name].grad is None:
            # not on the forward path (attn_gamma of the temporal variant)
            assert p.grad is None, name
            continue
        assert p.grad is not None and p.grad.dtype == p.dtype, name
        if name in scales:
            # a scalar gain's gradient is one sum over every token and
            # channel with heavy cancellation: its error is measured against
            # the sum of the absolute terms (as test_gamma_grad does)
            errs[name] = abs(float(p.grad) - float(P[name].grad)) / max(scales[name], 1e-30)
        elif name == "k_norm.bias":
            # exactly zero: the bias shifts every key's score of a query by the
            # same q.b, which the softmax cancels; both sides hold rounding
            # noise, so it is measured against the k_norm weight's gradient
            errs[name] = float(p.grad.double().abs().max() /
                               P["k_norm.weight"].grad.double().abs().max().clamp_min(1e-30))
        else:
            errs[name] = _err(p.grad, P[name].grad)
    return errs


def _run(mod, fn, x, go, amp):
    """Forward ``fn(x)`` (under ``torch.autocast(amp)`` when amp is a dtype)
    and backward with ``go`` in the output's dtype; returns the output, x's
    gradient and the output dtype. The module's gradients are left in
    ``.grad``."""
    mod.zero_grad(set_to_none=True)
    xf = x.detach().clone().requires_grad_(True)
    ctx = torch.autocast("cuda", dtype=amp) if amp is not None else contextlib.nullcontext()
    with ctx:
        y = fn(xf)
    y.backward(go.detach().to(y.dtype))
    return y.detach(), xf.grad, y.dtype


def _draw(mod, idx, table, x, go, H, W, T, amp=None):
    """One draw: the fused path and the reference's unfused chain on the same
    module, precision policy and inputs, both against the float32
    restatement. Returns (fused errors, chain errors, fused output dtype)."""
    ref = _fp32_reference(mod, idx, table, x, go, H, W, T)
    with torch.autocast("cuda", dtype=amp) if amp is not None else contextlib.nullcontext():
        assert mod._fused_dtype(x) is not None, "the call would not take the fused path"
    y, gx, ydt = _run(mod, lambda xf: mod(xf, H, W, idx, T * H * W, table), x, go, amp)
    fused = _errors(y, gx, mod, ref)
    yc, gxc, ycdt = _run(mod, lambda xf: mod.reference_forward(xf, H, W, idx, T * H * W, table), x, go, amp)
    chain = _errors(yc, gxc, mod, ref)
    assert ydt == ycdt, (ydt, ycdt)
    print(f"  y {fused['y']:.2e} / {chain['y']:.2e}, x {fused['x']:.2e} / {chain['x']:.2e}; fused / chain:",
          {k: f"{fused[k]:.1e}/{chain[k]:.1e}" for k in fused if k not in ("y", "x")}, flush=True)
    return fused, chain, ydt


def _check_draws(make, amp=None, tol=1e-2):
    """Runs ``_draw`` on ``make(seed)`` = (mod, idx, table, x, go, H, W, T)
    for every seed. Per quantity: the mean fused error is at most max(tol,
    1.5 x the mean chain error), and every fused error at most max(tol, 2 x
    the largest chain error). Returns the fused output dtypes."""
    draws = []
    for seed in SEEDS:
        print(f" seed {seed}", flush=True)
        draws.append(_draw(*make(seed), amp=amp))
    keys = list(draws[0][0])
    mean_f = {k: sum(d[0][k] for d in draws) / len(draws) for k in keys}
    mean_c = {k: sum(d[1][k] for d in draws) / len(draws) for k in keys}
    worst_c = {k: max(d[1][k] for d in draws) for k in keys}
    worst_f = {k: max(d[0][k] for d in draws) for k in keys}
    bar_mean = {k: max(tol, 1.5 * mean_c[k]) for k in keys}
    bar_each = {k: max(tol, 2.0 * worst_c[k]) for k in keys}
    km = max(keys, key=lambda k: mean_f[k] / bar_mean[k])
    ke = max(keys, key=lambda k: worst_f[k] / bar_each[k])
    print(f"  means closest to the bar: {km}: fused {mean_f[km]:.2e}, chain {mean_c[km]:.2e}, bar "
          f"{bar_mean[km]:.2e}; draws: {ke}: fused worst {worst_f[ke]:.2e}, chain worst {worst_c[ke]:.2e}, "
          f"bar {bar_each[ke]:.2e}", flush=True)
    for k in keys:
        assert mean_f[k] <= bar_mean[k], (k, "mean", mean_f[k], mean_c[k])
        assert worst_f[k] <= bar_each[k], (k, "draw", worst_f[k], worst_c[k])
    return [d[2] for d in draws]


@pytest.mark.parametrize("dname", ["float16", "bfloat16"])
@pytest.mark.parametrize("case", [
    dict(B=2, T=80, H=14, W=14, keep=0.55, embed=768, mlp_ratio=0.25, S=1, seed=31),
    dict(B=3, T=4, H=6, W=7, keep=0.3, embed=128, mlp_ratio=0.5, S=0, seed=32),
])
def test_fused_adapter_matches_fp32_reference(dev, dname, case):
    dt = getattr(torch, dname)
    c = dict(case)
    S = c.pop("S")
    print("adapter", dname, c, flush=True)

    def make(seed):
        mod, idx, table, x, go = _setup(dev, dt, S=S, **dict(c, seed=c["seed"] + 100 * seed))
        return mod, idx, table, x, go, c["H"], c["W"], c["T"]

    assert set(_check_draws(make)) == {dt}


def test_fused_adapter_packed_weight_cache(dev):
    """The fused adapter reuses its sparse conv's packed weight while the
    weight is unchanged and repacks after an in-place update: the same bits
    as a copy that packs on every call, and the training step still matches
    the float32 reference after the update."""
    import copy

    mod, idx, table, x, go = _setup(dev, torch.float16, B=3, T=4, H=6, W=7, keep=0.3, embed=128,
                                    mlp_ratio=0.5, S=0, seed=33)
    H, W, T = 6, 7, 4
    cache = mod.sparse_conv.packed_weight_cache
    with torch.no_grad():
        y1 = mod(x, H, W, idx, T * H * W, table)
        first = cache._packed
        y2 = mod(x, H, W, idx, T * H * W, table)
        assert cache._packed is first and first is not None
        assert torch.equal(y1, y2)
        mod.sparse_conv.weight.mul_(0.5)
        y3 = mod(x, H, W, idx, T * H * W, table)
        assert cache._packed is not first
        fresh = copy.deepcopy(mod)
        fresh.sparse_conv.packed_weight_cache = None
        assert torch.equal(y3, fresh(x, H, W, idx, T * H * W, table))
        assert not torch.equal(y3, y1)
    fused, chain, _ = _draw(mod, idx, table, x, go, H, W, T)
    for k in fused:
        assert fused[k] <= max(1e-2, 1.5 * chain[k]), (k, fused[k], chain[k])


# the production configurations set adapter_use_attn to 1, 2 or 3
# (configs/vitsparse/*/...sparse_adapter.py); 4 is the temporal variant
@pytest.mark.parametrize("dname", ["float16", "bfloat16"])
@pytest.mark.parametrize("use_attn,S,embed", [(1, 1, 512), (2, 3, 512), (3, 3, 512), (4, 2, 512), (1, 1, 256)])
def test_attention_variants_match_fp32_reference(dev, dname, use_attn, S, embed):
    """Hidden 128 (the ViT-S width: attention width 64, 4 heads) and hidden 64,
    whose attention width (32) has no tile configuration for the weight
    gradient kernel (a library GEMM then)."""
    dt = getattr(torch, dname)
    B, T, H, W = 2, 6, 7, 8
    print("adapter use_attn", use_attn, dname, "embed", embed, flush=True)

    def make(seed):
        mod, idx, table, x, go = _setup(dev, dt, B, T, H, W, 0.45, embed, 0.25, S, 50 + use_attn + 100 * seed,
                                        use_attn=use_attn, n_key_tokens=S)
        return mod, idx, table, x, go, H, W, T

    _check_draws(make)


@pytest.mark.parametrize("dname", ["float16", "bfloat16"])
@pytest.mark.parametrize("grid", [(7, 8), (3, 4)])
def test_heatmap_injection_matches_fp32_reference(dev, dname, grid):
    """n_key_tokens = 1 + heatmap cells, use_attn = 0: the heatmap gather-add
    on the SparseConv2D input, on the token grid itself and on a smaller
    heatmap grid (nearest-index resize)."""
    dt = getattr(torch, dname)
    B, T, H, W = 2, 6, 7, 8
    S = 1 + grid[0] * grid[1]
    print("adapter heatmap", grid, dname, flush=True)

    def make(seed):
        mod, idx, table, x, go = _setup(dev, dt, B, T, H, W, 0.5, 128, 0.5, S, 60 + grid[0] + 100 * seed,
                                        n_key_tokens=S, heatmap_grid_size=grid)
        assert mod._uses_heatmap()
        return mod, idx, table, x, go, H, W, T

    _check_draws(make)


@pytest.mark.parametrize("variant", [
    dict(use_attn=0, S=1, embed=768, B=2, T=20, H=14, W=14, keep=0.55),
    dict(use_attn=2, S=3, embed=512, n_key_tokens=3, B=2, T=6, H=7, W=8, keep=0.45),
    dict(use_attn=1, S=1, embed=512, n_key_tokens=1, B=2, T=6, H=7, W=8, keep=0.45),
    dict(use_attn=3, S=3, embed=512, n_key_tokens=3, B=2, T=6, H=7, W=8, keep=0.45),
    dict(use_attn=4, S=2, embed=512, n_key_tokens=2, B=2, T=6, H=7, W=8, keep=0.45),
    dict(use_attn=0, S=13, embed=256, n_key_tokens=13, heatmap_grid_size=(3, 4), B=2, T=6, H=7, W=8, keep=0.5),
])
def test_fused_adapter_under_autocast(dev, variant):
    """float32 parameters and input under torch.autocast(bfloat16), the
    reference's training and test mode: the fused path runs (casting x and
    the weights to bfloat16 inside its nodes), the output is float32 (gamma is
    a float32 parameter) and every parameter receives a float32 gradient,
    within the bar set by the reference's own autocast chain on the same
    draws."""
    v = dict(variant)
    B, T, H, W, keep, embed, S = (v.pop(k) for k in ("B", "T", "H", "W", "keep", "embed", "S"))
    print("adapter autocast(bf16)", variant, flush=True)

    def make(seed):
        mod, idx, table, x, go = _setup(dev, torch.float32, B, T, H, W, keep, embed,
                                        0.25 if embed > 256 else 0.5, S, 80 + 100 * seed + v.get("use_attn", 0), **v)
        return mod, idx, table, x, go, H, W, T

    assert set(_check_draws(make, amp=torch.bfloat16)) == {torch.float32}


@pytest.mark.parametrize("gate32", [False, True])
@pytest.mark.parametrize("dname", ["float16", "bfloat16"])
def test_heatmap_add_kernel(dev, dname, gate32):
    """heatmap_add_ against PyTorch's gather, multiply and add in the same
    dtype (bit for bit: each product and sum is rounded once, as there); with
    a float32 gate (autocast with float32 parameters) against PyTorch's
    float32 product and sum cast once to the patch dtype, also bit for bit;
    out-of-range source rows leave their row unchanged."""
    import eccv26_tad_amd as sv

    dt = getattr(torch, dname)
    g = torch.Generator().manual_seed(11)
    pa = torch.randn(301, 64, generator=g).to(dev, dt)
    sp = torch.randn(40, 64, generator=g).to(dev, dt)
    src = torch.randint(0, 40, (301,), generator=g, dtype=torch.int32)
    src[::17] = -1
    src[5] = 40
    src = src.to(dev)
    gate = torch.tensor([0.37], device=dev, dtype=torch.float32 if gate32 else dt)
    ok = (src >= 0) & (src < 40)
    ref = pa.clone()
    # float32 gate: PyTorch promotes to float32, the cast back rounds once
    ref[ok] = (pa[ok] + sp[src[ok].long()] * gate).to(dt)
    got = sv.ops.heatmap_add_(pa.clone(), sp, src, gate)
    bad = (got != ref).nonzero()
    if bad.numel():
        i, j = bad[0].tolist()
        print("  mismatches", bad.shape[0], "first at", (i, j), "src", int(src[i]), "got", float(got[i, j]),
              "ref", float(ref[i, j]), "pa", float(pa[i, j]), "sp", float(sp[int(src[i]), j]) if ok[i] else None,
              flush=True)
    assert torch.equal(got, ref)


def test_float32_input_runs_the_unfused_chain(dev):
    """A float32 module and input (no autocast) take the unfused chain with the
    float32 SparseConv2D kernels: float32 output and gradients at the float32
    bar of the reference chain (1e-4 max-scaled: library GEMMs on both sides)."""
    B, T, H, W = 2, 5, 6, 7
    mod, idx, table, x, go = _setup(dev, torch.float32, B, T, H, W, 0.5, 128, 0.5, 1, 72)
    assert mod._fused_dtype(x) is None
    tf32 = torch.backends.cudnn.allow_tf32
    torch.backends.cudnn.allow_tf32 = False  # a full-precision dense convolution on the reference side
    try:
        ref = _fp32_reference(mod, idx, table, x, go, H, W, T)
        y, gx, ydt = _run(mod, lambda xf: mod(xf, H, W, idx, T * H * W, table), x, go, None)
        errs = _errors(y, gx, mod, ref)
    finally:
        torch.backends.cudnn.allow_tf32 = tf32
    print("  errors:", {k: f"{v:.1e}" for k, v in errs.items()}, flush=True)
    assert ydt == torch.float32
    for k, v in errs.items():
        assert v <= 1e-4, (k, v)


@pytest.mark.parametrize("dname", ["float16", "bfloat16"])
def test_two_node_chain_matches_single_node(dev, dname):
    """AdapterDownFunction -> SparseConv2d -> AdapterUpFunction (three autograd
    nodes) against the module's single node: same kernels, so the output is
    identical; the gradients differ only where the single node adds the
    residual's term inside the input-gradient GEMM (bar 1e-2, max-scaled)."""
    import eccv26_tad_amd as sv

    dt = getattr(torch, dname)
    mod, idx, table, x, go = _setup(dev, dt, B=2, T=6, H=7, W=7, keep=0.4, embed=256, mlp_ratio=0.25,
                                    S=1, seed=41)
    H = W = 7
    xa = x.detach().clone().requires_grad_(True)
    ya = mod(xa, H, W, idx, 6 * H * W, table)
    ga = torch.autograd.grad(ya, [xa] + list(mod.parameters()), go)
    xb = x.detach().clone().requires_grad_(True)
    S = xb.shape[1] - idx.shape[1]
    sp, pa = sv.AdapterDownFunction.apply(xb, mod.down_proj.weight, mod.down_proj.bias, S)
    processed = mod.sparse_conv(pa, table.reshape(-1, 9), tokens_per_batch=0)
    yb = sv.AdapterUpFunction.apply(sp, processed, mod.up_proj.weight, mod.up_proj.bias, mod.gamma, xb)
    gb = torch.autograd.grad(yb, [xb] + list(mod.parameters()), go)
    assert torch.equal(ya, yb)
    for a, b in zip(ga, gb):
        assert _err(a, b) <= 1e-2


def test_local_table_matches_global(dev):
    """Per-sample (local) neighbor indices through the reference's max()
    heuristic (tokens_per_batch=None) give the same output and gradients as
    the global table, bit for bit."""
    dt = torch.float16
    mod, idx, table, x, go = _setup(dev, dt, B=2, T=5, H=7, W=7, keep=0.5, embed=128, mlp_ratio=0.5,
                                    S=1, seed=43)
    nk = idx.shape[1]
    local = torch.where(table >= 0, table % nk, table)
    assert int(local.max()) < nk <= int(table.max())
    outs = []
    for tab, tpb in ((table, 0), (local, None)):
        xi = x.detach().clone().requires_grad_(True)
        y = mod(xi, 7, 7, idx, 5 * 49, tab, tokens_per_batch=tpb)
        grads = torch.autograd.grad(y, [xi] + list(mod.parameters()), go)
        outs.append((y, grads))
    assert torch.equal(outs[0][0], outs[1][0])
    for a, b in zip(outs[0][1], outs[1][1]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("dname", ["float16", "bfloat16"])
def test_adapter_kernels_direct(dev, dname):
    import eccv26_tad_amd as sv

    dt = getattr(torch, dname)
    g = torch.Generator().manual_seed(7)
    B, N, S, k, n = 2, 301, 3, 256, 192
    x = torch.randn(B, N, k, generator=g).to(dev, dt)
    w = (torch.randn(n, k, generator=g) * 0.05).to(dev, dt)
    b = (torch.randn(n, generator=g) * 0.1).to(dev, dt)
    pre, sp, pa = sv.ops.adapter_down(x, w, b, S)
    u_ref = x.float() @ w.float().t() + b.float()
    assert _err(pre, u_ref) <= 1e-2
    gl = torch.nn.functional.gelu(pre.float())
    assert _err(sp, gl[:, :S]) <= 1e-2 and _err(pa, gl[:, S:].reshape(-1, n)) <= 1e-2
    # GELU is evaluated on the rounded pre-activation, as PyTorch's GELU of it
    assert _err(sp, torch.nn.functional.gelu(pre[:, :S]).float()) <= (2e-3 if dt == torch.float16 else 1e-2)

    wu = (torch.randn(k, n, generator=g) * 0.05).to(dev, dt)
    bu = (torch.randn(k, generator=g) * 0.1).to(dev, dt)
    gm = torch.tensor([0.6], device=dev, dtype=dt)
    res = torch.randn(B, N, k, generator=g).to(dev, dt)
    y = sv.ops.adapter_up(sp, pa, wu, bu, gm, res)
    c = torch.cat([sp, pa.view(B, N - S, n)], dim=1).float()
    y_ref = (c @ wu.float().t() + bu.float()) * 0.6 + res.float()
    assert _err(y, y_ref) <= 1e-2
    # without bias, and no special tokens
    pre0, sp0, pa0 = sv.ops.adapter_down(x, w, None, 0)
    assert sp0.numel() == 0 and _err(pa0, torch.nn.functional.gelu(x.float() @ w.float().t()).reshape(-1, n)) <= 1e-2
    y0 = sv.ops.adapter_up(sp0, pa0, wu, None, gm, res)
    assert _err(y0, (pa0.float() @ wu.float().t()).view(B, N, k) * 0.6 + res.float()) <= 1e-2


@pytest.mark.parametrize("dname", ["float16", "bfloat16"])
@pytest.mark.parametrize("n,c_g,c_x,mapped", [
    (17250, 256, 768, False), (17248, 768, 256, True), (1000, 64, 128, False), (77, 128, 64, True), (0, 256, 768, False),
])
def test_linear_wgrad(dev, dname, n, c_g, c_x, mapped):
    """g[rows]^T x on the split-row kernel against an fp32 matmul (bar 1e-2)."""
    import eccv26_tad_amd as sv

    dt = getattr(torch, dname)
    g_ = torch.Generator().manual_seed(n + c_g)
    n_g = n + 3 if mapped else n
    g = torch.randn(n_g, c_g, generator=g_).to(dev, dt)
    x = torch.randn(n, c_x, generator=g_).to(dev, dt)
    if mapped:
        rows = torch.randperm(n_g, generator=g_)[:n].to(torch.int32).to(dev)
        ref = g.float()[rows.long()].t() @ x.float()
    else:
        rows = torch.empty(0, dtype=torch.int32, device=dev)
        ref = g.float().t() @ x.float()
    print("linear_wgrad", dname, n, c_g, c_x, mapped, flush=True)
    out = sv.ops.linear_wgrad(g, rows, x)
    assert out.shape == (c_g, c_x) and out.dtype == dt
    out32 = sv.ops.linear_wgrad(g, rows, x, True)  # the unrounded fp32 sums
    assert out32.shape == (c_g, c_x) and out32.dtype == torch.float32
    assert torch.equal(out32.to(dt), out)  # the same sums, rounded once
    if n == 0:
        assert torch.count_nonzero(out) == 0
    else:
        assert _err(out, ref) <= 1e-2
        assert _err(out32, ref) <= 1e-5  # exact products, fp32 sums
        assert torch.equal(out, sv.ops.linear_wgrad(g, rows, x))  # deterministic


@pytest.mark.parametrize("dname", ["float16", "bfloat16"])
@pytest.mark.parametrize("rows,cols", [(17250, 768), (17248, 256), (513, 64), (1, 8), (0, 16)])
def test_column_sums(dev, dname, rows, cols):
    """Ordered column sums against an fp32 sum (bar 1e-2, max-scaled)."""
    import eccv26_tad_amd as sv

    dt = getattr(torch, dname)
    a = torch.randn(rows, cols, generator=torch.Generator().manual_seed(rows + cols)).to(dev, dt)
    out = sv.ops.column_sums(a)
    assert out.shape == (cols,) and out.dtype == dt
    ref = a.float().sum(0)
    if rows == 0:
        assert torch.count_nonzero(out) == 0
    else:
        assert _err(out, ref) <= 1e-2
        assert torch.equal(out, sv.ops.column_sums(a))


@pytest.mark.parametrize("dname", ["float16", "bfloat16"])
@pytest.mark.parametrize("B,N,S,n,missing", [
    (2, 8625, 1, 256, None), (3, 50, 0, 64, None), (2, 40, 40, 128, None), (2, 33, 2, 256, "special"),
    (2, 33, 2, 256, "patch"),
])
def test_gelu_backward_split(dev, dname, B, N, S, n, missing):
    """GELU backward from split gradients against PyTorch's gelu_backward of
    the assembled gradient (both fp32 evaluation, one rounding: bar 2e-3 for
    float16, 1e-2 for bfloat16, max-scaled)."""
    import eccv26_tad_amd as sv

    dt = getattr(torch, dname)
    g = torch.Generator().manual_seed(N + n)
    pre = (torch.randn(B, N, n, generator=g) * 2).to(dev, dt)
    g_sp = torch.randn(B, S, n, generator=g).to(dev, dt)
    g_pa = torch.randn(B * (N - S), n, generator=g).to(dev, dt)
    if missing == "special":
        g_sp_arg, g_sp = None, torch.zeros_like(g_sp)
    else:
        g_sp_arg = g_sp
    if missing == "patch":
        g_pa_arg, g_pa = None, torch.zeros_like(g_pa)
    else:
        g_pa_arg = g_pa
    print("gelu_backward_split", dname, B, N, S, n, missing, flush=True)
    got = sv.ops.gelu_backward_split(g_sp_arg, g_pa_arg, pre, S)
    dg = torch.cat([g_sp, g_pa.view(B, N - S, n)], dim=1)
    ref = torch.ops.aten.gelu_backward(dg.float(), pre.float())
    assert got.shape == pre.shape and got.dtype == dt
    assert _err(got, ref) <= (2e-3 if dt == torch.float16 else 1e-2)
    assert torch.equal(got, sv.ops.gelu_backward_split(g_sp_arg, g_pa_arg, pre, S))


@pytest.mark.parametrize("dname", ["float16", "bfloat16"])
@pytest.mark.parametrize("count,count_b", [(768 * 256, 768), (64 * 128, 0), (8, 8), (0, 0)])
def test_gamma_grad(dev, dname, count, count_b):
    """sum(w * g) + sum(b * gs) against an fp64 sum (bar 1e-2 of the sum of
    absolute products), deterministic."""
    import eccv26_tad_amd as sv

    dt = getattr(torch, dname)
    gen = torch.Generator().manual_seed(count + count_b)
    w = torch.randn(max(count, 1), generator=gen)[:count].to(dev, dt)
    gm = torch.randn(max(count, 1), generator=gen)[:count].to(dev, dt)
    b = torch.randn(count_b, generator=gen).to(dev, dt) if count_b else None
    gs = torch.randn(count_b, generator=gen).to(dev, dt) if count_b else None
    out = sv.ops.gamma_grad(w, gm, b, gs)
    prod = w.double() * gm.double()
    ref = prod.sum()
    scale = prod.abs().sum()
    if b is not None:
        pb = b.double() * gs.double()
        ref, scale = ref + pb.sum(), scale + pb.abs().sum()
    assert out.shape == (1,) and out.dtype == dt
    assert abs(float(out) - float(ref)) <= 1e-2 * max(float(scale), 1e-6) + 1e-3 * abs(float(ref))
    assert torch.equal(out, sv.ops.gamma_grad(w, gm, b, gs))


@pytest.mark.parametrize("dname", ["float16", "bfloat16"])
@pytest.mark.parametrize("with_bias", [True, False])
def test_up_proj_grads(dev, dname, with_bias):
    """The gamma gradient equals gamma_grad, and the scaled copies equal
    PyTorch's elementwise multiplies bit for bit (one fp32 product, one
    rounding)."""
    import eccv26_tad_amd as sv

    dt = getattr(torch, dname)
    gen = torch.Generator().manual_seed(5 + with_bias)
    w = torch.randn(768, 256, generator=gen).to(dev, dt)
    g = torch.randn(768, 256, generator=gen).to(dev, dt)
    b = torch.randn(768, generator=gen).to(dev, dt) if with_bias else None
    gs = torch.randn(768, generator=gen).to(dev, dt) if with_bias else None
    gamma = torch.tensor([0.37], device=dev, dtype=dt)
    gg, w_s, g_s, gs_s = sv.ops.up_proj_grads(w, g, b, gs, gamma)
    assert torch.equal(gg, sv.ops.gamma_grad(w, g, b, gs))
    assert torch.equal(w_s, w * gamma) and torch.equal(g_s, g * gamma)
    if with_bias:
        assert torch.equal(gs_s, gs * gamma)
    else:
        assert gs_s.numel() == 0


@pytest.mark.parametrize("dname", ["float16", "bfloat16"])
@pytest.mark.parametrize("res32,out32", [(True, True), (False, True), (False, False)])
def test_adapter_up_mixed_dtypes(dev, dname, res32, out32):
    """The up GEMM with a float32 gamma (autocast with float32 parameters):
    the epilogue is PyTorch's ``z * gamma + residual`` on the rounded z,
    bit for bit (float32 product, float32 add, then stored as float32 or cast
    once); z itself is taken from the same kernel with gamma 1 and a zero
    residual of the compute dtype."""
    import eccv26_tad_amd as sv

    dt = getattr(torch, dname)
    g = torch.Generator().manual_seed(17 + 2 * res32 + out32)
    B, N, S, k, n = 2, 203, 2, 256, 512
    sp = torch.randn(B, S, k, generator=g).to(dev, dt)
    pa = torch.randn(B * (N - S), k, generator=g).to(dev, dt)
    w = (torch.randn(n, k, generator=g) * 0.05).to(dev, dt)
    b = (torch.randn(n, generator=g) * 0.1).to(dev, dt)
    z = sv.ops.adapter_up(sp, pa, w, b, torch.ones(1, device=dev, dtype=dt), torch.zeros(B, N, n, device=dev, dtype=dt))
    gamma = torch.tensor([0.3711], device=dev, dtype=torch.float32)
    res = torch.randn(B, N, n, generator=g).to(dev, torch.float32 if res32 else dt)
    y = sv.ops.adapter_up(sp, pa, w, b, gamma, res, out32)
    ref = z * gamma + res  # float32 by PyTorch's promotion
    ref = ref if out32 else ref.to(dt)
    assert y.dtype == ref.dtype and y.shape == ref.shape
    bad = (y != ref).nonzero()
    if bad.numel():
        print("  mismatches", bad.shape[0], "first", bad[0].tolist(), flush=True)
    assert torch.equal(y, ref)
    zr = torch.cat([sp, pa.view(B, N - S, k)], dim=1).float() @ w.float().t() + b.float()
    assert _err(z, zr) <= 1e-2
    with pytest.raises(RuntimeError):
        # a float32 output with a gamma of the compute dtype is not the reference's promotion
        sv.ops.adapter_up(sp, pa, w, b, gamma.to(dt), res.to(dt), True)


@pytest.mark.parametrize("dname", ["float16", "bfloat16"])
def test_up_proj_grads_float32_gamma(dev, dname):
    """With a float32 gamma the gamma gradient is float32 and equals the
    float32-gamma-free sum (it does not depend on gamma), and the scaled
    copies are PyTorch's float32 products cast once to the compute dtype."""
    import eccv26_tad_amd as sv

    dt = getattr(torch, dname)
    gen = torch.Generator().manual_seed(23)
    w = torch.randn(768, 256, generator=gen).to(dev, dt)
    g = torch.randn(768, 256, generator=gen).to(dev, dt)
    b = torch.randn(768, generator=gen).to(dev, dt)
    gs = torch.randn(768, generator=gen).to(dev, dt)
    gamma = torch.tensor([0.3711], device=dev, dtype=torch.float32)
    gg, w_s, g_s, gs_s = sv.ops.up_proj_grads(w, g, b, gs, gamma)
    assert gg.dtype == torch.float32 and w_s.dtype == dt
    ref = (w.double() * g.double()).sum() + (b.double() * gs.double()).sum()
    scale = (w.double() * g.double()).abs().sum() + (b.double() * gs.double()).abs().sum()
    assert abs(float(gg) - float(ref)) <= 1e-5 * float(scale)
    assert torch.equal(gg.to(dt), sv.ops.gamma_grad(w, g, b, gs))
    assert torch.equal(w_s, (w * gamma).to(dt)) and torch.equal(g_s, (g * gamma).to(dt))
    assert torch.equal(gs_s, (gs * gamma).to(dt))
    # an fp32 g (the unrounded weight-gradient sums): g * gamma rounded once,
    # the dot product taken on the fp32 values
    g32 = torch.randn(768, 256, generator=gen).to(dev)
    gg32, w_s2, g_s2, _ = sv.ops.up_proj_grads(w, g32, b, gs, gamma)
    assert g_s2.dtype == dt and torch.equal(g_s2, (g32 * gamma).to(dt)) and torch.equal(w_s2, w_s)
    ref32 = (w.double() * g32.double()).sum() + (b.double() * gs.double()).sum()
    scale32 = (w.double() * g32.double()).abs().sum() + (b.double() * gs.double()).abs().sum()
    assert abs(float(gg32) - float(ref32)) <= 1e-5 * float(scale32)
