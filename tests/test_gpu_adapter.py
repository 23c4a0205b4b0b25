"""The fused sparse-conv adapter against an independent float32 restatement
of the reference adapter (``tests/adapter_ref.py``: the chain of
vit_sparse_adapter_poguise.py:288-362,511-653 in PyTorch float32 ops, its
convolution on the dense ``2d_conv`` path, which the CPU oracle pins) on the
same rounded weights and inputs: output and every gradient (x, down_proj,
up_proj, gamma, the sparse conv's weight and bias, and the attention /
heatmap parameters of those variants). Bar: max-scaled error <= 1e-2
(float16 / bfloat16). The kernels' direct outputs (pre-activation, split
GELU, fused up projection, heatmap gather-add) are checked against float32
PyTorch the same way.

Shapes: the ViT-B adapter (embed 768, hidden 256 after the reference's
power-of-two rounding) on B2 x T80 x 14x14 at 55 % keep with one CLS token,
a small case with no special token, every ``use_attn`` variant (1, 2, 3, 4)
and the heatmap injection on the same grid and on a resized heatmap grid.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.adapter_ref import adapter_fp32, gain_scales
from tests.helpers import topk_mask

pytestmark = pytest.mark.gpu


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


def _check_against_fp32(mod, idx, table, x, go, H, W, T, tol=1e-2):
    """The module's output and every gradient against adapter_fp32 on the same
    rounded parameters and inputs; prints the measured errors."""
    go_ref = go.detach().float().clone()
    xf = x.detach().clone().requires_grad_(True)
    y = mod(xf, H, W, idx, T * H * W, table)
    y.backward(go.detach().clone())
    xr = x.detach().float().requires_grad_(True)
    gains = {}
    yr, P = adapter_fp32(mod, xr, H, W, idx, T * H * W, gains)
    yr.backward(go_ref)
    scales = gain_scales(gains)
    assert y.shape == yr.shape
    errs = {"y": _err(y.detach(), yr.detach()), "x": _err(xf.grad, xr.grad)}
    for name, p in mod.named_parameters():
        if P[name].grad is None:
            # not on the forward path (attn_gamma of the temporal variant)
            assert p.grad is None, name
            continue
        if name in scales:
            # a scalar gain's gradient is one sum over every token and
            # channel with heavy cancellation: its error is measured against
            # the sum of the absolute terms (as test_gamma_grad does)
            errs[name] = abs(float(p.grad) - float(P[name].grad)) / max(scales[name], 1e-30)
            continue
        if name == "k_norm.bias":
            # exactly zero: the bias shifts every key's score of a query by the
            # same q.b, which the softmax cancels; both sides hold rounding
            # noise, so it is measured against the k_norm weight's gradient
            errs[name] = float(p.grad.double().abs().max() /
                               P["k_norm.weight"].grad.double().abs().max().clamp_min(1e-30))
            continue
        errs[name] = _err(p.grad, P[name].grad)
    worst = max(errs, key=errs.get)
    print(f"  worst max-scaled error {errs[worst]:.2e} ({worst}); y {errs['y']:.2e}, x {errs['x']:.2e}", flush=True)
    print("  all:", {k: f"{v:.1e}" for k, v in errs.items()}, flush=True)
    for name, p in mod.named_parameters():
        if p.numel() == 1 and p.grad is not None:
            print(f"  {name}: got {float(p.grad):.5g} ref {float(P[name].grad):.5g}", flush=True)
    for k, v in errs.items():
        # the attention branch's own parameters are PyTorch's bfloat16 ops
        # (LayerNorm, Linear, softmax gradients through bf16-rounded q, k):
        # their gradients carry bf16 rounding of sums with cancellation
        bar = 5e-2 if (x.dtype == torch.bfloat16 and k.startswith(_ATTN_PARAMS)) else tol
        assert v <= bar, (k, v)
    return y


_ATTN_PARAMS = ("attn_norm.", "down_attn.", "qkv.", "q_norm.", "k_norm.", "attn_proj.", "attn_mlp.")


@pytest.mark.parametrize("dname", ["float16", "bfloat16"])
@pytest.mark.parametrize("case", [
    dict(B=2, T=80, H=14, W=14, keep=0.55, embed=768, mlp_ratio=0.25, S=1, seed=31),
    dict(B=3, T=4, H=6, W=7, keep=0.3, embed=128, mlp_ratio=0.5, S=0, seed=32),
])
def test_fused_adapter_matches_fp32_reference(dev, dname, case):
    dt = getattr(torch, dname)
    c = dict(case)
    S = c.pop("S")
    mod, idx, table, x, go = _setup(dev, dt, S=S, **c)
    print("adapter", dname, case, "N", x.shape[1], "hidden", mod.hidden_dims, flush=True)
    y = _check_against_fp32(mod, idx, table, x, go, c["H"], c["W"], c["T"])
    assert y.dtype == dt


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
    _check_against_fp32(mod, idx, table, x, go, H, W, T)


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
    mod, idx, table, x, go = _setup(dev, dt, B, T, H, W, 0.45, embed, 0.25, S, 50 + use_attn,
                                    use_attn=use_attn, n_key_tokens=S)
    print("adapter use_attn", use_attn, dname, "N", x.shape[1], "hidden", mod.hidden_dims, flush=True)
    _check_against_fp32(mod, idx, table, x, go, H, W, T)


@pytest.mark.parametrize("dname", ["float16", "bfloat16"])
@pytest.mark.parametrize("grid", [(7, 8), (3, 4)])
def test_heatmap_injection_matches_fp32_reference(dev, dname, grid):
    """n_key_tokens = 1 + heatmap cells, use_attn = 0: the heatmap gather-add
    on the SparseConv2D input, on the token grid itself and on a smaller
    heatmap grid (nearest-index resize)."""
    dt = getattr(torch, dname)
    B, T, H, W = 2, 6, 7, 8
    S = 1 + grid[0] * grid[1]
    mod, idx, table, x, go = _setup(dev, dt, B, T, H, W, 0.5, 128, 0.5, S, 60 + grid[0],
                                    n_key_tokens=S, heatmap_grid_size=grid)
    assert mod._uses_heatmap()
    print("adapter heatmap", grid, dname, flush=True)
    _check_against_fp32(mod, idx, table, x, go, H, W, T)


@pytest.mark.parametrize("dname", ["float16", "bfloat16"])
def test_heatmap_add_kernel(dev, dname):
    """heatmap_add_ against PyTorch's gather, multiply and add in the same
    dtype (bit for bit: each product and sum is rounded once, as there);
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
    gate = torch.tensor([0.37], device=dev, dtype=dt)
    ok = (src >= 0) & (src < 40)
    ref = pa.clone()
    ref[ok] = pa[ok] + sp[src[ok].long()] * gate
    got = sv.ops.heatmap_add_(pa.clone(), sp, src, gate)
    bad = (got != ref).nonzero()
    if bad.numel():
        i, j = bad[0].tolist()
        print("  mismatches", bad.shape[0], "first at", (i, j), "src", int(src[i]), "got", float(got[i, j]),
              "ref", float(ref[i, j]), "pa", float(pa[i, j]), "sp", float(sp[int(src[i]), j]) if ok[i] else None,
              flush=True)
    assert torch.equal(got, ref)


def test_autocast_with_fp32_parameters(dev):
    """The reference's training loop: float32 parameters and input under
    torch.autocast(bfloat16) (opentad/cores/train_engine.py). The adapter runs
    the unfused chain with SparseConv2d's autocast casts: a float32 output
    (gamma is a float32 parameter) within the bfloat16 bar of the float32
    reference, and float32 gradients on every parameter."""
    B, T, H, W = 2, 6, 7, 8
    mod, idx, table, x, go = _setup(dev, torch.float32, B, T, H, W, 0.5, 256, 0.25, 1, 71)
    xf = x.detach().clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = mod(xf, H, W, idx, T * H * W, table)
    assert y.dtype == torch.float32
    y.backward(go)
    xr = x.detach().clone().requires_grad_(True)
    gains = {}
    yr, P = adapter_fp32(mod, xr, H, W, idx, T * H * W, gains)
    yr.backward(go)
    scales = gain_scales(gains)
    assert _err(y.detach(), yr.detach()) <= 1e-2 and _err(xf.grad, xr.grad) <= 1e-2
    for name, p in mod.named_parameters():
        assert p.grad is not None and p.grad.dtype == torch.float32, name
        if name in scales:
            assert abs(float(p.grad) - float(P[name].grad)) <= 1e-2 * scales[name], name
        else:
            assert _err(p.grad, P[name].grad) <= 1e-2, name


def test_float32_input_runs_the_unfused_chain(dev):
    """A float32 module and input (no autocast) take the unfused chain with the
    float32 SparseConv2D kernels: float32 output and gradients at the float32
    bar of the reference chain (1e-4 max-scaled: library GEMMs on both sides)."""
    B, T, H, W = 2, 5, 6, 7
    mod, idx, table, x, go = _setup(dev, torch.float32, B, T, H, W, 0.5, 128, 0.5, 1, 72)
    tf32 = torch.backends.cudnn.allow_tf32
    torch.backends.cudnn.allow_tf32 = False  # a full-precision dense convolution on the reference side
    try:
        y = _check_against_fp32(mod, idx, table, x, go, H, W, T, tol=1e-4)
    finally:
        torch.backends.cudnn.allow_tf32 = tf32
    assert y.dtype == torch.float32


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
    if n == 0:
        assert torch.count_nonzero(out) == 0
    else:
        assert _err(out, ref) <= 1e-2
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
