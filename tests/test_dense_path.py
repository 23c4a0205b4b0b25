"""The dense comparator path (scatter -> NCHW conv2d -> gather, reference
vit_sparse_adapter_poguise.py:372-412,484-490) against the oracle on the CPU,
and SparseConv2D against it on the GPU.

CPU (fp64, inputs exact in fp32): the comparator's output and its autograd
gradients equal the oracle's gather-form fwd / bwd_in / bwd_w / bias_grad on
the table built from the same keep set (max-scaled error <= 1e-12), which
pins the comparator and the weight re-layout; the keep-mask helper equals the
numpy mask; the weight helpers match the reference SparseConv2d init
re-layout (sparse_conv_layer.py:145-161).

GPU: SparseConv2d (fp16 / bf16 / fp32) forward and backward against the
comparator run in fp32 on the same rounded values, at the c2 shape
(B2 x T80 x 14x14, C = 192) and a small ragged one; bar 1e-2 (fp16 / bf16),
1e-5 (fp32), max-scaled.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.helpers import random_mask, topk_mask


def _indices(mask: np.ndarray) -> torch.Tensor:
    B = mask.shape[0]
    flat = mask.reshape(B, -1)
    k = int(flat[0].sum())
    assert (flat.sum(1) == k).all(), "equal keep counts per sample"
    return torch.from_numpy(np.stack([np.flatnonzero(flat[b]) for b in range(B)])).long()


def _conv_fn(weight, bias):
    return lambda t: torch.nn.functional.conv2d(t, weight, bias, padding=1)


@pytest.mark.parametrize("shape,keep", [((2, 3, 5, 6), 0.4), ((1, 2, 4, 4), 1.0), ((3, 2, 3, 7), 0.15)])
def test_dense_path_equals_oracle(oracle, shape, keep):
    import eccv26_tad_amd as sv

    B, T, H, W = shape
    rng = np.random.default_rng(11)
    mask = random_mask(rng, B, T, H, W, keep)
    idx = _indices(mask)
    n_kept = idx.shape[1]
    ci, co = 8, 12
    x = rng.standard_normal((B * n_kept, ci)).astype(np.float32)
    w9 = rng.standard_normal((9, ci, co)).astype(np.float32)
    b = rng.standard_normal(co).astype(np.float32)
    go = rng.standard_normal((B * n_kept, co)).astype(np.float32)

    xt = torch.tensor(x, dtype=torch.float64).view(B, n_kept, ci).requires_grad_(True)
    wc = sv.conv2d_weight_from_sparse(torch.tensor(w9, dtype=torch.float64)).requires_grad_(True)
    bt = torch.tensor(b, dtype=torch.float64, requires_grad=True)
    y = sv.dense_conv_tokens(xt, idx, T * H * W, H, W, _conv_fn(wc, bt))
    gi, gwc, gb = torch.autograd.grad(y, (xt, wc, bt), torch.tensor(go, dtype=torch.float64).view(B, n_kept, co))

    table = oracle.build_table(mask)
    assert oracle.rel_err(y.detach().reshape(-1, co).numpy(), oracle.fwd(x, table, w9, b)) <= 1e-12
    assert oracle.rel_err(gi.reshape(-1, ci).numpy(), oracle.bwd_in(go, table, w9)) <= 1e-12
    gw9 = sv.sparse_weight_from_conv2d(gwc).numpy()
    assert oracle.rel_err(gw9, oracle.bwd_w(go, x, table)) <= 1e-12
    assert oracle.rel_err(gb.numpy(), oracle.bias_grad(go)) <= 1e-12

    m = sv.keep_mask_from_indices(idx, T, H, W)
    assert m.dtype == torch.uint8 and np.array_equal(m.numpy(), mask)


def test_weight_relayout_matches_reference_init():
    import eccv26_tad_amd as sv

    g = torch.Generator().manual_seed(3)
    temp = torch.randn(7, 5, 3, 3, generator=g)
    ref = temp.view(7, 5, 9).permute(2, 1, 0)  # sparse_conv_layer.py:150-156
    w9 = sv.sparse_weight_from_conv2d(temp)
    assert w9.shape == (9, 5, 7) and torch.equal(w9, ref)
    assert torch.equal(sv.conv2d_weight_from_sparse(w9), temp)
    # k = ky * 3 + kx
    assert torch.equal(w9[1 * 3 + 2], temp[:, :, 1, 2].t())
    with pytest.raises(ValueError):
        sv.sparse_weight_from_conv2d(torch.zeros(2, 2, 5, 5))
    with pytest.raises(ValueError):
        sv.conv2d_weight_from_sparse(torch.zeros(8, 2, 2))


# --------------------------------------------------------------------------
# GPU: SparseConv2d against the dense comparator
# --------------------------------------------------------------------------

def _max_err(got: torch.Tensor, ref: torch.Tensor) -> float:
    got, ref = got.double(), ref.double()
    return float((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30))


@pytest.mark.gpu
@pytest.mark.parametrize("dname,shape,keep,c", [
    ("float16", (2, 80, 14, 14), 0.55, 192),
    ("bfloat16", (2, 80, 14, 14), 0.25, 192),
    ("float16", (2, 80, 14, 14), 1.0, 192),
    ("float32", (2, 6, 9, 11), 0.3, 48),
    ("bfloat16", (3, 5, 7, 8), 0.1, 256),
])
def test_sparse_conv_equals_dense_path(dev, dname, shape, keep, c):
    import eccv26_tad_amd as sv

    dt = getattr(torch, dname)
    tol = 1e-5 if dt == torch.float32 else 1e-2
    B, T, H, W = shape
    rng = np.random.default_rng(int(keep * 100) + c)
    mask = topk_mask(rng, B, T, H, W, keep)
    idx = _indices(mask).to(dev)
    n_kept = idx.shape[1]
    print("dense path", dname, shape, keep, c, "n_kept", n_kept, flush=True)
    table = sv.build_neighbor_table(sv.keep_mask_from_indices(idx, T, H, W))
    assert table.shape[0] == B * n_kept

    g = torch.Generator().manual_seed(5)
    mod = sv.SparseConv2d(c, c).to(dev)
    with torch.no_grad():
        mod.weight.copy_(mod.weight.to(dt).float())
        mod.bias.copy_((torch.rand(c, generator=g) * 0.2 - 0.1).to(dev).to(dt).float())
    mod = mod.to(dt)
    x = torch.randn(B, n_kept, c, generator=g).to(dev, dt).requires_grad_(True)
    go = torch.randn(B, n_kept, c, generator=g).to(dev, dt)
    y = mod(x, table.view(B, n_kept, 9), tokens_per_batch=0)
    y.backward(go)

    # comparator in fp32 on the same (rounded) values
    xr = x.detach().float().requires_grad_(True)
    wc = sv.conv2d_weight_from_sparse(mod.weight.detach().float()).requires_grad_(True)
    br = mod.bias.detach().float().requires_grad_(True)
    yr = sv.dense_conv_tokens(xr, idx, T * H * W, H, W, _conv_fn(wc, br))
    yr.backward(go.float())

    assert _max_err(y.detach(), yr.detach()) <= tol
    assert _max_err(x.grad, xr.grad) <= tol
    assert _max_err(mod.weight.grad, sv.sparse_weight_from_conv2d(wc.grad)) <= tol
    assert _max_err(mod.bias.grad, br.grad) <= tol
