"""The sparse-conv adapter with fused GEMM epilogues.

Reference: the ``conv_type == "sparse_conv"`` adapter of
``opentad/models/backbones/vit_sparse_adapter_poguise.py`` (constructor
``:95-111,163-166``, forward ``:290-362`` and ``:652-653``), without the
optional heatmap injection (``:316-355``) and attention branch, which this
module does not implement (it raises when asked for them):

    x_proj = GELU(down_proj(x))                      # [B, N, hidden]
    special, patches = x_proj[:, :S], x_proj[:, S:]  # S = N - indices.shape[1]
    processed = sparse_conv(patches, neighbor_indices)
    y = up_proj(cat(special, processed)) * gamma + x

The module runs as one autograd node (``SparseConvAdapterFunction``); its
forward is the down GEMM (``opentad_sparse_ops.adapter_down``), the
SparseConv2D forward (weight pack + gathered GEMM) and the up GEMM
(``opentad_sparse_ops.adapter_up``):

* the down GEMM's epilogue adds the bias, rounds the Linear output, applies
  GELU and writes the special tokens and the (contiguous) SparseConv2D input
  directly: no GELU pass and no slice copy;
* the up GEMM reads the special tokens and the SparseConv2D output in place of
  the concatenation and applies bias, ``gamma`` and the residual before its
  single store: no cat, no scale pass, no add pass;
* ``tokens_per_batch`` defaults to 0 (the tables the backbone builds are
  global), so there is no host sync; ``None`` restores the reference's
  ``max()`` heuristic (``sparse_conv_layer.py:174-177``).

The backward's weight gradients (sums over every token row) run on the
split-row kernel of SparseConv2D's backward-weight pass with one offset
(``opentad_sparse_ops.linear_wgrad``: deterministic, and a grid that fills the
chip where a library GEMM with a 17k-long reduction gets a dozen workgroups);
the input gradients use library GEMMs (``torch.matmul``). The GELU backward
reads the special-token and patch-token gradients in place of their
concatenation (``opentad_sparse_ops.gelu_backward_split``). ``gamma``'s
gradient needs ``z = cat(...) W_u^T + b_u``, which the fused forward never
stores: ``sum(go * z) = <W_u, go^T c> + <b_u, sum(go)>``, and ``go^T c`` is
the up-projection's weight-gradient reduction anyway; one launch adds both
products (``opentad_sparse_ops.gamma_grad``). The bias gradients (column sums
over the token rows) use ``opentad_sparse_ops.column_sums``.

The input gradient is one GEMM with the residual's term as its addend
(``addmm(go, du, W_d)``), which the single node makes possible.
``AdapterDownFunction`` and ``AdapterUpFunction`` are the same kernels as two
separate nodes around a ``SparseConv2d``.

The fused path takes float16 / bfloat16 (the matrix-core dtypes) and raises
otherwise; ``reference_forward`` runs the unfused chain in the reference's op
order (for tests and the benchmark).
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
from torch.autograd import Function

from . import opentad_sparse_ops as _ops
from .sparse_conv_layer import (BIAS_AFTER, BIAS_FP32, BIAS_NONE, IMPLICIT_GEMM_MIN_CIN, SparseConv2d)

_FUSED_DTYPES = (torch.float16, torch.bfloat16)


def _colsum(a):
    """Column sums of a [rows, n] matrix (the Linear bias gradients): fp32
    accumulation over row splits added in a fixed order, result in a's
    dtype. PyTorch's dim-0 reduction and a ones-vector GEMM take 24 and 58 µs
    at 17250 x 768."""
    return _ops.column_sums(a)


def _NO_ROWS(like):
    """Empty row list: the weight-gradient kernel then takes rows in order."""
    return torch.empty(0, dtype=torch.int32, device=like.device)


_PATCH_ROWS = {}


def _patch_rows(B, N, S, device):
    """Row of ``go.reshape(B * N, -1)`` for each patch token in the order of
    the SparseConv2D rows (``b * N + S + r``), cached per shape and device:
    built on every backward it costs five small integer kernels."""
    key = (B, N, S, device)
    rows = _PATCH_ROWS.get(key)
    if rows is None:
        P = N - S
        r = torch.arange(B * P, device=device, dtype=torch.int32)
        rows = (r // P) * N + S + r % P
        if len(_PATCH_ROWS) >= 64:
            _PATCH_ROWS.clear()
        _PATCH_ROWS[key] = rows
    return rows


class AdapterDownFunction(Function):
    """``(act_special, act_patch) = split(GELU(x W^T + b))``; x ``[B, N, k]``."""

    @staticmethod
    def forward(ctx, x, weight, bias, n_special):
        pre, sp, pa = _ops.adapter_down(x, weight, bias, int(n_special))
        ctx.save_for_backward(x, weight, pre)
        ctx.has_bias = bias is not None
        ctx.n_special = int(n_special)
        return sp, pa

    @staticmethod
    def backward(ctx, g_sp, g_pa):
        x, weight, pre = ctx.saved_tensors
        n = pre.shape[-1]
        # GELU backward straight from the two gradient buffers (no assembled dg)
        du = _ops.gelu_backward_split(g_sp, g_pa, pre, ctx.n_special)
        du2 = du.reshape(-1, n)
        gx = torch.matmul(du, weight) if ctx.needs_input_grad[0] else None
        gw = _ops.linear_wgrad(du2, _NO_ROWS(du2), x.reshape(-1, x.shape[-1])) if ctx.needs_input_grad[1] else None
        gb = _colsum(du2) if ctx.has_bias and ctx.needs_input_grad[2] else None
        return gx, gw, gb, None


class AdapterUpFunction(Function):
    """``out = T(z * gamma) + residual``, ``z = cat(a_special, a_patch) W^T + b``."""

    @staticmethod
    def forward(ctx, a_special, a_patch, weight, bias, gamma, residual):
        out = _ops.adapter_up(a_special, a_patch, weight, bias, gamma, residual)
        ctx.save_for_backward(a_special, a_patch, weight, bias, gamma)
        return out

    @staticmethod
    def backward(ctx, go):
        a_sp, a_pa, weight, bias, gamma = ctx.saved_tensors
        B, N, n = go.shape
        S = a_sp.shape[1]
        k = weight.shape[1]
        go = go.contiguous()
        go2 = go.reshape(-1, n)
        # go^T c without building c = cat(a_special, a_patch): the patch rows
        # on the split-row kernel (rows of go picked by a row list), the few
        # special rows as a small GEMM
        if S > 0:
            G = _ops.linear_wgrad(go2, _patch_rows(B, N, S, go.device), a_pa)
            G = G + torch.matmul(go[:, :S].reshape(-1, n).t(), a_sp.reshape(-1, k))
        else:
            G = _ops.linear_wgrad(go2, _NO_ROWS(go2), a_pa)
        gsum = _colsum(go2)
        g_gamma = None
        if ctx.needs_input_grad[4]:
            g_gamma = _ops.gamma_grad(weight, G, bias, gsum if bias is not None else None)
            g_gamma = g_gamma.view(gamma.shape).to(gamma.dtype)
        g_sp = g_pa = None
        if ctx.needs_input_grad[0] or ctx.needs_input_grad[1]:
            # (go * gamma) W = go (gamma W): gamma folded into the small weight
            dc = torch.matmul(go, weight * gamma)  # [B, N, k]
            g_sp = dc[:, :S] if ctx.needs_input_grad[0] else None
            g_pa = dc[:, S:].reshape(-1, k) if ctx.needs_input_grad[1] else None
        gw = G * gamma if ctx.needs_input_grad[2] else None
        gb = gsum * gamma if bias is not None and ctx.needs_input_grad[3] else None
        return g_sp, g_pa, gw, gb, g_gamma, go


class SparseConvAdapterFunction(Function):
    """The whole adapter (down GEMM + GELU, SparseConv2D, up GEMM + gamma +
    residual) as one autograd node, so that its backward can hand the input
    gradient's two terms to one GEMM: ``grad_x = go + du W_d`` is
    ``addmm(go, du, W_d)``, where the two-node chain computes ``du W_d`` and
    then autograd adds ``go`` in a separate pass over the 768-wide tokens.
    The kernels are those of ``AdapterDownFunction``, ``SparseConv2dFunction``
    and ``AdapterUpFunction``."""

    @staticmethod
    def forward(ctx, x, w_d, b_d, w_c, b_c, w_u, b_u, gamma, nbr, n_special, tpb):
        S = int(n_special)
        pre, sp, pa = _ops.adapter_down(x, w_d, b_d, S)
        c_in = w_c.shape[1]
        if c_in % 4 != 0:
            raise ValueError(f"C_in ({c_in}) must be divisible by 4 for optimized kernel.")
        mode = BIAS_NONE if b_c is None else (BIAS_FP32 if c_in >= IMPLICIT_GEMM_MIN_CIN else BIAS_AFTER)
        pf, pb = _ops.pack_weight(w_c, True, any(ctx.needs_input_grad))
        processed = _ops.fwd_packed(pa, nbr, w_c, pf, b_c, tpb, mode)
        out = _ops.adapter_up(sp, processed, w_u, b_u, gamma, x)
        ctx.save_for_backward(x, w_d, pre, sp, pa, nbr, w_c, b_c, pb, processed, w_u, b_u, gamma)
        ctx.flags = (S, int(tpb), b_d is not None)
        return out

    @staticmethod
    def backward(ctx, go):
        x, w_d, pre, sp, pa, nbr, w_c, b_c, pb, processed, w_u, b_u, gamma = ctx.saved_tensors
        S, tpb, has_bd = ctx.flags
        need = ctx.needs_input_grad
        B, N, n = go.shape
        k = w_u.shape[1]
        go = go.contiguous()
        go2 = go.reshape(-1, n)
        # up projection: G = go^T cat(sp, processed) without the cat
        if S > 0:
            G = _ops.linear_wgrad(go2, _patch_rows(B, N, S, go.device), processed)
            G = G + torch.matmul(go[:, :S].reshape(-1, n).t(), sp.reshape(-1, k))
        else:
            G = _ops.linear_wgrad(go2, _NO_ROWS(go2), processed)
        gsum = _colsum(go2)
        # gamma's gradient and the gamma-scaled W_u, G and sum(go) in one pass
        g_gamma, w_u_g, gw_u, gb_u = _ops.up_proj_grads(w_u, G, b_u, gsum if b_u is not None else None, gamma)
        g_gamma = g_gamma.view(gamma.shape) if need[7] else None
        gw_u = gw_u if need[5] else None
        gb_u = gb_u if b_u is not None and need[6] else None
        dc = torch.matmul(go, w_u_g)  # [B, N, k]: (go * gamma) W_u
        g_sp = dc[:, :S]
        g_pa = dc[:, S:].reshape(-1, k)
        # SparseConv2D
        need_bc = b_c is not None and need[4]
        gi_pa, gw_c, gb_c = _ops.bwd_packed(g_pa, pa, nbr, w_c, pb, w_c.shape[1], tpb, need_bc)
        # down projection: GELU backward from the two gradient buffers, then
        # the input gradient with the residual's go in the same GEMM
        du = _ops.gelu_backward_split(g_sp, gi_pa, pre, S)
        du2 = du.reshape(-1, du.shape[-1])
        x2 = x.reshape(-1, x.shape[-1])
        gx = torch.addmm(go2, du2, w_d).view(x.shape) if need[0] else None
        gw_d = _ops.linear_wgrad(du2, _NO_ROWS(du2), x2) if need[1] else None
        gb_d = _colsum(du2) if has_bd and need[2] else None
        return (gx, gw_d, gb_d, gw_c if need[3] else None, gb_c if need_bc else None, gw_u, gb_u, g_gamma,
                None, None, None)


class SparseConvAdapter(nn.Module):
    """The reference adapter with ``conv_type="sparse_conv"``, ``use_attn=0``
    and no heatmap injection, on fused HIP GEMM epilogues."""

    def __init__(self, embed_dims: int, mlp_ratio: float = 0.25, n_key_tokens: int = 1,
                 heatmap_grid_size=None):
        super().__init__()
        if n_key_tokens > 1 and heatmap_grid_size is not None:
            raise NotImplementedError("SparseConvAdapter: heatmap injection is not implemented")
        self.embed_dims = embed_dims
        hidden = int(embed_dims * mlp_ratio)
        hidden = int(2 ** round(math.log2(hidden)))  # power of two, as the reference rounds
        self.hidden_dims = hidden
        self.down_proj = nn.Linear(embed_dims, hidden)
        nn.init.trunc_normal_(self.down_proj.weight, std=0.02)
        nn.init.zeros_(self.down_proj.bias)
        self.act = nn.GELU()
        self.up_proj = nn.Linear(hidden, embed_dims)
        nn.init.zeros_(self.up_proj.weight)
        nn.init.zeros_(self.up_proj.bias)
        self.gamma = nn.Parameter(torch.ones(1))
        self.sparse_conv = SparseConv2d(hidden, hidden)

    @staticmethod
    def _n_special(x, indices):
        return x.shape[1] - indices.shape[1]

    def forward(self, x, h, w, indices, total_num_patches, neighbor_indices=None, tokens_per_batch=0):
        """``x [B, N, embed]``; ``indices [B, N_kept]``; ``neighbor_indices``
        ``[B, N_kept, 9]`` or ``[B * N_kept, 9]``. ``h``, ``w`` and
        ``total_num_patches`` are accepted for signature compatibility."""
        if x.dtype not in _FUSED_DTYPES or not x.is_cuda:
            raise RuntimeError(f"SparseConvAdapter: the fused path takes float16 / bfloat16 GPU "
                               f"tensors, got {x.dtype} on {x.device}")
        if self.down_proj.weight.dtype != x.dtype:
            raise RuntimeError("SparseConvAdapter: convert the module to the input dtype first")
        S = self._n_special(x, indices)
        if indices.shape[1] == 0:
            return self.reference_forward(x, h, w, indices, total_num_patches, neighbor_indices)
        nbr = neighbor_indices.reshape(-1, 9)
        if tokens_per_batch is None:
            tokens_per_batch = indices.shape[1] if int(nbr.max()) < indices.shape[1] else 0
        if nbr.dtype != torch.int32:
            nbr = nbr.to(torch.int32)
        conv = self.sparse_conv
        return SparseConvAdapterFunction.apply(x, self.down_proj.weight, self.down_proj.bias, conv.weight,
                                               conv.bias, self.up_proj.weight, self.up_proj.bias, self.gamma,
                                               nbr, S, tokens_per_batch)

    def reference_forward(self, x, h, w, indices, total_num_patches, neighbor_indices=None):
        """The unfused chain in the reference's op order
        (vit_sparse_adapter_poguise.py:305-362,652-653), including its
        ``.max()`` heuristic inside SparseConv2d."""
        inputs = x
        x_proj = self.act(self.down_proj(x))
        S = self._n_special(x, indices)
        special = x_proj[:, :S, :]
        patches = x_proj[:, S:, :]
        if patches.shape[1] == 0:
            # the reference applies the activation a second time here (:356-358)
            return self.up_proj(self.act(x_proj)) * self.gamma + inputs
        processed = self.sparse_conv(patches, neighbor_indices)
        return self.up_proj(torch.cat([special, processed], dim=1)) * self.gamma + inputs
