"""The sparse-conv adapter with fused GEMM epilogues.

Reference: the ``conv_type == "sparse_conv"`` adapter of
``opentad/models/backbones/vit_sparse_adapter_poguise.py`` (constructor
``:78-166``, forward ``:288-362`` and ``:511-653``), every variant of it:

    x_proj = GELU(down_proj(x))                      # [B, N, hidden]
    special, patches = x_proj[:, :S], x_proj[:, S:]  # S = N - indices.shape[1]
    patches += heatmap_gate * special[1 + cell(i)]   # heatmap injection (:311-355)
    processed = sparse_conv(patches, neighbor_indices)
    c = cat(special, processed)
    c = attention_branch(c)                          # use_attn >= 1 (:511-650)
    y = up_proj(c) * gamma + x

The heatmap injection runs when ``n_key_tokens > 1``, ``heatmap_grid_size``
is set and ``use_attn == 0``; ``use_attn`` 1-3 adds the attention over the
adapter tokens (1: all tokens, 2: visual tokens attend to the key tokens,
3: key tokens attend to the visual tokens; ``shortcut + attn_proj(.) *
attn_gamma``), 4 and above the temporal attention over frame-pooled tokens.

Without attention the module runs as one autograd node
(``SparseConvAdapterFunction``); its forward is the down GEMM
(``opentad_sparse_ops.adapter_down``), the heatmap gather-add when it
applies (``heatmap_add_``), the SparseConv2D forward (weight pack +
gathered GEMM) and the up GEMM (``opentad_sparse_ops.adapter_up``):

* the down GEMM's epilogue adds the bias, rounds the Linear output, applies
  GELU and writes the special tokens and the (contiguous) SparseConv2D input
  directly: no GELU pass and no slice copy;
* the up GEMM reads the special tokens and the SparseConv2D output in place of
  the concatenation and applies bias, ``gamma`` and the residual before its
  single store: no cat, no scale pass, no add pass;
* ``tokens_per_batch`` defaults to 0 (the tables the backbone builds are
  global), so there is no host sync; ``None`` restores the reference's
  ``max()`` heuristic (``sparse_conv_layer.py:174-177``).

With attention the adapter is a chain of nodes: the fused down GEMM
(``AdapterDownFunction``), SparseConv2D, the concatenation and the
reference's attention ops (LayerNorm, Linear, attention), then the same up
GEMM epilogue for both ``shortcut + attn_proj(.) * attn_gamma`` and
``up_proj(c) * gamma + x`` (``AdapterUpFunction`` with no special tokens: the
A rows are the ``[B, N, .]`` input itself). The attention is evaluated in
float32 (``_attention``).

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
over the token rows) use ``opentad_sparse_ops.column_sums``. The heatmap
injection's backward is the gather's: a scatter-add of ``g * gate`` into the
special-token gradient and ``sum(g * sampled)`` for the gate, in PyTorch.

The input gradient is one GEMM with the residual's term as its addend
(``addmm(go, du, W_d)``), which the single node makes possible.
``AdapterDownFunction`` and ``AdapterUpFunction`` are the same kernels as two
separate nodes around a ``SparseConv2d``.

The fused path runs in a compute dtype ``cd`` of float16 / bfloat16:

* outside autocast, the dtype of x when x and every parameter share it;
* under ``torch.autocast("cuda")`` with a float16 / bfloat16 target, the
  autocast dtype, with x and the parameters in it or in float32. This is how
  the reference runs the adapter: its training and test loops wrap the model
  in ``torch.cuda.amp.autocast(dtype=torch.bfloat16)`` with float32
  parameters (``opentad/cores/train_engine.py:672``,
  ``opentad/cores/test_engine.py:63``, ``amp=True`` in the vitsparse
  configs). The nodes cast x and the weights to ``cd`` as autocast casts
  them for ``nn.Linear`` and SparseConv2d (``sparse_conv_layer.py:191-202``).
  ``gamma`` stays float32, so ``up_proj(c) * gamma`` promotes to float32 as
  in the reference: the up GEMM's epilogue multiplies the rounded ``z`` by the
  float32 gamma and adds the residual in float32, and the output is float32.
  The heatmap injection adds ``sampled * gate`` in float32 with one rounding
  to ``cd`` (SparseConv2d's cast of its float32 input there). Gradients reach
  the parameters in their own dtype; the gradient of a float32 gain is summed
  in fp32 and stored as float32.

Any other call (float32 input and parameters without autocast, a CPU tensor,
mixed dtypes outside autocast, no kept tokens) runs ``reference_forward``:
the unfused chain in the reference's op order.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
from torch.autograd import Function

from . import opentad_sparse_ops as _ops
from .neighbor import _keep_symmetric, global_neighbor_table, is_symmetric_table
from .sparse_conv_layer import (BIAS_AFTER, BIAS_FP32, BIAS_NONE, IMPLICIT_GEMM_MIN_CIN, SparseConv2d)

_FUSED_DTYPES = (torch.float16, torch.bfloat16)


def _cast(t, dtype):
    """``t`` in ``dtype`` (None stays None): autocast's cast of an operand."""
    return t if t is None or t.dtype == dtype else t.to(dtype)


def _colsum(a):
    """Column sums of a [rows, n] matrix (the Linear bias gradients): fp32
    accumulation over row splits added in a fixed order, result in a's
    dtype. PyTorch's dim-0 reduction and a ones-vector GEMM take 24 and 58 µs
    at 17250 x 768."""
    return _ops.column_sums(a)


def _NO_ROWS(like):
    """Empty row list: the weight-gradient kernel then takes rows in order."""
    return torch.empty(0, dtype=torch.int32, device=like.device)


def _wgrad(g, rows, x, f32=False):
    """A Linear layer's weight gradient ``g[rows]^T x`` (``rows`` empty: the
    first ``len(x)`` rows of g) on the split-row kernel; widths that are not
    multiples of 64 (no tile configuration there) take a library GEMM. With
    ``f32`` the fp32 sums come back unrounded."""
    if g.shape[1] % 64 == 0 and x.shape[1] % 64 == 0:
        return _ops.linear_wgrad(g, rows, x, f32)
    gr = g.index_select(0, rows) if rows.numel() else g[: x.shape[0]]
    if f32:
        return torch.matmul(gr.t().float(), x.float())
    return torch.matmul(gr.t(), x)


def _up_wgrad(go, B, N, S, a_sp, a_pa):
    """``G = go^T cat(a_special, a_patch)`` of the up projection in fp32,
    unrounded (rounded once later, after the gamma scale, as the reference
    rounds the gradient of ``(c W^T + b) * gamma`` once): the patch rows on
    the split-row kernel (rows of go picked by a row list), the few special
    rows as a small fp32 product."""
    n = go.shape[-1]
    go2 = go.reshape(-1, n)
    if S == 0:
        return _wgrad(go2, _NO_ROWS(go2), a_pa, True)
    k = a_pa.shape[-1]
    G = _wgrad(go2, _patch_rows(B, N, S, go.device), a_pa, True)
    return G.add_(torch.matmul(go[:, :S].reshape(-1, n).t().float(), a_sp.reshape(-1, k).float()))


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
    """``(act_special, act_patch) = split(GELU(x W^T + b))``; x ``[B, N, k]``.
    ``cd`` (default: x's dtype) is the compute dtype that x, the weight and
    the bias are cast to (autocast's casts)."""

    @staticmethod
    def forward(ctx, x, weight, bias, n_special, cd=None):
        cd = x.dtype if cd is None else cd
        xc, wc, bc = _cast(x, cd), _cast(weight, cd), _cast(bias, cd)
        pre, sp, pa = _ops.adapter_down(xc, wc, bc, int(n_special))
        ctx.save_for_backward(xc, wc, pre)
        ctx.dtypes = (x.dtype, weight.dtype, None if bias is None else bias.dtype)
        ctx.n_special = int(n_special)
        return sp, pa

    @staticmethod
    def backward(ctx, g_sp, g_pa):
        xc, wc, pre = ctx.saved_tensors
        x_dt, w_dt, b_dt = ctx.dtypes
        n = pre.shape[-1]
        cd = pre.dtype
        # GELU backward straight from the two gradient buffers (no assembled dg)
        du = _ops.gelu_backward_split(_cast(g_sp, cd), _cast(g_pa, cd), pre, ctx.n_special)
        du2 = du.reshape(-1, n)
        gx = torch.matmul(du, wc).to(x_dt) if ctx.needs_input_grad[0] else None
        gw = _wgrad(du2, _NO_ROWS(du2), xc.reshape(-1, xc.shape[-1])).to(w_dt) if ctx.needs_input_grad[1] else None
        gb = _colsum(du2).to(b_dt) if b_dt is not None and ctx.needs_input_grad[2] else None
        return gx, gw, gb, None, None


class AdapterUpFunction(Function):
    """``out = z * gamma + residual``, ``z = T(cat(a_special, a_patch) W^T + b)``.

    ``cd`` (default: a_patch's dtype) is the compute dtype the A rows, the
    weight and the bias are cast to. With a gamma of ``cd`` the product is
    rounded to ``cd`` and so is the sum (residual of ``cd``). With a float32
    gamma (autocast, float32 parameters) the product and the residual add are
    float32; the output is float32 with ``out_float32`` (the reference's
    promotion of ``z * gamma + x``) and otherwise rounded once to ``cd``."""

    @staticmethod
    def forward(ctx, a_special, a_patch, weight, bias, gamma, residual, out_float32=False, cd=None):
        cd = a_patch.dtype if cd is None else cd
        sp, pa, wc, bc = _cast(a_special, cd), _cast(a_patch, cd), _cast(weight, cd), _cast(bias, cd)
        out = _ops.adapter_up(sp, pa, wc, bc, gamma, residual, bool(out_float32))
        ctx.save_for_backward(sp, pa, wc, bc, gamma)
        ctx.dtypes = (a_special.dtype, a_patch.dtype, weight.dtype, None if bias is None else bias.dtype,
                      residual.dtype)
        return out

    @staticmethod
    def backward(ctx, go):
        a_sp, a_pa, wc, bc, gamma = ctx.saved_tensors
        sp_dt, pa_dt, w_dt, b_dt, res_dt = ctx.dtypes
        B, N, n = go.shape
        S = a_sp.shape[1]
        k = wc.shape[1]
        go = go.contiguous()
        goc = _cast(go, wc.dtype)  # a float32 output gradient rounded to the compute dtype
        go2 = goc.reshape(-1, n)
        # go^T c without building c = cat(a_special, a_patch), in fp32
        G = _up_wgrad(goc, B, N, S, a_sp, a_pa)
        gsum = _colsum(go2)
        # gamma's gradient (in gamma's dtype) and the gamma-scaled W, G and
        # sum(go) in one pass
        g_gamma, w_g, gw, gb = _ops.up_proj_grads(wc, G, bc, gsum if bc is not None else None, gamma)
        g_gamma = g_gamma.view(gamma.shape) if ctx.needs_input_grad[4] else None
        g_sp = g_pa = None
        if ctx.needs_input_grad[0] or ctx.needs_input_grad[1]:
            # (go * gamma) W = go (gamma W): gamma folded into the small weight
            dc = torch.matmul(goc, w_g)  # [B, N, k]
            g_sp = dc[:, :S].to(sp_dt) if ctx.needs_input_grad[0] else None
            g_pa = dc[:, S:].reshape(-1, k).to(pa_dt) if ctx.needs_input_grad[1] else None
        gw = gw.to(w_dt) if ctx.needs_input_grad[2] else None
        gb = gb.to(b_dt) if b_dt is not None and ctx.needs_input_grad[3] else None
        return g_sp, g_pa, gw, gb, g_gamma, go.to(res_dt), None, None


class SparseConvAdapterFunction(Function):
    """The whole adapter (down GEMM + GELU, SparseConv2D, up GEMM + gamma +
    residual) as one autograd node, so that its backward can hand the input
    gradient's two terms to one GEMM: ``grad_x = go + du W_d`` is
    ``addmm(go, du, W_d)``, where the two-node chain computes ``du W_d`` and
    then autograd adds ``go`` in a separate pass over the 768-wide tokens.
    The kernels are those of ``AdapterDownFunction``, ``SparseConv2dFunction``
    and ``AdapterUpFunction``; ``packed`` is the SparseConv2D weight's
    ``(packed_fwd, packed_bwd)`` as ``SparseConv2dFunction`` takes it."""

    @staticmethod
    def forward(ctx, x, w_d, b_d, w_c, b_c, w_u, b_u, gamma, nbr, n_special, tpb, hm_rows=None, hm_gate=None,
                packed=None, cd=None):
        S = int(n_special)
        ctx.symmetric = is_symmetric_table(nbr)
        cd = x.dtype if cd is None else cd
        # autocast's casts (none when everything is already in cd); gamma and
        # the heatmap gate keep their dtype, as in the reference chain
        params = (w_d, b_d, w_c, b_c, w_u, b_u, gamma, hm_gate)
        ctx.dtypes = tuple(None if t is None else t.dtype for t in (x,) + params)
        xc = _cast(x, cd)
        w_d, b_d, w_c, b_c, w_u, b_u = (_cast(t, cd) for t in (w_d, b_d, w_c, b_c, w_u, b_u))
        pre, sp, pa = _ops.adapter_down(xc, w_d, b_d, S)
        if hm_rows is not None:
            # heatmap injection on the SparseConv2D input (in place)
            _ops.heatmap_add_(pa, sp, hm_rows, hm_gate)
        c_in = w_c.shape[1]
        if c_in % 4 != 0:
            raise ValueError(f"C_in ({c_in}) must be divisible by 4 for optimized kernel.")
        mode = BIAS_NONE if b_c is None else (BIAS_FP32 if c_in >= IMPLICIT_GEMM_MIN_CIN else BIAS_AFTER)
        need_bwd = any(ctx.needs_input_grad)
        if packed is None or (need_bwd and packed[1] is None):
            packed = _ops.pack_weight(w_c, True, need_bwd)
        pf, pb = packed
        processed = _ops.fwd_packed(pa, nbr, w_c, pf, b_c, tpb, mode)
        # z * gamma + x: float32 when gamma is a float32 parameter (the
        # reference's dtype promotion under autocast), else in cd
        out = _ops.adapter_up(sp, processed, w_u, b_u, gamma, x, gamma.dtype == torch.float32 and cd != gamma.dtype)
        ctx.save_for_backward(xc, w_d, pre, sp, pa, nbr, w_c, b_c, pb, processed, w_u, b_u, gamma, hm_rows, hm_gate)
        ctx.flags = (S, int(tpb), b_d is not None)
        return out

    @staticmethod
    def backward(ctx, go):
        x, w_d, pre, sp, pa, nbr, w_c, b_c, pb, processed, w_u, b_u, gamma, hm_rows, hm_gate = ctx.saved_tensors
        S, tpb, has_bd = ctx.flags
        x_dt, wd_dt, bd_dt, wc_dt, bc_dt, wu_dt, bu_dt, _, _ = ctx.dtypes
        need = ctx.needs_input_grad
        B, N, n = go.shape
        k = w_u.shape[1]
        cd = x.dtype
        go = go.contiguous()
        go_res = go  # the residual's gradient (float32 under autocast)
        go = _cast(go, cd)
        go2 = go.reshape(-1, n)
        # up projection: G = go^T cat(sp, processed) without the cat, in fp32
        G = _up_wgrad(go, B, N, S, sp, processed)
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
        gi_pa, gw_c, gb_c = _ops.bwd_packed(g_pa, pa, nbr, w_c, pb, w_c.shape[1], tpb, need_bc,
                                            symmetric=ctx.symmetric)
        g_gate = None
        if hm_rows is not None:
            # backward of patches + special[hm_rows] * gate: the gather's
            # scatter-add into the special-token gradient, and the gate's sum
            hidden = sp.shape[-1]
            sp_rows = sp.reshape(-1, hidden)
            if need[12]:
                g_gate = (gi_pa.float() * sp_rows.index_select(0, hm_rows).float()).sum().view(hm_gate.shape)
                g_gate = g_gate.to(hm_gate.dtype)
            # the products g * gate summed into the special-token gradient in
            # float32 and rounded to cd once: an index_add in cd rounds at
            # every atomic add, in an order that changes from run to run
            g_sp = g_sp.reshape(-1, hidden).float().index_add(0, hm_rows, gi_pa.float() * hm_gate.float())
            g_sp = g_sp.to(cd).view(sp.shape)
        # down projection: GELU backward from the two gradient buffers, then
        # the input gradient with the residual's go in the same GEMM
        du = _ops.gelu_backward_split(g_sp, gi_pa, pre, S)
        du2 = du.reshape(-1, du.shape[-1])
        x2 = x.reshape(-1, x.shape[-1])
        gx = None
        if need[0]:
            if x_dt == cd:
                gx = torch.addmm(go2, du2, w_d).view(x.shape)
            else:
                # float32 x under autocast: the down projection's gradient
                # (in cd) upcast and added to the residual's float32 gradient
                gx = torch.matmul(du2, w_d).to(x_dt).add_(go_res.reshape(-1, n)).view(x.shape)
        gw_d = _wgrad(du2, _NO_ROWS(du2), x2).to(wd_dt) if need[1] else None
        gb_d = _colsum(du2).to(bd_dt) if has_bd and need[2] else None
        return (gx, gw_d, gb_d, gw_c.to(wc_dt) if need[3] else None,
                gb_c.to(bc_dt) if need_bc else None, _cast(gw_u, wu_dt), _cast(gb_u, bu_dt), g_gamma,
                None, None, None, None, g_gate, None, None)


def _trunc_normal_init(layer, std):
    """mmengine's trunc_normal_init(layer, std=std, bias=0) as the reference calls
    it: weight ~ N(0, std) truncated to [-2, 2], bias 0."""
    nn.init.trunc_normal_(layer.weight, mean=0.0, std=std, a=-2.0, b=2.0)
    if getattr(layer, "bias", None) is not None:
        nn.init.zeros_(layer.bias)


def _attention(q, k, v):
    """Scaled dot-product attention ``softmax(q k^T / sqrt(d)) v`` evaluated in
    float32 with the operands made contiguous, result in q's dtype (the
    reference calls F.scaled_dot_product_attention in the module dtype)."""
    qf, kf, vf = q.float(), k.float(), v.float()
    s = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * (1.0 / math.sqrt(q.shape[-1]))
    return torch.matmul(torch.softmax(s, dim=-1), vf.contiguous()).to(q.dtype)


class SparseConvAdapter(nn.Module):
    """The reference adapter with ``conv_type="sparse_conv"``
    (vit_sparse_adapter_poguise.py:78-166,288-653): every ``use_attn`` variant
    and the heatmap injection, with the same parameter names, shapes and
    initialisation, on fused HIP GEMM epilogues."""

    def __init__(self, embed_dims: int, mlp_ratio: float = 0.25, conv_type: str = "sparse_conv",
                 use_attn=0, n_key_tokens: int = 1, heatmap_grid_size=None, **kwargs):
        super().__init__()
        if conv_type != "sparse_conv":
            raise NotImplementedError(f"SparseConvAdapter: conv_type {conv_type!r} (only 'sparse_conv')")
        self.conv_type = conv_type
        self.use_attn = int(use_attn)
        self.n_key_tokens = n_key_tokens
        self.heatmap_grid_size = heatmap_grid_size
        self.embed_dims = embed_dims
        hidden = int(embed_dims * mlp_ratio)
        hidden = int(2 ** round(math.log2(hidden)))  # power of two, as the reference rounds
        self.hidden_dims = hidden
        self.down_proj = nn.Linear(embed_dims, hidden)
        _trunc_normal_init(self.down_proj, 0.02)
        self.act = nn.GELU()
        self.up_proj = nn.Linear(hidden, embed_dims)
        nn.init.zeros_(self.up_proj.weight)
        nn.init.zeros_(self.up_proj.bias)
        self.gamma = nn.Parameter(torch.ones(1))
        if self.n_key_tokens > 1 and self.use_attn == 0:
            self.heatmap_gate = nn.Parameter(torch.zeros(1))
        if self.use_attn:
            self.attn_norm = nn.LayerNorm(hidden)
            self.attn_gamma = nn.Parameter(torch.ones(1))
            if self.use_attn >= 4:
                self.num_heads = max(1, hidden // 64)
                self.qkv = nn.Linear(hidden, hidden * 3, bias=False)
                _trunc_normal_init(self.qkv, 0.02)
                self.attn_proj = nn.Linear(hidden, hidden)
                _trunc_normal_init(self.attn_proj, 0.02)
                self.attn_mlp = nn.Sequential(nn.LayerNorm(hidden), nn.Linear(hidden, hidden), nn.GELU(),
                                              nn.Linear(hidden, hidden))
                _trunc_normal_init(self.attn_mlp[1], 0.02)
                nn.init.zeros_(self.attn_mlp[3].weight)
                nn.init.zeros_(self.attn_mlp[3].bias)
            else:
                attn_dim = hidden // 2
                self.num_heads = 4
                self.down_attn = nn.Linear(hidden, attn_dim)
                _trunc_normal_init(self.down_attn, 0.02)
                self.qkv = nn.Linear(attn_dim, attn_dim * 3)
                self.q_norm = nn.LayerNorm(attn_dim // self.num_heads)
                self.k_norm = nn.LayerNorm(attn_dim // self.num_heads)
                _trunc_normal_init(self.qkv, 0.02)
                self.attn_proj = nn.Linear(attn_dim, hidden)
                _trunc_normal_init(self.attn_proj, 0.02)
        self.sparse_conv = SparseConv2d(hidden, hidden)

    @staticmethod
    def _n_special(x, indices):
        return x.shape[1] - indices.shape[1]

    def _uses_heatmap(self):
        return self.n_key_tokens > 1 and self.heatmap_grid_size is not None and self.use_attn == 0

    def _heatmap_cells(self, indices, h, w):
        """Heatmap cell each kept token samples (vit_sparse_adapter_poguise.py:
        321-339): its spatial position, mapped to the heatmap grid by nearest
        index when the grids differ."""
        H_hm, W_hm = self.heatmap_grid_size
        spatial = indices % (h * w)
        if H_hm != h or W_hm != w:
            y = spatial // w
            xc = spatial % w
            return ((y * H_hm) // h) * W_hm + (xc * W_hm) // w
        return spatial

    def _fused_dtype(self, x):
        """The compute dtype of the fused path for input ``x``, or None when the
        call runs the unfused chain: outside autocast, x's float16 / bfloat16
        dtype when every parameter has it; under ``torch.autocast("cuda")``
        with a float16 / bfloat16 target, that target when x and every
        parameter are in it or in float32 (a float32 x needs a float32 gamma,
        which makes the output float32 as in the reference)."""
        if not x.is_cuda:
            return None
        dts = {p.dtype for p in self.parameters()}
        if torch.is_autocast_enabled("cuda"):
            cd = torch.get_autocast_dtype("cuda")
            if cd not in _FUSED_DTYPES or x.dtype not in (cd, torch.float32) or not dts <= {cd, torch.float32}:
                return None
            if x.dtype == torch.float32 and self.gamma.dtype != torch.float32:
                return None
            return cd
        if x.dtype in _FUSED_DTYPES and dts == {x.dtype}:
            return x.dtype
        return None

    def forward(self, x, h, w, indices, total_num_patches, neighbor_indices=None, tokens_per_batch=0):
        """``x [B, N, embed]``; ``indices [B, N_kept]`` (flattened ``t*h*w + y*w
        + x`` positions of the kept tokens); ``neighbor_indices`` ``[B, N_kept,
        9]`` or ``[B * N_kept, 9]``. ``total_num_patches`` is ``T*h*w``."""
        cd = self._fused_dtype(x)
        if cd is None or indices.shape[1] == 0:
            return self.reference_forward(x, h, w, indices, total_num_patches, neighbor_indices)
        B, N, _ = x.shape
        S = self._n_special(x, indices)
        if tokens_per_batch is None:
            # the reference's max() < N rule, on the device (no host sync)
            nbr, tokens_per_batch = global_neighbor_table(neighbor_indices, indices.shape[1]), 0
        else:
            nbr = neighbor_indices.reshape(-1, 9)
            if nbr.dtype != torch.int32:
                nbr = nbr.to(torch.int32)
            nbr = _keep_symmetric(neighbor_indices, nbr)
        conv = self.sparse_conv
        if not self.use_attn:
            hm_rows = hm_gate = None
            if self._uses_heatmap():
                H_hm, W_hm = self.heatmap_grid_size
                if S < 1 + H_hm * W_hm:
                    raise ValueError(f"SparseConvAdapter: {S} special tokens hold no {H_hm}x{W_hm} heatmap after CLS")
                cells = self._heatmap_cells(indices, h, w)
                base = torch.arange(B, device=x.device).view(B, 1) * S + 1
                hm_rows = (base + cells).reshape(-1).to(torch.int32)
                hm_gate = self.heatmap_gate
            cache = conv.packed_weight_cache
            packed = None
            if cache is not None:
                packed = cache.get(conv.weight, _cast(conv.weight, cd), torch.is_grad_enabled())
            return SparseConvAdapterFunction.apply(x, self.down_proj.weight, self.down_proj.bias, conv.weight,
                                                   conv.bias, self.up_proj.weight, self.up_proj.bias, self.gamma,
                                                   nbr, S, tokens_per_batch, hm_rows, hm_gate, packed, cd)
        sp, pa = AdapterDownFunction.apply(x, self.down_proj.weight, self.down_proj.bias, S, cd)
        processed = conv(pa, nbr, tokens_per_batch=tokens_per_batch)
        x_comb = torch.cat([sp, processed.view(B, N - S, -1)], dim=1)
        x_comb = self._attention_branch(x_comb, S, indices, h, w, total_num_patches, fused=True, cd=cd)
        empty = x_comb.new_empty(B, 0, x_comb.shape[-1])
        return AdapterUpFunction.apply(empty, x_comb.reshape(B * N, -1), self.up_proj.weight, self.up_proj.bias,
                                       self.gamma, x, self.gamma.dtype == torch.float32 and cd != torch.float32, cd)

    def _attention_branch(self, x_comb, S, indices, h, w, total_num_patches, fused, cd=None):
        """The ``use_attn`` branch on ``x_combined`` (vit_sparse_adapter_poguise.py:
        511-650). With ``fused`` the ``shortcut + attn_proj(.) * attn_gamma`` of
        variants 1-3 runs on the up GEMM's epilogue, in the compute dtype
        ``cd``. Under autocast with a float32 ``attn_gamma`` the reference's
        sum is float32 and its only consumer, ``up_proj``, casts it to the
        autocast dtype; the epilogue rounds the float32 sum to ``cd`` once,
        which gives that cast's values directly."""
        shortcut = x_comb
        B, N, C = x_comb.shape
        if self.use_attn >= 4:
            # temporal attention over frame-pooled tokens (:513-596)
            special = x_comb[:, :S]
            patches = x_comb[:, S:]
            hw = h * w
            frame = indices // hw
            n_frames = total_num_patches // hw
            idx = frame.unsqueeze(-1).expand(-1, -1, C)
            # The fused path sums the frames, and the gather's backward sums
            # the patch gradients per frame, in float32 and rounds once; the
            # reference's scatter_add in the module dtype rounds at every
            # atomic add, in an order that changes from run to run.
            acc = torch.float32 if fused else patches.dtype
            feats = patches.new_zeros(B, n_frames, C, dtype=acc).scatter_add(1, idx, patches.to(acc))
            counts = patches.new_zeros(B, n_frames, 1, dtype=acc).scatter_add(
                1, frame.unsqueeze(-1), torch.ones_like(frame, dtype=acc).unsqueeze(-1))
            feats = (feats / (counts + 1e-6)).to(patches.dtype)
            attn_in = torch.cat([special, feats], dim=1)
            xa = self.attn_norm(attn_in)
            qkv = self.qkv(xa).reshape(B, -1, 3, self.num_heads, C // self.num_heads).permute(2, 0, 3, 1, 4)
            xa = _attention(qkv[0], qkv[1], qkv[2]).transpose(1, 2).reshape(B, -1, C)
            xa = self.attn_proj(xa)
            coarse = xa + self.attn_mlp(xa)
            sp_out = coarse[:, :S]
            fr_out = coarse[:, S:]
            pa_out = torch.gather(fr_out.float(), 1, idx).to(fr_out.dtype) if fused else torch.gather(fr_out, 1, idx)
            return shortcut + torch.cat([sp_out, pa_out], dim=1)
        xa = self.down_attn(self.attn_norm(x_comb))
        A = xa.shape[-1]
        hd = A // self.num_heads
        q, k, v = self.qkv(xa).reshape(B, N, 3, self.num_heads, hd).permute(2, 0, 3, 1, 4)
        q = self.q_norm(q)
        k = self.k_norm(k)
        nk = self.n_key_tokens
        if self.use_attn == 2:  # visual tokens attend to the key tokens (:608-620)
            vis = _attention(q[:, :, nk:], k[:, :, :nk], v[:, :, :nk])
            xa = torch.cat([torch.zeros_like(q[:, :, :nk]), vis], dim=2)
        elif self.use_attn == 3:  # key tokens attend to the visual tokens (:621-634)
            key = _attention(q[:, :, :nk], k[:, :, nk:], v[:, :, nk:])
            xa = torch.cat([key, torch.zeros_like(q[:, :, nk:])], dim=2)
        else:
            xa = _attention(q, k, v)
        xa = xa.transpose(1, 2).reshape(B, N, A)
        if fused:
            empty = xa.new_empty(B, 0, A)
            return AdapterUpFunction.apply(empty, xa.reshape(B * N, A), self.attn_proj.weight, self.attn_proj.bias,
                                           self.attn_gamma, shortcut, False, cd)
        return shortcut + self.attn_proj(xa) * self.attn_gamma

    def reference_forward(self, x, h, w, indices, total_num_patches, neighbor_indices=None):
        """The unfused chain in the reference's op order
        (vit_sparse_adapter_poguise.py:288-362,511-653), including its
        ``.max()`` heuristic inside SparseConv2d and its autocast casts."""
        inputs = x
        x_proj = self.act(self.down_proj(x))
        S = self._n_special(x, indices)
        special = x_proj[:, :S, :]
        patches = x_proj[:, S:, :]
        if self._uses_heatmap():
            heat = special[:, 1:, :]
            cells = self._heatmap_cells(indices, h, w)
            sampled = torch.gather(heat, 1, cells.unsqueeze(-1).expand(-1, -1, self.hidden_dims))
            patches = patches + sampled * self.heatmap_gate
        if patches.shape[1] == 0:
            # the reference applies the activation a second time here (:356-358)
            return self.up_proj(self.act(x_proj)) * self.gamma + inputs
        processed = self.sparse_conv(patches, neighbor_indices)
        x_comb = torch.cat([special, processed], dim=1)
        if self.use_attn:
            x_comb = self._attention_branch(x_comb, S, indices, h, w, total_num_patches, fused=False)
        return self.up_proj(x_comb) * self.gamma + inputs
