"""Float32 restatement of the reference adapter's forward for the adapter tests.

Follows the ``conv_type == "sparse_conv"`` adapter of
``opentad/models/backbones/vit_sparse_adapter_poguise.py`` (forward
``:288-362``, attention branch ``:511-650``, output ``:652-653``) op for op,
with plain PyTorch functional ops in float32 on copies of a module's
parameters. The sparse convolution is NOT this repository's kernel: it is the
reference's dense ``2d_conv`` path on the kept tokens (scatter into the zero
grid, ``F.conv2d(padding=1)``, gather; ``eccv26_tad_amd.dense_path``), which
equals the sparse convolution for a neighbor table built from the same keep
set and is pinned to the CPU oracle in ``tests/test_dense_path.py``. The
attention is written out (softmax of the scaled scores times the values) in
float32 rather than calling ``F.scaled_dot_product_attention``.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def _attn(q, k, v):
    s = torch.matmul(q, k.transpose(-1, -2).contiguous()) / math.sqrt(q.shape[-1])
    return torch.matmul(torch.softmax(s, dim=-1), v)


def gain_scales(gains):
    """For each scalar gain (gamma, attn_gamma, heatmap_gate) of an
    ``adapter_fp32`` forward whose backward has run: the sum of the absolute
    terms of its gradient, sum |dL/d(out) * (what the gain multiplies)|, the
    natural scale of that cancelling sum."""
    return {name: float((out.grad.double() * term.double()).abs().sum()) for name, (out, term) in gains.items()}


def adapter_fp32(mod, x, h, w, indices, total_num_patches, gains=None):
    """Returns ``(y, params)``: the reference adapter's output for ``x`` (any
    dtype; computed in float32) and the float32 leaf copies of ``mod``'s
    parameters it used (their ``.grad`` after ``y.backward``). With a dict
    ``gains``, each scalar gain's (product output, multiplied term) pair is
    recorded in it for ``gain_scales``."""
    from eccv26_tad_amd.dense_path import conv2d_weight_from_sparse, dense_conv_tokens

    P = {name: p.detach().float().clone().requires_grad_(True) for name, p in mod.named_parameters()}
    x = x.float()
    B, N, _ = x.shape
    S = N - indices.shape[1]
    hid = mod.hidden_dims
    x_proj = F.gelu(F.linear(x, P["down_proj.weight"], P["down_proj.bias"]))
    special, patches = x_proj[:, :S], x_proj[:, S:]
    if mod.n_key_tokens > 1 and mod.heatmap_grid_size is not None and mod.use_attn == 0:
        H_hm, W_hm = mod.heatmap_grid_size
        sp_idx = indices % (h * w)
        if (H_hm, W_hm) != (h, w):
            sp_idx = ((sp_idx // w) * H_hm // h) * W_hm + (sp_idx % w) * W_hm // w
        sampled = torch.gather(special[:, 1:], 1, sp_idx.long().unsqueeze(-1).expand(-1, -1, hid))
        injected = sampled * P["heatmap_gate"]
        patches = patches + injected
        if gains is not None:
            injected.retain_grad()
            gains["heatmap_gate"] = (injected, sampled.detach())
    wc = conv2d_weight_from_sparse(P["sparse_conv.weight"])
    bc = P.get("sparse_conv.bias")
    processed = dense_conv_tokens(patches, indices, total_num_patches, h, w,
                                  lambda t: F.conv2d(t, wc, bc, padding=1))
    xc = torch.cat([special, processed], dim=1)
    if mod.use_attn:
        shortcut = xc
        if mod.use_attn >= 4:
            hw = h * w
            frame = (indices // hw).long()
            T = total_num_patches // hw
            idx = frame.unsqueeze(-1).expand(-1, -1, hid)
            feats = xc.new_zeros(B, T, hid).scatter_add(1, idx, processed)
            counts = xc.new_zeros(B, T, 1).scatter_add(1, frame.unsqueeze(-1), torch.ones_like(frame, dtype=xc.dtype).unsqueeze(-1))
            feats = feats / (counts + 1e-6)
            a_in = torch.cat([special, feats], dim=1)
            xa = F.layer_norm(a_in, (hid,), P["attn_norm.weight"], P["attn_norm.bias"])
            H = mod.num_heads
            qkv = F.linear(xa, P["qkv.weight"]).reshape(B, -1, 3, H, hid // H).permute(2, 0, 3, 1, 4)
            xa = _attn(qkv[0], qkv[1], qkv[2]).transpose(1, 2).reshape(B, -1, hid)
            xa = F.linear(xa, P["attn_proj.weight"], P["attn_proj.bias"])
            m = F.layer_norm(xa, (hid,), P["attn_mlp.0.weight"], P["attn_mlp.0.bias"])
            m = F.linear(F.gelu(F.linear(m, P["attn_mlp.1.weight"], P["attn_mlp.1.bias"])),
                         P["attn_mlp.3.weight"], P["attn_mlp.3.bias"])
            coarse = xa + m
            xc = shortcut + torch.cat([coarse[:, :S], torch.gather(coarse[:, S:], 1, idx)], dim=1)
        else:
            xa = F.layer_norm(xc, (hid,), P["attn_norm.weight"], P["attn_norm.bias"])
            xa = F.linear(xa, P["down_attn.weight"], P["down_attn.bias"])
            A = xa.shape[-1]
            H = mod.num_heads
            hd = A // H
            q, k, v = F.linear(xa, P["qkv.weight"], P["qkv.bias"]).reshape(B, N, 3, H, hd).permute(2, 0, 3, 1, 4)
            q = F.layer_norm(q, (hd,), P["q_norm.weight"], P["q_norm.bias"])
            k = F.layer_norm(k, (hd,), P["k_norm.weight"], P["k_norm.bias"])
            nk = mod.n_key_tokens
            if mod.use_attn == 2:
                att = torch.cat([torch.zeros_like(q[:, :, :nk]), _attn(q[:, :, nk:], k[:, :, :nk], v[:, :, :nk])], dim=2)
            elif mod.use_attn == 3:
                att = torch.cat([_attn(q[:, :, :nk], k[:, :, nk:], v[:, :, nk:]), torch.zeros_like(q[:, :, nk:])], dim=2)
            else:
                att = _attn(q, k, v)
            att = att.transpose(1, 2).reshape(B, N, A)
            proj = F.linear(att, P["attn_proj.weight"], P["attn_proj.bias"])
            scaled = proj * P["attn_gamma"]
            xc = shortcut + scaled
            if gains is not None:
                scaled.retain_grad()
                gains["attn_gamma"] = (scaled, proj.detach())
    z = F.linear(xc, P["up_proj.weight"], P["up_proj.bias"])
    zg = z * P["gamma"]
    if gains is not None:
        zg.retain_grad()
        gains["gamma"] = (zg, z.detach())
    y = zg + x
    return y, P
