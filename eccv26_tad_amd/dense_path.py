"""The dense 3x3 convolution path of the sparse adapter, kept as the comparator
for SparseConv2D.

The reference adapter (``opentad/models/backbones/vit_sparse_adapter_poguise.py``)
has a ``conv_type == "2d_conv"`` variant next to ``"sparse_conv"``: an
``nn.Conv2d(hidden, hidden, 3, padding=1)`` (``:163-171``) run on the kept
tokens by scattering them into a zero grid, convolving every frame in NCHW,
and gathering the kept positions back (``:372-412``, gather ``:484-490``).
This module restates that path on PyTorch (MIOpen convolution), so that the
speedup figures use the denominator the paper's model would run, and so that
the sparse kernels can be checked against a dense convolution on the same
tokens: for a neighbor table built from the same keep set, SparseConv2D and
this path compute the same function.

Weight layouts: ``nn.Conv2d`` holds ``(C_out, C_in, 3, 3)``; SparseConv2d holds
``(9, C_in, C_out)`` with ``k = ky * 3 + kx``, the re-layout the reference's
SparseConv2d init applies (``sparse_conv_layer.py:145-161``).
"""
from __future__ import annotations

import torch


def sparse_weight_from_conv2d(weight: torch.Tensor) -> torch.Tensor:
    """``(C_out, C_in, 3, 3)`` -> ``(9, C_in, C_out)``."""
    c_out, c_in = weight.shape[0], weight.shape[1]
    if tuple(weight.shape[2:]) != (3, 3):
        raise ValueError(f"expected a 3x3 kernel, got {tuple(weight.shape)}")
    return weight.reshape(c_out, c_in, 9).permute(2, 1, 0).contiguous()


def conv2d_weight_from_sparse(weight: torch.Tensor) -> torch.Tensor:
    """``(9, C_in, C_out)`` -> ``(C_out, C_in, 3, 3)``."""
    if weight.dim() != 3 or weight.shape[0] != 9:
        raise ValueError(f"expected (9, C_in, C_out), got {tuple(weight.shape)}")
    return weight.permute(2, 1, 0).reshape(weight.shape[2], weight.shape[1], 3, 3).contiguous()


def keep_mask_from_indices(indices: torch.Tensor, T: int, h: int, w: int) -> torch.Tensor:
    """Kept-token indices ``(B, N_kept)`` (flattened ``t*h*w + y*w + x``
    positions per sample) -> uint8 keep mask ``(B, T, h, w)``, on the indices'
    device, without a host sync. With sorted indices the kept tokens are in
    the row order of ``build_neighbor_table(mask)``."""
    B = indices.shape[0]
    mask = torch.zeros(B, T * h * w, dtype=torch.uint8, device=indices.device)
    mask.scatter_(1, indices.long(), 1)
    return mask.view(B, T, h, w)


def dense_conv_tokens(patch_tokens: torch.Tensor, indices: torch.Tensor, total_num_patches: int,
                      h: int, w: int, conv) -> torch.Tensor:
    """The ``2d_conv`` branch of the reference adapter on the kept tokens.

    ``patch_tokens`` ``(B, N_kept, C_in)``, ``indices`` ``(B, N_kept)`` into the
    ``total_num_patches = T*h*w`` grid of each sample, ``conv`` a callable on
    ``(B*T, C_in, h, w)`` (an ``nn.Conv2d`` in the reference). Returns the
    convolved kept tokens ``(B, N_kept, C_out)``. Without pruning
    (``N_kept == total_num_patches``) the tokens are the grid and are used in
    place, as in the reference (which then assumes the identity order).
    """
    B, N, C = patch_tokens.shape
    T = total_num_patches // (h * w)
    no_pruning = indices.shape[1] == total_num_patches
    if no_pruning:
        tokens = patch_tokens
    else:
        grid = patch_tokens.new_zeros(B, total_num_patches, C)
        tokens = grid.scatter(1, indices.long().unsqueeze(-1).expand(-1, -1, C), patch_tokens)
    conv_in = tokens.reshape(B * T, h, w, C).permute(0, 3, 1, 2).contiguous()
    conv_out = conv(conv_in)
    c_out = conv_out.shape[1]
    full = conv_out.permute(0, 2, 3, 1).reshape(B, -1, c_out)
    if no_pruning:
        return full
    return torch.gather(full, 1, indices.long().unsqueeze(-1).expand(-1, -1, c_out))
