"""Neighbor-index table utilities over the HIP table kernels.

The reference builds and remaps its tables with ~25 small torch launches in the
backbones (opentad/models/backbones/vit_sparse_adapter_poguise.py:1623-1670,
913-977; internvideo_next.py:1896-1945, 1447-1492). Here each is one to three
integer kernels with bit-identical output.
"""
from __future__ import annotations

import torch

from . import opentad_sparse_ops as _ops


def build_neighbor_table(mask: torch.Tensor, batched: bool = False) -> torch.Tensor:
    """Table from a keep mask ``[B, T, H, W]`` (or any ``[..., H, W]``).

    Returns int32 ``[N, 9]`` of global indices (-1 = missing) with
    k = (dy+1)*3 + (dx+1), rows in flattened mask order. With ``batched=True``
    and a 4-D mask whose samples keep equal counts, returns ``[B, N/B, 9]``.
    """
    table = _ops.build_neighbor_table(mask)
    if batched:
        B = mask.shape[0]
        if table.shape[0] % B:
            raise ValueError("batched=True needs the same number of kept cells per sample")
        table = table.view(B, table.shape[0] // B, 9)
    return table


def get_initial_neighbor_indices(h: int, w: int, T: int, device, B: int,
                                 dtype: torch.dtype = torch.int32) -> torch.Tensor:
    """Full-grid table ``(B, T*h*w, 9)`` of global indices, as
    ``get_initial_neighbor_indices`` (vit_sparse_adapter_poguise.py:1623-1670 with
    int32; internvideo_next.py:1896-1945 with int64)."""
    mask = torch.ones((B, T, h, w), dtype=torch.uint8, device=device)
    table = _ops.build_neighbor_table(mask).view(B, T * h * w, 9)
    return table if dtype == torch.int32 else table.to(dtype)


def remap_neighbor_table(neighbor_indices: torch.Tensor, keep_idx: torch.Tensor) -> torch.Tensor:
    """Table after a prune: keep the rows ``keep_idx`` ``[B, N_new]`` (local
    indices, as from topk) of ``neighbor_indices`` ``[B, N_prev, 9]`` and map
    every global entry to its new global index, -1 for pruned
    (vit_sparse_adapter_poguise.py:913-977). Output dtype follows the input."""
    dt = neighbor_indices.dtype
    t = neighbor_indices if dt == torch.int32 else neighbor_indices.to(torch.int32)
    out = _ops.remap_neighbor_table(t, keep_idx)
    return out if dt == torch.int32 else out.to(dt)


def prune_tokens(x: torch.Tensor, keep_idx: torch.Tensor, last_idx=None, neighbor_indices=None,
                 num_key_tokens: int = 0):
    """The Block prune step (vit_sparse_adapter_poguise.py:899-977) in two or
    three launches.

    ``x`` is ``[B, num_key_tokens + N_prev, C]``, where the first
    ``num_key_tokens`` rows are kept as they are. ``keep_idx`` ``[B, N_new]``
    holds local indices into the ``N_prev`` other rows, as from topk.

    Returns ``(x_new, idx_new, neighbor_indices_new)``:
    * ``x_new = cat(x[:, :S], gather(x[:, S:], keep_idx))``;
    * ``idx_new = gather(last_idx, keep_idx)``, or None without ``last_idx``;
    * the table remapped like ``remap_neighbor_table``, or None without
      ``neighbor_indices``. Its dtype follows the input.
    """
    empty = torch.empty(0, dtype=torch.long, device=x.device)
    tab = empty
    dt = None
    if neighbor_indices is not None:
        dt = neighbor_indices.dtype
        tab = neighbor_indices if dt == torch.int32 else neighbor_indices.to(torch.int32)
    last = empty if last_idx is None else last_idx
    x_new, idx_new, t_new = _ops.prune_tokens(x, keep_idx, last, tab, int(num_key_tokens))
    if last_idx is None:
        idx_new = None
    elif idx_new.dtype != last_idx.dtype:
        idx_new = idx_new.to(last_idx.dtype)
    if neighbor_indices is None:
        t_new = None
    elif dt != torch.int32:
        t_new = t_new.to(dt)
    return x_new, idx_new, t_new


def transpose_neighbor_table(table: torch.Tensor, tokens_per_batch: int = 0):
    """``(table_t, collisions)``: table_t[j,k] = i where src(i,k) = j. For
    mask-built tables table_t[:, k] == table[:, 8-k] and collisions == 0."""
    t = table.reshape(-1, 9)
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    tt, coll = _ops.transpose_neighbor_table(t, tokens_per_batch)
    return tt, int(coll.item())


def validate_neighbor_table(neighbor_indices, num_tokens: int, where: str = "") -> None:
    """Raise RuntimeError if the table does not match ``num_tokens`` or holds an
    entry outside {-1} U [0, B*N) (checks of _validate_neighbor_indices,
    internvideo_next.py:41-70)."""
    if neighbor_indices is None:
        return
    B, N, K = neighbor_indices.shape
    if N != num_tokens:
        raise RuntimeError(
            f"[sparse-conv check @ {where}] neighbor_indices second dim ({N}) != current "
            f"patch-token count ({num_tokens}). neighbor_indices is out of sync with the "
            f"pruned token set.")
    t = neighbor_indices if neighbor_indices.dtype == torch.int32 else neighbor_indices.to(torch.int32)
    stats = _ops.validate_neighbor_table(t, B * N).cpu()
    bad, vmin, vmax = (int(v) for v in stats)
    if bad:
        raise RuntimeError(
            f"[sparse-conv check @ {where}] neighbor index out of bounds: min={vmin}, "
            f"max={vmax}, valid range [0, {B * N}) for B={B}, N={N}.")
