"""Neighbor-index table utilities over the HIP table kernels.

The reference builds and remaps its tables with ~25 small torch launches in the
backbones (opentad/models/backbones/vit_sparse_adapter_poguise.py:1623-1670,
913-977; internvideo_next.py:1896-1945, 1447-1492). Here each is one to three
integer kernels with bit-identical output.
"""
from __future__ import annotations

import os

import torch

from . import opentad_sparse_ops as _ops

# Debug validation of the table after every prune step, as the reference's
# OPENTAD_DEBUG_SPARSE=1 (internvideo_next.py:32-70, called at :454, :1387,
# :1426). Off by default: the check synchronises with the host.
DEBUG_SPARSE = os.environ.get("OPENTAD_DEBUG_SPARSE", "0") == "1"


def set_debug_sparse(enabled: bool) -> None:
    """Switch the prune-step table validation on or off at run time."""
    global DEBUG_SPARSE
    DEBUG_SPARSE = bool(enabled)


# A table built from a keep mask is symmetric: every entry (i, k) -> j has its
# partner (j, 8-k) -> i. The builders below record that on the tensor they
# return, with the tensor's version counter (shared with its views), so any
# in-place change drops the record. The backward ops skip their partner checks
# for a table that carries it (symmetric=True); every other table takes the
# checked path, which gives the same results for symmetric tables.
_SYM_ATTR = "_svtad_symmetric"


def mark_symmetric_table(table: torch.Tensor) -> torch.Tensor:
    """Record on ``table`` (returned) that every entry has its partner. For
    tables known to be built from a keep mask; a wrong record gives wrong
    backward-input gradients. An inference tensor (``torch.inference_mode``)
    has no version counter and gets no record."""
    if not table.is_inference():
        setattr(table, _SYM_ATTR, table._version)
    return table


def is_symmetric_table(table) -> bool:
    """Whether ``table`` carries the symmetric record and is unchanged since."""
    if table is None:
        return False
    v = getattr(table, _SYM_ATTR, None)
    return v is not None and v == table._version


def _keep_symmetric(src, out):
    """``out`` carries the record when ``src`` does (operations that keep the
    property: dtype and shape changes, the global-index conversion)."""
    if out is not None and is_symmetric_table(src):
        mark_symmetric_table(out)
    return out


def build_neighbor_table(mask: torch.Tensor, batched: bool = False, n: int | None = None,
                         dtype: torch.dtype = torch.int32) -> torch.Tensor:
    """Table from a keep mask ``[B, T, H, W]`` (or any ``[..., H, W]``).

    Returns ``[N, 9]`` of global indices (-1 = missing) with
    k = (dy+1)*3 + (dx+1), rows in flattened mask order, int32 or int64
    (``dtype``). With ``n``, the number of kept cells the caller knows (the
    backbone's top-k count), the build is one launch with no host
    synchronisation; rows past the mask's count are -1. Without it, the table
    is sized by reading the count back. With ``batched=True`` and a 4-D mask
    whose samples keep equal counts, returns ``[B, N/B, 9]``.
    """
    if n is None:
        table = _ops.build_neighbor_table(mask)
        if dtype != torch.int32:
            table = table.to(dtype)
    else:
        table = _ops.build_neighbor_table_n(mask, int(n), dtype == torch.int64)
    if batched:
        B = mask.shape[0]
        if table.shape[0] % B:
            raise ValueError("batched=True needs the same number of kept cells per sample")
        table = table.view(B, table.shape[0] // B, 9)
    return mark_symmetric_table(table)


def get_initial_neighbor_indices(h: int, w: int, T: int, device, B: int,
                                 dtype: torch.dtype = torch.int32) -> torch.Tensor:
    """Full-grid table ``(B, T*h*w, 9)`` of global indices, as
    ``get_initial_neighbor_indices`` (vit_sparse_adapter_poguise.py:1623-1670 with
    int32; internvideo_next.py:1896-1945 with int64): one launch of the closed
    form, no mask, no host synchronisation."""
    like = torch.empty(0, device=device)
    table = _ops.grid_neighbor_table(B * T, h, w, dtype == torch.int64, like)
    return mark_symmetric_table(table.view(B, T * h * w, 9))


def global_neighbor_table(neighbor_indices: torch.Tensor, tokens_per_batch: int) -> torch.Tensor:
    """int32 ``[rows, 9]`` global table from ``neighbor_indices`` ``[..., 9]``
    (int32 / int64): the reference wrapper's rule (sparse_conv_layer.py:170-177)
    evaluated on the device. When the table's maximum is below
    ``tokens_per_batch`` (N of a ``[B, N, C]`` input) the entries are
    per-sample indices and row i's valid entries get ``(i // N) * N`` added;
    otherwise they are global already. No host synchronisation. The result
    keeps the input's symmetric record."""
    return _keep_symmetric(neighbor_indices, _ops.table_to_global(neighbor_indices, int(tokens_per_batch)))


def remap_neighbor_table(neighbor_indices: torch.Tensor, keep_idx: torch.Tensor) -> torch.Tensor:
    """Table after a prune: keep the rows ``keep_idx`` ``[B, N_new]`` (local
    indices, as from topk) of ``neighbor_indices`` ``[B, N_prev, 9]`` and map
    every global entry to its new global index, -1 for pruned
    (vit_sparse_adapter_poguise.py:913-977). Output dtype follows the input.

    The result carries no symmetric record. It is symmetric only when each
    sample's keep indices are distinct, as topk's are; a repeated index leaves
    a copied row whose neighbors point back to one copy only. Checking that
    would read a result back to the host, so the backward ops check the
    partners of a remapped table instead (in the combined backward that adds
    nothing measurable)."""
    dt = neighbor_indices.dtype
    t = neighbor_indices if dt == torch.int32 else neighbor_indices.to(torch.int32)
    out = _ops.remap_neighbor_table(t, keep_idx)
    if DEBUG_SPARSE:
        validate_neighbor_table(out, keep_idx.shape[1], "remap_neighbor_table")
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
    else:
        if DEBUG_SPARSE:
            validate_neighbor_table(t_new, keep_idx.shape[1], "prune_tokens")
        if dt != torch.int32:
            t_new = t_new.to(dt)  # no symmetric record, as remap_neighbor_table
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
