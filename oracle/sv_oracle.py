"""CPU oracle for SparseConv2D (SV-TAD, pcr-upm/eccv26_tad).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, always as the checker or the timed CPU
restatement, never by the product path (``eccv26_tad_amd``).

Two layers:

* ``libsv_oracle.so`` (``sv_oracle.c``), reached through ctypes: the closed-form
  neighbor table, the step-by-step remap, and fp64 forward / backward-input /
  backward-weight / bias-grad for the full and depthwise convolutions, plus the
  OpenMP fp32 "port" of the reference dataflow that ``bench.py`` times.
* Pure numpy/Python restatements of the reference's *table procedures*, used to
  pin the C closed form:
  ``ref_initial_table`` restates ``get_initial_neighbor_indices``
  (opentad/models/backbones/vit_sparse_adapter_poguise.py:1623-1670), and
  ``ref_remap`` restates the Block remap (same file, :913-977), and
  ``ref_prune_step`` the whole prune step around it (:899-977).

Parity status: every function here is pinned by a check in
``tests/test_oracle.py`` that is independent of the function's own formula
(torch ``conv2d``/autograd on a zero-filled grid, brute force on tiny grids,
the numpy restatement of the reference procedure, symmetry invariants, and the
committed golden fixtures).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libsv_oracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile ``libsv_oracle.so`` with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-C", _HERE, "-B" if force else "all"], check=True,
                       stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        I = ctypes.c_int
        L.svo_count.restype = I64
        L.svo_count.argtypes = [P, I64]
        L.svo_build_table.argtypes = [P, I64, I64, I64, I64, P]
        L.svo_remap_table.argtypes = [P, I64, I64, P, I64, P, P]
        for nm in ("svo_fwd_f64",):
            getattr(L, nm).argtypes = [P, P, P, P, I64, I, I, I64, P]
        L.svo_bwd_in_f64.argtypes = [P, P, P, I64, I, I, I64, P]
        L.svo_bwd_w_f64.argtypes = [P, P, P, I64, I, I, I64, P]
        L.svo_bias_grad_f64.argtypes = [P, I64, I, P]
        L.svo_dw_fwd_f64.argtypes = [P, P, P, P, I64, I, I64, P]
        L.svo_dw_bwd_in_f64.argtypes = [P, P, P, I64, I, I64, P]
        L.svo_dw_bwd_w_f64.argtypes = [P, P, P, I64, I, I64, P]
        L.svo_fwd_f32.argtypes = [P, P, P, P, I64, I, I, I64, P, P, P]
        L.svo_bwd_in_f32.argtypes = [P, P, P, I64, I, I, I64, P]
        L.svo_bwd_w_f32.argtypes = [P, P, P, I64, I, I, I64, P]
        L.svo_num_threads.restype = I
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


# --------------------------------------------------------------------------
# neighbor table
# --------------------------------------------------------------------------

def build_table(mask: np.ndarray) -> np.ndarray:
    """Closed-form table from a keep mask ``[B,T,H,W]`` -> int32 ``[N,9]``."""
    m = np.ascontiguousarray(np.asarray(mask) != 0, dtype=np.uint8)
    assert m.ndim == 4
    B, T, H, W = m.shape
    n = int(lib().svo_count(_p(m), m.size))
    out = np.empty((n, 9), dtype=np.int32)
    lib().svo_build_table(_p(m), B, T, H, W, _p(out))
    return out


def remap_table(table: np.ndarray, keep_idx: np.ndarray) -> np.ndarray:
    """C restatement of the Block remap. ``table`` [B,N_prev,9] global, ``keep_idx`` [B,N_new]."""
    t = _i32(table)
    B, n_prev, _ = t.shape
    kp = np.ascontiguousarray(np.asarray(keep_idx, dtype=np.int64))
    n_new = kp.shape[1]
    ws = np.empty(B * n_prev, dtype=np.int32)
    out = np.empty((B, n_new, 9), dtype=np.int32)
    lib().svo_remap_table(_p(t), B, n_prev, _p(kp), n_new, _p(ws), _p(out))
    return out


def ref_initial_table(h: int, w: int, T: int, B: int) -> np.ndarray:
    """numpy restatement of get_initial_neighbor_indices
    (vit_sparse_adapter_poguise.py:1623-1670): pad the per-frame arange with -1,
    stack the 9 shifted slices (dy outer, dx inner), add t*h*w and b*T*h*w to
    the valid entries. Returns int32 ``[B, T*h*w, 9]``."""
    n_sp = h * w
    idx = np.arange(n_sp, dtype=np.int32).reshape(h, w)
    padded = np.full((h + 2, w + 2), -1, dtype=np.int32)
    padded[1:-1, 1:-1] = idx
    cols = []
    for dy in range(-1, 2):
        for dx in range(-1, 2):
            cols.append(padded[1 + dy:1 + dy + h, 1 + dx:1 + dx + w].reshape(-1))
    sp = np.stack(cols, axis=1)                              # (n_sp, 9)
    t = np.broadcast_to(sp, (T, n_sp, 9)).copy()
    t_off = (np.arange(T, dtype=np.int32) * n_sp).reshape(T, 1, 1)
    valid = t != -1
    t[valid] += np.broadcast_to(t_off, t.shape)[valid]
    t = t.reshape(T * n_sp, 9)
    b = np.broadcast_to(t, (B, T * n_sp, 9)).copy()
    b_off = (np.arange(B, dtype=np.int32) * (T * n_sp)).reshape(B, 1, 1)
    valid = b != -1
    b[valid] += np.broadcast_to(b_off, b.shape)[valid]
    return b


def ref_remap(table: np.ndarray, keep_idx: np.ndarray) -> np.ndarray:
    """numpy restatement of the Block remap (vit_sparse_adapter_poguise.py:913-977).
    ``table`` [B, N_prev, 9] global indices, ``keep_idx`` [B, N_new] local."""
    table = np.asarray(table, dtype=np.int32)
    keep_idx = np.asarray(keep_idx, dtype=np.int64)
    B, n_prev, _ = table.shape
    n_new = keep_idx.shape[1]
    kept = np.take_along_axis(table, np.repeat(keep_idx[:, :, None], 9, axis=2), axis=1)
    mapping = np.full(B * n_prev, -1, dtype=np.int32)
    old_global = (keep_idx + (np.arange(B) * n_prev)[:, None]).reshape(-1)
    new_global = (np.arange(n_new)[None, :] + (np.arange(B) * n_new)[:, None]).reshape(-1)
    mapping[old_global] = new_global.astype(np.int32)
    flat = kept.reshape(-1)
    valid = flat != -1
    new_flat = np.where(valid, mapping[np.clip(flat, 0, None)], np.int32(-1))
    return new_flat.reshape(B, n_new, 9).astype(np.int32)


def ref_prune_step(x: np.ndarray, keep_idx: np.ndarray, last_idx, table, n_key: int):
    """numpy restatement of the Block prune step (vit_sparse_adapter_poguise.py:899-977):
    ``x`` [B, n_key + N_prev, C] -> cat(x[:, :n_key], gather(x[:, n_key:], keep_idx));
    ``last_idx`` [B, N_prev] -> gather(last_idx, keep_idx) (:908); ``table``
    [B, N_prev, 9] -> the remapped table (:913-977, ``ref_remap``). ``last_idx``
    and ``table`` may be None (the reference skips the table when it is None, :913)."""
    x = np.asarray(x)
    keep_idx = np.asarray(keep_idx, dtype=np.int64)
    x_key = x[:, :n_key]
    x_nonkey = x[:, n_key:]
    kept = np.take_along_axis(x_nonkey, keep_idx[:, :, None], axis=1)
    x_new = np.concatenate([x_key, kept], axis=1)
    idx_new = None if last_idx is None else np.take_along_axis(np.asarray(last_idx, dtype=np.int64), keep_idx, axis=1)
    t_new = None if table is None else ref_remap(table, keep_idx)
    return x_new, idx_new, t_new


def ref_topk_sorted(score: np.ndarray, keep: int) -> np.ndarray:
    """Keep-set rule of KTPAttention (vit_sparse_adapter_poguise.py:763,785-787):
    top-``keep`` per row, then sorted ascending. Ties broken by lower index."""
    order = np.argsort(-score, axis=1, kind="stable")[:, :keep]
    return np.sort(order, axis=1)


# --------------------------------------------------------------------------
# full SparseConv2D, fp64
# --------------------------------------------------------------------------

def fwd(x, nbr, w, bias=None, tpb: int = 0) -> np.ndarray:
    x, nbr, w = _f32(x), _i32(nbr), _f32(w)
    n, ci = x.shape
    co = w.shape[2]
    b = _f32(bias) if bias is not None else None
    out = np.empty((n, co), dtype=np.float64)
    lib().svo_fwd_f64(_p(x), _p(nbr), _p(w), _p(b) if b is not None else None, n, ci, co, tpb, _p(out))
    return out


def bwd_in(go, nbr, w, tpb: int = 0) -> np.ndarray:
    go, nbr, w = _f32(go), _i32(nbr), _f32(w)
    n, co = go.shape
    ci = w.shape[1]
    gi = np.empty((n, ci), dtype=np.float64)
    lib().svo_bwd_in_f64(_p(go), _p(nbr), _p(w), n, ci, co, tpb, _p(gi))
    return gi


def bwd_w(go, x, nbr, tpb: int = 0) -> np.ndarray:
    go, x, nbr = _f32(go), _f32(x), _i32(nbr)
    n, co = go.shape
    ci = x.shape[1]
    gw = np.empty((9, ci, co), dtype=np.float64)
    lib().svo_bwd_w_f64(_p(go), _p(x), _p(nbr), n, ci, co, tpb, _p(gw))
    return gw


def bias_grad(go) -> np.ndarray:
    go = _f32(go)
    n, co = go.shape
    gb = np.empty(co, dtype=np.float64)
    lib().svo_bias_grad_f64(_p(go), n, co, _p(gb))
    return gb


# --------------------------------------------------------------------------
# depthwise SparseConv2D (groups = C), fp64; W layout (9, C)
# --------------------------------------------------------------------------

def dw_fwd(x, nbr, w, bias=None, tpb: int = 0) -> np.ndarray:
    x, nbr, w = _f32(x), _i32(nbr), _f32(w)
    n, c = x.shape
    b = _f32(bias) if bias is not None else None
    out = np.empty((n, c), dtype=np.float64)
    lib().svo_dw_fwd_f64(_p(x), _p(nbr), _p(w), _p(b) if b is not None else None, n, c, tpb, _p(out))
    return out


def dw_bwd_in(go, nbr, w, tpb: int = 0) -> np.ndarray:
    go, nbr, w = _f32(go), _i32(nbr), _f32(w)
    n, c = go.shape
    gi = np.empty((n, c), dtype=np.float64)
    lib().svo_dw_bwd_in_f64(_p(go), _p(nbr), _p(w), n, c, tpb, _p(gi))
    return gi


def dw_bwd_w(go, x, nbr, tpb: int = 0) -> np.ndarray:
    go, x, nbr = _f32(go), _f32(x), _i32(nbr)
    n, c = go.shape
    gw = np.empty((9, c), dtype=np.float64)
    lib().svo_dw_bwd_w_f64(_p(go), _p(x), _p(nbr), n, c, tpb, _p(gw))
    return gw


# --------------------------------------------------------------------------
# fp32 OpenMP port of the reference dataflow (timed CPU baseline)
# --------------------------------------------------------------------------

class Fp32Port:
    """Holds the workspaces of the fp32 port so that timing excludes allocation."""

    def __init__(self, n: int, ci: int, co: int):
        self.n, self.ci, self.co = n, ci, co
        self.xg = np.empty((9, n, ci), dtype=np.float32)
        self.of = np.empty((9, n, co), dtype=np.float32)
        self.out = np.empty((n, co), dtype=np.float32)
        self.gi = np.empty((n, ci), dtype=np.float32)
        self.gw = np.empty((9, ci, co), dtype=np.float32)

    def fwd(self, x, nbr, w, bias, tpb=0):
        lib().svo_fwd_f32(_p(x), _p(nbr), _p(w), _p(bias) if bias is not None else None,
                          self.n, self.ci, self.co, tpb, _p(self.xg), _p(self.of), _p(self.out))
        return self.out

    def bwd(self, go, x, nbr, w, tpb=0):
        lib().svo_bwd_in_f32(_p(go), _p(nbr), _p(w), self.n, self.ci, self.co, tpb, _p(self.gi))
        lib().svo_bwd_w_f32(_p(go), _p(x), _p(nbr), self.n, self.ci, self.co, tpb, _p(self.gw))
        return self.gi, self.gw


def num_threads() -> int:
    return int(lib().svo_num_threads())


# --------------------------------------------------------------------------
# tolerance metric
# --------------------------------------------------------------------------

def rel_err(got, ref) -> float:
    """Max-scaled error: max|got-ref| / max(max|ref|, tiny). Element-wise relative
    error is ill-conditioned where the reference is near zero."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if ref.size == 0:
        return 0.0
    scale = max(float(np.max(np.abs(ref))), 1e-30)
    return float(np.max(np.abs(got - ref))) / scale
