"""Committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from a numpy restatement of the reference's table
procedures and from dense float64 conv2d) checked against the CPU oracle and,
on a GPU, against the HIP kernels through opentad_sparse_ops.

Bar: tables bit-exact; convolution max-scaled error <= 1e-12 (fp64), 1e-5
(fp32), 1e-2 (fp16 / bf16). Fixture inputs are exact in every dtype.
"""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = {"float64": 1e-12, "float32": 1e-5, "float16": 1e-2, "bfloat16": 1e-2}


def load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


# --------------------------------------------------------------------------
# oracle (CPU)
# --------------------------------------------------------------------------

def test_oracle_initial_table(oracle):
    g = load("table_initial")
    B, T, h, w = int(g["B"]), int(g["T"]), int(g["h"]), int(g["w"])
    got = oracle.build_table(np.ones((B, T, h, w), np.uint8))
    np.testing.assert_array_equal(got, g["table"].reshape(-1, 9))


def test_oracle_pruned_table(oracle):
    g = load("table_pruned")
    np.testing.assert_array_equal(oracle.build_table(g["mask"]), g["table"].reshape(-1, 9))
    B, T, H, W = g["mask"].shape
    t = oracle.ref_initial_table(H, W, T, B)
    for key in ("keep0", "keep1"):
        t = oracle.remap_table(t, g[key])
    np.testing.assert_array_equal(t, g["table"])


def test_oracle_conv(oracle):
    g = load("conv")
    t = oracle.build_table(g["mask"])
    assert oracle.rel_err(oracle.fwd(g["x"], t, g["w"], g["b"]), g["y"]) <= 1e-12
    assert oracle.rel_err(oracle.bwd_in(g["go"], t, g["w"]), g["gi"]) <= 1e-12
    assert oracle.rel_err(oracle.bwd_w(g["go"], g["x"], t), g["gw"]) <= 1e-12
    assert oracle.rel_err(oracle.bias_grad(g["go"]), g["gb"]) <= 1e-12


def test_oracle_depthwise(oracle):
    g = load("depthwise")
    t = oracle.build_table(g["mask"])
    assert oracle.rel_err(oracle.dw_fwd(g["x"], t, g["w"], g["b"]), g["y"]) <= 1e-12
    assert oracle.rel_err(oracle.dw_bwd_in(g["go"], t, g["w"]), g["gi"]) <= 1e-12
    assert oracle.rel_err(oracle.dw_bwd_w(g["go"], g["x"], t), g["gw"]) <= 1e-12


# --------------------------------------------------------------------------
# HIP kernels (GPU)
# --------------------------------------------------------------------------

def _err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


@pytest.mark.gpu
def test_hip_tables(dev):
    import torch

    import eccv26_tad_amd as sv

    g = load("table_initial")
    B, T, h, w = int(g["B"]), int(g["T"]), int(g["h"]), int(g["w"])
    init = sv.get_initial_neighbor_indices(h, w, T, dev, B)
    np.testing.assert_array_equal(init.cpu().numpy(), g["table"])
    p = load("table_pruned")
    got = sv.build_neighbor_table(torch.from_numpy(p["mask"]).to(dev)).cpu().numpy()
    np.testing.assert_array_equal(got, p["table"].reshape(-1, 9))
    B, T, H, W = p["mask"].shape
    t = sv.get_initial_neighbor_indices(H, W, T, dev, B)
    for key in ("keep0", "keep1"):
        t = sv.remap_neighbor_table(t, torch.from_numpy(p[key]).to(dev))
    np.testing.assert_array_equal(t.cpu().numpy(), p["table"])


@pytest.mark.gpu
@pytest.mark.parametrize("dname", ["float64", "float32", "float16", "bfloat16"])
def test_hip_conv(dev, dname):
    import torch

    import eccv26_tad_amd as sv

    ops = sv.ops
    g = load("conv")
    dt = getattr(torch, dname)
    T_ = sv.build_neighbor_table(torch.from_numpy(g["mask"]).to(dev))
    X, Wt, Bb, G = (torch.from_numpy(g[k]).to(dev, dt) for k in ("x", "w", "b", "go"))
    tol = TOL[dname]
    print("golden conv", dname, flush=True)
    assert _err(ops.implicit_gemm_fwd_v2(X, T_, Wt, Bb, 0).cpu().double(), g["y"]) <= tol
    assert _err(ops.bwd_in(G, T_, Wt, X.shape[0], X.shape[1], 0).cpu().double(), g["gi"]) <= tol
    gw, gb = ops.bwd_w_bias(G, X, T_, X.shape[1], 0, True)
    assert _err(gw.cpu().double(), g["gw"]) <= tol
    assert _err(gb.cpu().double(), g["gb"]) <= tol


@pytest.mark.gpu
@pytest.mark.parametrize("dname", ["float32", "float16", "bfloat16"])
def test_hip_depthwise(dev, dname):
    import torch

    import eccv26_tad_amd as sv

    ops = sv.ops
    g = load("depthwise")
    dt = getattr(torch, dname)
    T_ = sv.build_neighbor_table(torch.from_numpy(g["mask"]).to(dev))
    X, Wt, Bb, G = (torch.from_numpy(g[k]).to(dev, dt) for k in ("x", "w", "b", "go"))
    tol = TOL[dname]
    assert _err(ops.dw_fwd(X, T_, Wt, Bb, 0).cpu().double(), g["y"]) <= tol
    assert _err(ops.dw_bwd_in(G, T_, Wt, 0).cpu().double(), g["gi"]) <= tol
    gw, gb = ops.dw_bwd_w(G, X, T_, 0, True)
    assert _err(gw.cpu().double(), g["gw"]) <= tol
    assert _err(gb.cpu().double(), g["gb"]) <= tol
