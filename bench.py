"""SparseConv2D fwd+bwd benchmark on one MI355X.

Workload (benchmark config 2, the ViT-B adapter bottleneck): B=2 samples x 80
temporal slices x 14x14 grid, C_in = C_out = 192, fp16, 3x3 sparse conv with
bias. Keep sets: per sample top-k of a seeded U(0,1) score (k = ceil(r*15680)),
sorted; the neighbor table is built on the GPU from the keep mask.

One step = the work of one training step of the op, exactly what
SparseConv2dFunction.forward/backward run: pack the weight for the matrix
cores (forward and backward-input layouts, one launch), forward (bias added in
fp32), backward-input, backward-weight with the bias gradient. Inputs are
resident in HBM before the timed region.

Printed: ONE JSON line on stdout. ``value`` is the algorithmic HBM throughput
of fwd+bwd (GB/s) at the headline keep rate; ``sweep`` holds us / GB/s /
TFLOP/s / speedup over a dense 3x3 conv (MIOpen, same shape) for every keep
rate, and over the reference adapter's dense path on the same kept tokens
(scatter -> conv2d -> gather, fwd + bwd), and ``gpu_us``, the step's GPU
time with the steps queued ahead of the GPU (at low keep rates the host
enqueues a step more slowly than the GPU runs it); ``roofline`` covers the
dominant kernel, timed with HIP events on the stream it is launched on; ``cpu_baseline`` times the OpenMP fp32 port of the
reference dataflow (oracle/, kind "port") on the host cores.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = {"f16": 2500.0, "bf16": 2500.0, "f32": 157.3, "f64": 78.6}
KEEPS = (0.10, 0.25, 0.40, 0.55, 0.70, 1.00)
B, T, H, W, C = 2, 80, 14, 14, 192
SEED = 1002  # 1000 + config id


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_mask(keep: float):
    """[B, T, H, W] uint8 keep mask: per sample top-k (k = ceil(keep*T*H*W)) of a
    seeded U(0,1) score, the keep-set rule of vit_sparse_adapter_poguise.py:763,785-787."""
    import torch

    g = torch.Generator().manual_seed(SEED)
    n = T * H * W
    k = math.ceil(keep * n)
    score = torch.rand(B, n, generator=g)
    idx = torch.topk(score, k, dim=1).indices
    m = torch.zeros(B, n, dtype=torch.uint8)
    m.scatter_(1, idx, 1)
    return m.view(B, T, H, W)


def op_bytes(n, ci, co, s):
    """Algorithmic HBM bytes of each pass (unique compulsory traffic):
    activations read/written once per pass, the int32 table (36 B/row) once per
    pass, the weight once per pass, bias / bias grad."""
    wsz = 9 * ci * co
    fwd = n * ci * s + n * co * s + 36 * n + wsz * s + 4 * co
    bwd_in = n * co * s + n * ci * s + 36 * n + wsz * s
    bwd_w = n * co * s + n * ci * s + 36 * n + wsz * s + co * s
    return {"fwd": fwd, "bwd_in": bwd_in, "bwd_w": bwd_w}


TRAFFIC_PROFILE = os.path.join("profiles", "sparseconv2d_c2_keep055_hbm_traffic.md")


def pmc_traffic(kernel_key):
    """HBM bytes per launch of the kernel whose name contains kernel_key: the
    committed rocprofv3 --pmc summary's last column, FETCH_SIZE and WRITE_SIZE
    (KiB per dispatch) each scaled by what the counter reads for a plain 1 GiB
    copy, for this workload at keep 0.55; None if absent."""
    try:
        with open(os.path.join(ROOT, TRAFFIC_PROFILE)) as f:
            for line in f:
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                if len(cells) == 5 and kernel_key in cells[0]:
                    return int(cells[4])
    except (OSError, ValueError):
        pass
    return None


def time_kernel(fn, reps, warm=3):
    """Per-launch duration of a single-kernel call fn(): ``(median, mean)``
    in ms over ``reps`` launches, each bracketed by its own pair of HIP
    events on torch's current stream (the stream the extension launches
    on), so a launch's time includes its dispatch but not the host's."""
    import torch

    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for s, e in evs:
        s.record()
        fn()
        e.record()
    torch.cuda.synchronize()
    t = sorted(s.elapsed_time(e) for s, e in evs)
    return t[len(t) // 2], sum(t) / len(t)


def time_events(fn, reps, warm=3):
    """Average ms per call of fn() from HIP events on torch's current stream,
    the stream the extension launches on."""
    import torch

    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps


def time_queued(fn, reps, warm=3):
    """Average ms per call of fn() on the GPU alone: the calls are queued
    behind a spinning kernel (torch.cuda._sleep) while the host enqueues
    them, and the events bracket only their execution, so a call whose host
    side takes longer than its GPU work is timed by the latter. The spin is
    lengthened until the host is done before it ends (checked with an event
    recorded at its end); None if it never is (the row then reports null)."""
    import torch

    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    cycles = 1 << 21
    for _ in range(6):
        h0, s, e = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        h0.record()
        torch.cuda._sleep(cycles)
        s.record()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        host_ms = (time.perf_counter() - t0) * 1e3
        e.record()
        torch.cuda.synchronize()
        if h0.elapsed_time(s) > 1.2 * host_ms:  # the spin outlasted the enqueueing
            return s.elapsed_time(e) / reps
        cycles *= 4
    log("bench: time_queued: the host did not finish enqueueing within the spin")
    return None


class Problem:
    def __init__(self, keep, dev, dtype):
        import torch

        import eccv26_tad_amd as sv

        self.ops = sv.ops
        self.keep = keep
        self.mask = make_mask(keep).to(dev)
        self.table = sv.build_neighbor_table(self.mask)
        self.n = int(self.table.shape[0])
        g = torch.Generator().manual_seed(SEED + 1)
        bound = 1.0 / math.sqrt(9 * C)
        self.x = torch.randn(self.n, C, generator=g).to(dev, dtype)
        self.w = ((torch.rand(9, C, C, generator=g) * 2 - 1) * bound).to(dev, dtype)
        self.b = ((torch.rand(C, generator=g) * 2 - 1) * bound).to(dev, dtype)
        self.go = torch.randn(self.n, C, generator=g).to(dev, dtype)
        self.valid = int((self.table >= 0).sum())
        # the builder's symmetric record: the autograd backward passes it to
        # the backward ops (no partner checks)
        self.sym = sv.is_symmetric_table(self.table)

        self.pf, self.pb = self.ops.pack_weight(self.w, True, True)

    # the calls SparseConv2dFunction makes (sparse_conv_layer.py)
    def pack(self):
        return self.ops.pack_weight(self.w, True, True)

    def fwd(self):
        return self.ops.fwd_packed(self.x, self.table, self.w, self.pf, self.b, 0, 1)

    def bwd_in(self):
        return self.ops.bwd_in_packed(self.go, self.table, self.w, self.pb, self.n, C, 0, symmetric=self.sym)

    def bwd_in_gemm(self):  # the gathered GEMM of bwd_in alone (no orphan-pass launch)
        return self.ops.bwd_in_gemm(self.go, self.table, self.pb, C, 0, symmetric=self.sym)

    def bwd_w(self):
        return self.ops.bwd_w_bias(self.go, self.x, self.table, C, 0, True)

    def bwd_w_partials(self):  # the partial-sum kernel of bwd_w alone
        return self.ops.bwd_w_partials(self.go, self.x, self.table, C, 0, True)

    def bwd(self):  # the autograd backward: bwd_in + bwd_w in one call
        return self.ops.bwd_packed(self.go, self.x, self.table, self.w, self.pb, C, 0, True, symmetric=self.sym)

    def bwd_checked(self):  # bwd with the partner checks (a table without the record)
        return self.ops.bwd_packed(self.go, self.x, self.table, self.w, self.pb, C, 0, True)

    def bwd_in_gemm_checked(self):
        return self.ops.bwd_in_gemm(self.go, self.table, self.pb, C, 0)

    def step(self):
        pf, pb = self.ops.pack_weight(self.w, True, True)
        y = self.ops.fwd_packed(self.x, self.table, self.w, pf, self.b, 0, 1)
        gi, gw, gb = self.ops.bwd_packed(self.go, self.x, self.table, self.w, pb, C, 0, True, symmetric=self.sym)
        return y, gi, gw, gb


def dense_ms(dev, dtype, reps, timer=None):
    """Dense 3x3 conv (MIOpen) fwd + input grad + weight grad + bias grad on the
    full [B*T, C, H, W] grid; best of NCHW and channels_last (timed by timer,
    time_events by default)."""
    import torch
    import torch.nn.functional as F

    torch.backends.cudnn.benchmark = True
    g = torch.Generator().manual_seed(SEED + 2)
    best = None
    for fmt in (torch.contiguous_format, torch.channels_last):
        x = torch.randn(B * T, C, H, W, generator=g).to(dev, dtype).contiguous(memory_format=fmt)
        x.requires_grad_(True)
        w = (torch.randn(C, C, 3, 3, generator=g) * 0.02).to(dev, dtype).contiguous(memory_format=fmt)
        w.requires_grad_(True)
        b = torch.zeros(C, device=dev, dtype=dtype, requires_grad=True)
        dy = torch.randn(B * T, C, H, W, generator=g).to(dev, dtype).contiguous(memory_format=fmt)

        def run():
            y = F.conv2d(x, w, b, padding=1)
            gx, gw, gb = torch.autograd.grad(y, (x, w, b), dy)
            return gx

        t = (timer or time_events)(run, reps, warm=5)
        best = min((v for v in (best, t) if v is not None), default=None)
    return best


def dense_adapter_ms(prob, dev, dtype, reps):
    """The reference adapter's dense ``2d_conv`` branch on the same kept tokens
    (vit_sparse_adapter_poguise.py:372-412,484-490: scatter into the zero grid,
    NCHW conv2d, gather), forward + input / weight / bias gradients: the
    speedup denominator as the paper's model would run it."""
    import torch

    import eccv26_tad_amd as sv

    torch.backends.cudnn.benchmark = True
    n_kept = prob.n // B
    idx = torch.nonzero(prob.mask.view(B, -1))[:, 1].view(B, n_kept)
    x = prob.x.view(B, n_kept, C).detach().clone().requires_grad_(True)
    go = prob.go.view(B, n_kept, C)
    conv = torch.nn.Conv2d(C, C, 3, padding=1).to(dev, dtype)

    def run():
        y = sv.dense_conv_tokens(x, idx, T * H * W, H, W, conv)
        return torch.autograd.grad(y, (x, conv.weight, conv.bias), go)

    return time_events(run, reps, warm=5)


def adapter_measure(dev, reps, amp=False, use_attn=0):
    """SparseConvAdapter (fused GEMM epilogues, no host sync) against the
    unfused chain of the reference adapter (vit_sparse_adapter_poguise.py:
    305-362,511-653, with the .max() heuristic) at the ViT-B adapter shape:
    B2 x (1 CLS + kept tokens of T80 x 14x14 at 55 % keep) x 768, hidden 256
    (the reference rounds 768 / 4 up to a power of two). Forward alone and
    forward + backward (input and all parameter gradients). Precision: a
    float16 module and input, or with ``amp`` the reference's training mode,
    float32 parameters and input under torch.autocast(bfloat16)
    (opentad/cores/train_engine.py:672), where both paths cast to bfloat16
    and return float32. ``use_attn`` 2 is the vitsparse configs' variant
    (visual tokens attend to the key tokens; one key token here)."""
    import contextlib

    import torch

    import eccv26_tad_amd as sv

    dtype = torch.float32 if amp else torch.float16
    mask = make_mask(0.55).to(dev)
    table = sv.build_neighbor_table(mask)
    n_kept = table.shape[0] // B
    table = table.view(B, n_kept, 9)
    idx = torch.nonzero(mask.view(B, -1))[:, 1].view(B, n_kept)
    g = torch.Generator().manual_seed(SEED + 5)
    mod = sv.SparseConvAdapter(768, 0.25, use_attn=use_attn, n_key_tokens=1)
    with torch.no_grad():
        mod.up_proj.weight.copy_(torch.randn(mod.up_proj.weight.shape, generator=g) * 0.02)
    mod = mod.to(dev, dtype)
    x = torch.randn(B, 1 + n_kept, 768, generator=g).to(dev, dtype).requires_grad_(True)
    go = torch.randn(B, 1 + n_kept, 768, generator=g).to(dev, dtype)
    params = [x] + list(mod.parameters())
    args = (H, W, idx, T * H * W, table)
    ctx = (lambda: torch.autocast("cuda", dtype=torch.bfloat16)) if amp else contextlib.nullcontext
    with ctx():
        if mod._fused_dtype(x) is None:
            raise RuntimeError("adapter bench: the fused path would not run")

    def fwd_fused():
        with torch.no_grad(), ctx():
            return mod(x, *args)

    def fwd_unfused():
        with torch.no_grad(), ctx():
            return mod.reference_forward(x, *args)

    def step_fused():
        with ctx():
            y = mod(x, *args)
        return torch.autograd.grad(y, params, go)

    def step_unfused():
        with ctx():
            y = mod.reference_forward(x, *args)
        return torch.autograd.grad(y, params, go)

    t = {name: time_events(fn, reps, warm=5) for name, fn in
         (("fwd", fwd_fused), ("fwd_unfused", fwd_unfused), ("step", step_fused), ("step_unfused", step_unfused))}
    prec = "fp32 params and input under autocast(bf16)" if amp else "fp16"
    out = {"workload": f"x [{B}, 1+{n_kept}, 768] {prec}, hidden {mod.hidden_dims}, use_attn {use_attn}, "
                       f"keep 0.55"}
    for k, v in t.items():
        out[k + "_us"] = round(v * 1e3, 2)
    out["fwd_speedup"] = round(t["fwd_unfused"] / t["fwd"], 3)
    out["step_speedup"] = round(t["step_unfused"] / t["step"], 3)
    return out


def adapter_rows(dev, reps):
    """The adapter rows of the bench: a float16 module, and the reference's
    training mode (float32 parameters under autocast(bfloat16)), both
    without attention. (With use_attn 2 and one key token both paths spend
    about 2 x 11 ms of host time per step before two of PyTorch's bfloat16
    batched products of the attention branch, which hides the adapter.)"""
    return {"fp16": adapter_measure(dev, reps),
            "autocast_bf16": adapter_measure(dev, reps, amp=True)}


def blob_mask(keep: float, seed: int = SEED + 1):
    """[B, T, H, W] uint8 clustered keep mask (benchmark config 3): per frame a
    score that is the sum of two isotropic 2D Gaussian blobs (sigma 2.5 cells,
    centres drifting by a seeded random walk over the frames) plus 1e-3 U(0,1)
    noise; per sample the top-k (k = ceil(keep * T*H*W)) of the score."""
    import torch

    g = torch.Generator().manual_seed(seed)
    ys = torch.arange(H).float().view(H, 1)
    xs = torch.arange(W).float().view(1, W)
    n = T * H * W
    k = math.ceil(keep * n)
    m = torch.zeros(B, n, dtype=torch.uint8)
    for b in range(B):
        c = torch.rand(2, 2, generator=g) * torch.tensor([H - 1.0, W - 1.0])
        frames = []
        for _ in range(T):
            c = (c + torch.randn(2, 2, generator=g) * 0.7).clamp(min=0.0)
            c[:, 0] = c[:, 0].clamp(max=H - 1.0)
            c[:, 1] = c[:, 1].clamp(max=W - 1.0)
            sc = sum(torch.exp(-((ys - c[j, 0]) ** 2 + (xs - c[j, 1]) ** 2) / (2 * 2.5 ** 2)) for j in range(2))
            frames.append(sc + 1e-3 * torch.rand(H, W, generator=g))
        score = torch.stack(frames).view(-1)
        m[b, torch.topk(score, k).indices] = 1
    return m.view(B, T, H, W)


def depthwise_measure(dev, reps, keeps=None):
    """benchmark config 3: depthwise (groups = C = 192) 3x3 SparseConv2D, fp16,
    B2 x T80 x 14x14, clustered keep masks, fwd + bwd_in + bwd_w with bias (the
    autograd step of SparseDepthwiseConv2d: the forward, then the one-pass
    backward), at every keep rate; the separate backward passes are timed
    too (pass_us). Algorithmic
    bytes per step: the three passes each read their activation rows and the
    table once and write their output once, plus weights."""
    import torch

    import eccv26_tad_amd as sv

    ops = sv.ops
    import torch.nn.functional as F

    # dense comparator: grouped (depthwise) MIOpen conv2d fwd + input / weight
    # / bias gradients on the full grid, best of NCHW and channels_last
    torch.backends.cudnn.benchmark = True
    gd = torch.Generator().manual_seed(SEED + 4)
    dense = dense_q = None
    for fmt in (torch.contiguous_format, torch.channels_last):
        xd = torch.randn(B * T, C, H, W, generator=gd).to(dev, torch.float16).contiguous(memory_format=fmt)
        xd.requires_grad_(True)
        wd = (torch.randn(C, 1, 3, 3, generator=gd) * 0.3).to(dev, torch.float16).requires_grad_(True)
        bd = torch.zeros(C, device=dev, dtype=torch.float16, requires_grad=True)
        dy = torch.randn(B * T, C, H, W, generator=gd).to(dev, torch.float16).contiguous(memory_format=fmt)

        def run_dense():
            y = F.conv2d(xd, wd, bd, padding=1, groups=C)
            return torch.autograd.grad(y, (xd, wd, bd), dy)

        td = time_events(run_dense, reps, warm=5)
        dense = td if dense is None else min(dense, td)
        tq = time_queued(run_dense, reps, warm=5)
        dense_q = min((v for v in (dense_q, tq) if v is not None), default=None)
    rows = []
    for kr in keeps or KEEPS:
        mask = blob_mask(kr).to(dev)
        table = sv.build_neighbor_table(mask)
        n = int(table.shape[0])
        g = torch.Generator().manual_seed(SEED + 3)
        x = torch.randn(n, C, generator=g).to(dev, torch.float16)
        w = (torch.rand(9, C, generator=g) * 2 - 1).div(3).to(dev, torch.float16)
        b = (torch.rand(C, generator=g) * 0.2 - 0.1).to(dev, torch.float16)
        go = torch.randn(n, C, generator=g).to(dev, torch.float16)
        hit = float((table >= 0).sum()) / (9 * n)
        sym = sv.is_symmetric_table(table)

        def step():  # the calls SparseDepthwiseConv2d's autograd makes
            y = ops.dw_fwd(x, table, w, b, 0)
            gi, gw, gb = ops.dw_bwd(go, x, table, w, 0, True, symmetric=sym)
            return y, gi, gw, gb

        t = time_events(step, reps)
        tq = time_queued(step, reps)
        parts = {"fwd": lambda: ops.dw_fwd(x, table, w, b, 0),
                 "bwd": lambda: ops.dw_bwd(go, x, table, w, 0, True, symmetric=sym),
                 "bwd_checked": lambda: ops.dw_bwd(go, x, table, w, 0, True),
                 "bwd_in": lambda: ops.dw_bwd_in(go, table, w, 0, symmetric=sym),
                 "bwd_w": lambda: ops.dw_bwd_w(go, x, table, 0, True)}
        pt = {k2: round(time_events(f, reps) * 1e3, 2) for k2, f in parts.items()}
        # fwd: x, y, table; bwd_in: go, gi, table; bwd_w: go, x, table; weights and bias
        by = 3 * (2 * n * C * 2 + 36 * n) + 3 * 9 * C * 2 + 3 * C * 2
        rows.append({"keep": kr, "n": n, "hit_rate": round(hit, 4), "us": round(t * 1e3, 2),
                     "gbs": round(by / (t * 1e-3) / 1e9, 1),
                     "hbm_frac": round(by / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "pass_us": pt,
                     "speedup_vs_dense": round(dense / t, 3),
                     "gpu_us": round(tq * 1e3, 2) if tq else None,
                     "speedup_vs_dense_gpu": round(dense_q / tq, 3) if tq and dense_q else None})
        log(f"bench: depthwise {rows[-1]}")
    return {"workload": f"depthwise 3x3, C={C} fp16, B{B} x T{T} x {H}x{W}, clustered (Gaussian-blob) keep masks",
            "dense_us": round(dense * 1e3, 2), "dense_gpu_us": round(dense_q * 1e3, 2) if dense_q else None,
            "sweep": rows}


def large_channel_measure(dev, reps, cases=None):
    """Benchmark configs 4 and 5, the matrix-core path at large widths: the same
    autograd step as config 2 (weight pack, forward with fp32 bias, combined
    backward). Config 4: ViT-L adapter, C = 256 bf16, B2 x T96 x 16x16, top-k
    keeps 10 / 25 / 55 %. Config 5: C = 512 bf16, B4 x T128 x 16x16, ragged
    per-frame keeps ~ U(5 %, 15 %) (global table). Reported per case: the
    table's hit rate E / 9N, step µs, and TFLOP/s as a fraction of the bf16
    MFMA peak on two bases: dense-K (three GEMM passes of 2 * 9 * N * C^2,
    the products the implicit GEMM issues, zero rows of missing neighbors
    included) and useful (2 * E * C^2 per pass, E = valid table entries);
    and the forward and backward-input gathered GEMMs timed alone."""
    import torch

    import eccv26_tad_amd as sv

    ops = sv.ops
    out = []

    def case(name, mask, c):
        table = sv.build_neighbor_table(mask)
        n = int(table.shape[0])
        g = torch.Generator().manual_seed(SEED + 7)
        bound = 1.0 / math.sqrt(9 * c)
        x = torch.randn(n, c, generator=g).to(dev, torch.bfloat16)
        w = ((torch.rand(9, c, c, generator=g) * 2 - 1) * bound).to(dev, torch.bfloat16)
        b = ((torch.rand(c, generator=g) * 2 - 1) * bound).to(dev, torch.bfloat16)
        go = torch.randn(n, c, generator=g).to(dev, torch.bfloat16)
        sym = sv.is_symmetric_table(table)

        def step():
            pf, pb = ops.pack_weight(w, True, True)
            y = ops.fwd_packed(x, table, w, pf, b, 0, 1)
            return y, ops.bwd_packed(go, x, table, w, pb, c, 0, True, symmetric=sym)

        t = time_events(step, reps)
        f = 3 * 2 * 9 * n * c * c
        e = int((table >= 0).sum())  # valid (row, offset) entries
        fu = 3 * 2 * e * c * c
        pf, pb = ops.pack_weight(w, True, True)
        t_fwd = time_events(lambda: ops.fwd_packed(x, table, w, pf, b, 0, 1), max(reps, 20))
        t_bin = time_events(lambda: ops.bwd_in_gemm(go, table, pb, c, 0, symmetric=sym), max(reps, 20))
        row = {"config": name, "channels": c, "n": n, "hit_rate": round(e / (9 * n), 4), "us": round(t * 1e3, 2),
               "tflops_9n": round(f / (t * 1e-3) / 1e12, 1),
               "mfma_frac": round(f / (t * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS["bf16"], 4),
               "tflops_useful": round(fu / (t * 1e-3) / 1e12, 1),
               "mfma_frac_useful": round(fu / (t * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS["bf16"], 4),
               "fwd_us": round(t_fwd * 1e3, 2), "bwd_in_gemm_us": round(t_bin * 1e3, 2),
               "fwd_mfma_frac_useful": round(2 * e * c * c / (t_fwd * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS["bf16"], 4),
               "fwd_mfma_frac_9n": round(2 * 9 * n * c * c / (t_fwd * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS["bf16"], 4)}
        out.append(row)
        log(f"bench: large-channel {row}")

    for kr in (0.10, 0.25, 0.55):
        if cases and f"c4_{int(round(kr * 100)):02d}" not in cases:
            continue
        gm = torch.Generator().manual_seed(SEED + 2)
        nc = 96 * 16 * 16
        k = math.ceil(kr * nc)
        m = torch.zeros(2, nc, dtype=torch.uint8)
        m.scatter_(1, torch.topk(torch.rand(2, nc, generator=gm), k, dim=1).indices, 1)
        case(f"c4 keep {kr}", m.view(2, 96, 16, 16).to(dev), 256)
    if cases and "c5" not in cases:
        return out
    gm = torch.Generator().manual_seed(SEED + 3)
    m = torch.zeros(4 * 128, 256, dtype=torch.uint8)
    for f in range(4 * 128):
        kf = int(round(float(torch.empty(1).uniform_(0.05, 0.15, generator=gm)) * 256))
        m[f, torch.randperm(256, generator=gm)[:kf]] = 1
    case("c5 ragged 5-15 %", m.view(4, 128, 16, 16).to(dev), 512)
    return out


PRUNE_C = 768  # ViT-B token width, where the Block prune step runs


def prune_bytes(b, n_key, n_prev, n_new, row_bytes):
    """Algorithmic HBM bytes of one prune step (vit_sparse_adapter_poguise.py
    :899-977): kept and key rows read and written once; keep_idx and last_idx
    read and the new idx written (8 B each); the kept table rows read and
    the new table written (36 B each); the old -> new mapping filled, scattered
    and read once per table entry (4 B each)."""
    rows = b * (n_key + n_new)
    return (2 * rows * row_bytes + b * n_new * (8 + 8 + 8) + b * n_new * 36 * 2
            + b * n_prev * 4 + b * n_new * 4 + b * n_new * 9 * 4)


def prune_measure(dev, reps, cpu: bool):
    """The fused prune step on config 2's ViT-B tokens: x [B, 1 + T*H*W, 768]
    fp16, keep 0.55 of the patch tokens (sorted top-k), with the index
    bookkeeping and the table remap. Timed with HIP events; the oracle's numpy
    restatement of the reference step is timed on the host beside it."""
    import numpy as np
    import torch

    import eccv26_tad_amd as sv

    n = T * H * W
    g = torch.Generator().manual_seed(SEED + 7)
    k = math.ceil(0.55 * n)
    idx = torch.topk(torch.rand(B, n, generator=g), k, dim=1).indices.sort(dim=1).values
    x = torch.randn(B, 1 + n, PRUNE_C, generator=g).to(dev, torch.float16)
    last = torch.arange(n, dtype=torch.long).repeat(B, 1).to(dev)
    table = sv.get_initial_neighbor_indices(H, W, T, dev, B)
    idx_d = idx.to(dev)
    ms = time_events(lambda: sv.prune_tokens(x, idx_d, last, table, 1), reps)
    by = prune_bytes(B, 1, n, k, PRUNE_C * 2)
    out = {"workload": f"x [{B}, 1+{n}, {PRUNE_C}] fp16, keep 0.55, idx + table", "us": round(ms * 1e3, 2),
           "gbs": round(by / (ms * 1e-3) / 1e9, 1), "hbm_frac": round(by / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
           "bytes": by, "launches": 3}
    if cpu:
        from oracle import sv_oracle

        xs, ids, ls, ts = x.cpu().numpy(), idx.numpy(), last.cpu().numpy(), table.cpu().numpy()
        t0 = time.perf_counter()
        reps_c = 0
        while True:
            sv_oracle.ref_prune_step(xs, ids, ls, ts, 1)
            reps_c += 1
            if time.perf_counter() - t0 > 2.0 or reps_c >= 20:
                break
        out["cpu_reference_us"] = round((time.perf_counter() - t0) / reps_c * 1e6, 1)
        out["cpu_reference"] = "numpy restatement of the reference step (oracle.ref_prune_step), 1 thread"
    return out


def cpu_baseline(budget_s: float):
    """The OpenMP fp32 port of the reference dataflow (oracle/sv_oracle.c,
    svo_fwd_f32 / svo_bwd_in_f32 / svo_bwd_w_f32) on the host cores, on the
    same workload at the headline keep rate, repeated until about budget_s."""
    import numpy as np

    from oracle import sv_oracle

    sv_oracle.lib()
    keep = 0.55
    mask = make_mask(keep).numpy()
    table = sv_oracle.build_table(mask)
    n = table.shape[0]
    rng = np.random.default_rng(SEED)
    x = rng.standard_normal((n, C), dtype=np.float32)
    w = (rng.random((9, C, C), dtype=np.float32) * 2 - 1) / math.sqrt(9 * C)
    b = (rng.random(C, dtype=np.float32) * 2 - 1) / math.sqrt(9 * C)
    go = rng.standard_normal((n, C), dtype=np.float32)
    port = sv_oracle.Fp32Port(n, C, C)
    steps, t0 = 0, time.perf_counter()
    while True:
        port.fwd(x, table, w, b)
        port.bwd(go, x, table, w)
        steps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or steps >= 50:
            break
    per = el / steps
    by = sum(op_bytes(n, C, C, 4).values())
    cpu = "unknown"
    phys = set()
    try:
        with open("/proc/cpuinfo") as f:
            pid = None
            for line in f:
                if line.startswith("model name") and cpu == "unknown":
                    cpu = line.split(":", 1)[1].strip()
                elif line.startswith("physical id"):
                    pid = line.split(":", 1)[1].strip()
                elif line.startswith("core id"):
                    phys.add((pid, line.split(":", 1)[1].strip()))
    except OSError:
        pass
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    # the fp64 torch oracle of the test suite (dense conv2d on the zero-filled
    # grid and its autograd) on the same workload, torch's CPU threads
    import torch

    from tests.helpers import dense_reference

    t1 = time.perf_counter()
    dense_reference(mask, x, w, b, go)
    fp64_s = time.perf_counter() - t1
    return {
        "value": round(by / per / 1e9, 3), "unit": "GB/s",
        "cores": sv_oracle.num_threads(), "kind": "port",
        "sample": (f"fp32 fwd+bwd of the same config-2 workload at keep {keep} (N={n}), "
                   f"{steps} step(s) in {el:.1f} s, {per * 1e3:.1f} ms/step; "
                   f"host {cpu} ({platform.machine()})"),
        "ms_per_step": round(per * 1e3, 3),
        "host": {"cpu": cpu, "logical_cpus_available": avail, "logical_cpus": os.cpu_count(),
                 "physical_cores": len(phys) or None, "omp_threads": sv_oracle.num_threads()},
        "torch_fp64_oracle": {"ms_per_step": round(fp64_s * 1e3, 1), "threads": torch.get_num_threads(),
                              "what": "dense float64 conv2d on the zero-filled grid + autograd (tests/helpers.py)"},
    }


def replay_measure(dev, dtype, keep, steps, graph):
    """The headline step (pack, forward, combined backward) at ``keep``,
    eager or as replays of one HIP-graph capture of it, timed over ``steps``
    between one pair of events. Run alone under a kernel trace, each mode
    shows where its time goes: the kernels' durations, and the gaps between
    them and between replays."""
    import torch

    p = Problem(keep, dev, dtype)
    for _ in range(5):
        p.step()
    torch.cuda.synchronize()
    fn = p.step
    if graph:
        st = torch.cuda.Stream()
        st.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(st):
            for _ in range(3):
                p.step()
        torch.cuda.current_stream().wait_stream(st)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            p.step()
        fn = g.replay
    for _ in range(10):
        fn()
    torch.cuda.synchronize()
    return {"mode": "graph" if graph else "eager", "keep": keep, "n": p.n, "steps": steps,
            "us_per_step": round(time_events(fn, steps) * 1e3, 2)}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--keep", type=float, default=0.55, help="headline keep rate")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-dense", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (scales rocprofv3 FETCH_SIZE / "
                         "WRITE_SIZE counters) and exit")
    ap.add_argument("--one-keep", action="store_true",
                    help="with --only depthwise: time the --keep rate alone (for counter runs)")
    ap.add_argument("--large-cases", default=None,
                    help="with --only large: comma-separated subset of c4_10,c4_25,c4_55,c5")
    ap.add_argument("--only", choices=("adapter", "prune", "depthwise", "large", "replay"), default=None,
                    help="only time the fused adapter, the prune step, ... print its JSON and exit "
                         "(for kernel traces of those paths); replay: the headline step at --keep, "
                         "eager or (--graph) as HIP-graph replays")
    ap.add_argument("--graph", action="store_true", help="with --only replay: time HIP-graph replays")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only; the SparseConv2D path has no "
              "collective (multi-GPU sharding is described, not run). Use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    dtype, dname, s = torch.float16, "f16", 2
    if args.copy_calibration:
        nbytes = args.copy_calibration << 20
        src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": nbytes, "launches": 5}), flush=True)
        return
    if args.only == "adapter":
        print(json.dumps({"adapter": adapter_rows(dev, args.steps)}), flush=True)
        return
    if args.only == "prune":
        print(json.dumps({"prune_step": prune_measure(dev, args.steps, False)}), flush=True)
        return
    if args.only == "depthwise":
        keeps = [args.keep] if args.one_keep else KEEPS
        print(json.dumps({"depthwise": depthwise_measure(dev, args.steps, keeps)}), flush=True)
        return
    if args.only == "large":
        cases = set(args.large_cases.split(",")) if args.large_cases else None
        print(json.dumps({"large_channel": large_channel_measure(dev, args.steps, cases)}), flush=True)
        return
    if args.only == "replay":
        print(json.dumps({"replay": replay_measure(dev, dtype, args.keep, args.steps, args.graph)}), flush=True)
        return

    log(f"bench: building problem keep={args.keep}")
    prob = Problem(args.keep, dev, dtype)
    n = prob.n
    by = op_bytes(n, C, C, s)
    total_bytes = sum(by.values())
    flops_9n = 3 * 2 * 9 * n * C * C
    flops_useful = 3 * 2 * prob.valid * C * C

    # table build (mask already resident): one launch with the kept count the
    # caller knows (no host sync), and the full-grid table of the backbone's
    # first block (closed form, one launch)
    import eccv26_tad_amd as sv

    table_ms = time_events(lambda: sv.build_neighbor_table(prob.mask, n=n), 50)
    grid_ms = time_events(lambda: sv.get_initial_neighbor_indices(H, W, T, dev, B), 50)
    # the launch floor: an empty kernel (torch.cuda._sleep(0), one workgroup)
    # launched back to back, the least any launch of the step costs
    floor_ms = time_events(lambda: torch.cuda._sleep(0), 200)
    if not torch.equal(sv.build_neighbor_table(prob.mask, n=n), prob.table):
        raise RuntimeError("one-launch table differs from the scan + fill table")

    # timed fwd+bwd steps
    log(f"bench: N={n}, warmup {args.warmup}, steps {args.steps}")
    for _ in range(args.warmup):
        prob.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    # the K steps back to back between one pair of events: ms_per_step
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(args.steps):
        prob.step()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / args.steps
    # the per-step spread from a second pass with an event after every step
    # (each event record between steps adds to the step it follows, so this
    # pass is not the timed one)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    evs[0].record()
    for i in range(args.steps):
        prob.step()
        evs[i + 1].record()
    torch.cuda.synchronize()
    per_step = sorted(evs[i].elapsed_time(evs[i + 1]) for i in range(args.steps))
    med_ms = per_step[len(per_step) // 2]
    log(f"bench: {ms * 1e3:.1f} us/step mean, {med_ms * 1e3:.1f} median (wall {wall / args.steps * 1e3:.1f} us/step)")

    # HIP graph replay of the same step
    graph_ms = None
    try:
        st = torch.cuda.Stream()
        st.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(st):
            for _ in range(3):
                ref = prob.step()
        torch.cuda.current_stream().wait_stream(st)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            outs = prob.step()
        for _ in range(3):
            gr.replay()
            torch.cuda.synchronize()
            eager = prob.step()
            torch.cuda.synchronize()
            for a, b in zip(outs, eager):
                if not torch.equal(a, b):
                    raise RuntimeError("graph replay differs from eager")
        graph_ms = time_events(gr.replay, args.steps)
        del gr
    except Exception as exc:  # reported, not fatal
        log(f"bench: graph replay skipped: {exc}")

    # per-pass timing (back-to-back calls). fwd is one kernel (gathered
    # GEMM); bwd_in adds the orphan-pass launch to its GEMM (bwd_in_gemm);
    # bwd_w is the partial-sum kernel (bwd_w_partials) plus the split
    # reduction; bwd is the step's backward (bwd_in + bwd_w in one call, the
    # orphan pass inside the reduction); the *_checked passes are the same
    # calls without the table's symmetric record (partner checks on).
    phases = {p: time_events(getattr(prob, p), max(args.steps, 20))
              for p in ("pack", "fwd", "bwd_in", "bwd_in_gemm", "bwd_w", "bwd_w_partials", "bwd", "bwd_checked",
                        "bwd_in_gemm_checked")}
    # The roofline names the longest single kernel of the step among the
    # three GEMM-shaped kernels: its duration is the mean over back-to-back
    # launches between one pair of HIP events (what a kernel trace's
    # average duration measures); each launch bracketed by its own events
    # (dispatch latency included) is reported beside it.
    kernels = {p: phases[p] for p in ("fwd", "bwd_in_gemm", "bwd_w_partials")}
    isolated = {p: time_kernel(getattr(prob, p), max(args.steps, 50)) for p in kernels}
    dom = max(kernels, key=kernels.get)
    # algorithmic flops of one GEMM pass: the valid (row, offset) entries E
    # of the table times 2 * C_in * C_out (the dense-K count 9 * N, which
    # includes the products with missing neighbors' zero rows, is reported
    # beside it)
    f_pass = 2 * prob.valid * C * C
    f_pass_9n = 2 * 9 * n * C * C
    t_dom = kernels[dom] * 1e-3
    by_dom = by[{"fwd": "fwd", "bwd_in_gemm": "bwd_in", "bwd_w_partials": "bwd_w"}[dom]]
    mfma_t = f_pass / (MFMA_PEAK_TFLOPS[dname] * 1e12)
    hbm_t = by_dom / (HBM_PEAK_GBS * 1e9)
    if mfma_t >= hbm_t:
        roof = {"bound": "mfma", "achieved": round(f_pass / t_dom / 1e12, 3),
                "peak": MFMA_PEAK_TFLOPS[dname], "unit": "TFLOP/s"}
    else:
        roof = {"bound": "hbm", "achieved": round(by_dom / t_dom / 1e9, 3),
                "peak": HBM_PEAK_GBS, "unit": "GB/s"}
    roof["frac"] = round(roof["achieved"] / roof["peak"], 5)
    if roof["unit"] == "TFLOP/s":
        roof["basis"] = "useful flops 2*E*C^2 per launch, E = valid table entries"
        roof["achieved_9n"] = round(f_pass_9n / t_dom / 1e12, 3)
        roof["frac_9n"] = round(roof["achieved_9n"] / roof["peak"], 5)
    key = {"fwd": "k_gg_wideIDF16_Li0", "bwd_in_gemm": "k_gg_wideIDF16_Li1", "bwd_w_partials": "k_bw_big"}[dom]
    roof["traffic"] = pmc_traffic(key) if abs(args.keep - 0.55) < 1e-9 else None
    if roof["traffic"] is not None:
        roof["traffic_source"] = TRAFFIC_PROFILE
        roof["traffic_algorithmic"] = int(by_dom)
    roof["kernel"] = {"fwd": "k_gg_wide MODE 0 (forward gathered GEMM)",
                      "bwd_in_gemm": "k_gg_wide MODE 1 (backward-input gathered GEMM)",
                      "bwd_w_partials": "k_bw_big (backward-weight partial sums)"}[dom]
    roof["kernel_us"] = round(kernels[dom] * 1e3, 2)
    roof["kernel_us_all"] = {p: {"back_to_back": round(v * 1e3, 2),
                                 "isolated_median": round(isolated[p][0] * 1e3, 2)} for p, v in kernels.items()}

    dense = None if args.no_dense else dense_ms(dev, dtype, 20)
    dense_q = None if args.no_dense else dense_ms(dev, dtype, 20, timer=time_queued)

    sweep = []
    if not args.no_sweep:
        for kr in KEEPS:
            p = prob if abs(kr - args.keep) < 1e-9 else Problem(kr, dev, dtype)
            t = time_events(p.step, 20)
            tq = time_queued(p.step, 20)
            b2 = sum(op_bytes(p.n, C, C, s).values())
            f9 = 3 * 2 * 9 * p.n * C * C
            fu = 3 * 2 * p.valid * C * C
            row = {"keep": kr, "n": p.n, "hit_rate": round(p.valid / (9 * p.n), 4),
                   "us": round(t * 1e3, 2), "gbs": round(b2 / (t * 1e-3) / 1e9, 1),
                   "tflops_9n": round(f9 / (t * 1e-3) / 1e12, 2),
                   "roofline_frac": round(max(b2 / (HBM_PEAK_GBS * 1e9),
                                              fu / (MFMA_PEAK_TFLOPS[dname] * 1e12)) / (t * 1e-3), 4)}
            row["gpu_us"] = round(tq * 1e3, 2) if tq else None
            if dense is not None:
                row["speedup_vs_dense"] = round(dense / t, 3)
                row["speedup_vs_dense_gpu"] = round(dense_q / tq, 3) if tq and dense_q else None
                da = dense_adapter_ms(p, dev, dtype, 20)
                row["dense_adapter_us"] = round(da * 1e3, 2)
                row["speedup_vs_dense_adapter"] = round(da / t, 3)
            sweep.append(row)
            if p is not prob:
                del p
            log(f"bench: sweep {row}")

    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
    prune = None if args.no_sweep else prune_measure(dev, 20, not args.no_cpu)
    adapter = None if args.no_sweep else adapter_rows(dev, 20)
    depthwise = None if args.no_sweep else depthwise_measure(dev, 20)
    large = None if args.no_sweep else large_channel_measure(dev, 30)  # 30 steps: single runs of 10 moved by ~5 %
    if adapter is not None:
        log(f"bench: adapter {adapter}")

    out = {
        "metric": "SparseConv2D fwd+bwd µs & HBM GB/s (% roofline), speedup vs dense @10-55% keep",
        "value": round(total_bytes / (ms * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "us_per_step": round(ms * 1e3, 2),
        "median_us_per_step": round(med_ms * 1e3, 2),
        "median_note": "second pass with an event recorded after every step (the records add to the steps)",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dname,
        "data": "synthetic (seeded top-k keep masks, N(0,1) activations, uniform weights)",
        "config": {"workload": "SparseConv2D fwd+bwd, ViT-B adapter bottleneck (benchmark config 2)",
                   "grid": f"B{B} x T{T} x {H}x{W}", "channels": C, "keep": args.keep, "n_kept": n,
                   "hit_rate": round(prob.valid / (9 * n), 4), "bias": True},
        "hbm_frac": round(total_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "tflops_9n": round(flops_9n / (ms * 1e-3) / 1e12, 3),
        "tflops_useful": round(flops_useful / (ms * 1e-3) / 1e12, 3),
        "roofline_frac": round(max(total_bytes / (HBM_PEAK_GBS * 1e9),
                                   flops_useful / (MFMA_PEAK_TFLOPS[dname] * 1e12)) / (ms * 1e-3), 4),
        "graph_us_per_step": round(graph_ms * 1e3, 2) if graph_ms else None,
        "pass_us": {k: round(v * 1e3, 2) for k, v in phases.items()},
        "table_build_us": round(table_ms * 1e3, 2),
        "table_build_bytes": int(prob.mask.numel() + 36 * n),
        "table_build_gbs": round((prob.mask.numel() + 36 * n) / (table_ms * 1e-3) / 1e9, 1),
        "grid_table_us": round(grid_ms * 1e3, 2),
        "launch_floor_us": round(floor_ms * 1e3, 2),
        "dense_us": round(dense * 1e3, 2) if dense is not None else None,
        "speedup_vs_dense": round(dense / ms, 3) if dense is not None else None,
        "roofline": roof,
        "cpu_baseline": cpu,
        "sweep": sweep,
        "prune_step": prune,
        "adapter": adapter,
        "depthwise": depthwise,
        "large_channel": large,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
