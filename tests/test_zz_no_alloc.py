"""svtad_fwd_noalloc (the forward with its packed-weight workspace in the
library's static device array) against svtad_fwd with a caller workspace,
through the C ABI: bit-identical outputs on two calls in a row, the second
one smaller, and the host-side rejection of a weight too large for the
array."""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from tests.helpers import kaiming_weight, topk_mask

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "eccv26_tad_amd", "libsvtad_sparse.so")
I64 = ctypes.c_int64
F16, BF16 = 1, 2
BIAS_FP32 = 1


def _lib():
    lib = ctypes.CDLL(LIB)
    lib.svtad_last_error.restype = ctypes.c_char_p
    lib.svtad_fwd_workspace_bytes.restype = ctypes.c_size_t
    lib.svtad_fwd_noalloc_max_workspace_bytes.restype = ctypes.c_size_t
    return lib


def _case(dev, seed, keep, B, T, H, W, c, dt):
    import torch

    import eccv26_tad_amd as sv

    rng = np.random.default_rng(seed)
    mask = topk_mask(rng, B, T, H, W, keep)
    table = sv.build_neighbor_table(torch.from_numpy(mask).to(dev))
    n = table.shape[0]
    x = torch.from_numpy(rng.standard_normal((n, c)).astype(np.float32)).to(dev, dt)
    w = torch.from_numpy(kaiming_weight(rng, c, c)).to(dev, dt)
    b = torch.from_numpy((rng.random(c).astype(np.float32) - 0.5) * 0.2).to(dev)
    return table, x, w, b


def _run_both(lib, dev, table, x, w, b, code):
    import torch

    n, c = x.shape
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    out_na = torch.full((n, c), float("nan"), device=dev, dtype=x.dtype)
    st = lib.svtad_fwd_noalloc(ptr(x), ptr(table), ptr(w), ptr(b), BIAS_FP32, ptr(out_na), I64(n), c, c, I64(0),
                               code, stream)
    assert st == 0, lib.svtad_last_error()
    wsb = lib.svtad_fwd_workspace_bytes(c, c, code)
    assert 0 < wsb <= lib.svtad_fwd_noalloc_max_workspace_bytes()
    ws = torch.empty(wsb, device=dev, dtype=torch.uint8)
    out = torch.full((n, c), float("nan"), device=dev, dtype=x.dtype)
    st = lib.svtad_fwd(ptr(x), ptr(table), ptr(w), ptr(b), BIAS_FP32, ptr(out), ptr(ws), ctypes.c_size_t(wsb),
                       I64(n), c, c, I64(0), code, stream)
    assert st == 0, lib.svtad_last_error()
    torch.cuda.synchronize()
    return out_na, out


def test_fwd_noalloc_matches_fwd(dev):
    import torch

    lib = _lib()
    # call 1: config 2 at 55 % keep (C = 192 fp16, N = 17248)
    print("fwd_noalloc: c2, C=192 fp16", flush=True)
    table, x, w, b = _case(dev, 7001, 0.55, 2, 80, 14, 14, 192, torch.float16)
    a, ref = _run_both(lib, dev, table, x, w, b, F16)
    assert not torch.isnan(ref).any()
    assert torch.equal(a, ref)
    # call 2, smaller: C = 64 bf16 on a few frames (the array keeps call 1's
    # packed weight; this call repacks into its front)
    print("fwd_noalloc: C=64 bf16, 6 frames", flush=True)
    table, x, w, b = _case(dev, 7002, 0.4, 1, 6, 14, 14, 64, torch.bfloat16)
    a, ref = _run_both(lib, dev, table, x, w, b, BF16)
    assert not torch.isnan(ref).any()
    assert torch.equal(a, ref)


def test_fwd_noalloc_rejects_weights_beyond_the_array(dev):
    lib = _lib()
    # C_in = 512, C_out = 1024: a 9 MiB packed weight
    assert lib.svtad_fwd_workspace_bytes(512, 1024, F16) > lib.svtad_fwd_noalloc_max_workspace_bytes()
    buf = ctypes.create_string_buffer(64)
    st = lib.svtad_fwd_noalloc(buf, buf, buf, None, 0, buf, I64(16), 512, 1024, I64(0), F16, None)
    assert st == -3 and b"static workspace" in lib.svtad_last_error()


def test_fwd_noalloc_replays_in_a_hip_graph(dev):
    """The allocation-free forward captured in a HIP graph (torch.cuda.graph),
    after one eager call on the device (the first call per device looks up the
    array's device address, which stays outside the capture): three replays,
    with other GPU work and synchronisations between them, each equal to the
    eager svtad_fwd bit for bit."""
    import torch

    lib = _lib()
    print("fwd_noalloc under graph capture: c2 at 25 % keep, C=192 fp16", flush=True)
    table, x, w, b = _case(dev, 7003, 0.25, 2, 80, 14, 14, 192, torch.float16)
    a, ref = _run_both(lib, dev, table, x, w, b, F16)  # the eager call (and the reference)
    assert torch.equal(a, ref)
    n, c = x.shape
    out = torch.full((n, c), float("nan"), device=dev, dtype=x.dtype)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    graph = torch.cuda.CUDAGraph()
    status = []
    with torch.cuda.graph(graph):
        stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        status.append(lib.svtad_fwd_noalloc(ptr(x), ptr(table), ptr(w), ptr(b), BIAS_FP32, ptr(out), I64(n), c, c,
                                            I64(0), F16, stream))
    assert status == [0], lib.svtad_last_error()
    for r in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {r}"
        # other work on the array's device between replays
        junk = torch.randn(512, 512, device=dev) @ torch.randn(512, 512, device=dev)
        torch.cuda.synchronize()
        del junk
