"""CPU checks of the C-ABI library and the extension module (no GPU compute).

* libsvtad_sparse.so loads and exports every function include/svtad_sparse.h
  declares.
* Argument errors are rejected on the host, before any launch, with a message.
* The torch extension exposes the reference's five functions plus the additions.
"""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "eccv26_tad_amd", "libsvtad_sparse.so")
HEADER = os.path.join(ROOT, "include", "svtad_sparse.h")

I64 = ctypes.c_int64
Z = ctypes.c_size_t(0)


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(svtad_\w+)\s*\(", src)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail("libsvtad_sparse.so not built (run python -m eccv26_tad_amd.build)")
    L = ctypes.CDLL(LIB)
    L.svtad_last_error.restype = ctypes.c_char_p
    L.svtad_version.restype = ctypes.c_char_p
    L.svtad_bwd_w_workspace_bytes.restype = ctypes.c_size_t
    L.svtad_dw_bwd_w_workspace_bytes.restype = ctypes.c_size_t
    return L


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), f"{name} declared in svtad_sparse.h but not exported"


def test_version(lib):
    assert b"gfx950" in lib.svtad_version()


def test_bad_dtype_rejected_on_host(lib):
    st = lib.svtad_fwd(None, None, None, None, 0, None, None, Z, I64(10), 8, 8, I64(0), 9, None)
    assert st == -1
    assert b"dtype" in lib.svtad_last_error()


def test_bad_cin_rejected_on_host(lib):
    st = lib.svtad_fwd(None, None, None, None, 0, None, None, Z, I64(10), 6, 8, I64(0), 0, None)
    assert st == -1
    assert b"divisible by 4" in lib.svtad_last_error()


def test_bias_mode_needs_pointer(lib):
    st = lib.svtad_fwd(None, None, None, None, 1, None, None, Z, I64(10), 8, 8, I64(0), 0, None)
    assert st == -1 and b"bias" in lib.svtad_last_error()


def test_negative_sizes_rejected(lib):
    assert lib.svtad_bwd_in(None, None, None, None, None, Z, I64(-1), 8, 8, I64(0), 0, None) == -1
    assert lib.svtad_bwd_in(None, None, None, None, None, Z, I64(4), 8, 8, I64(-3), 0, None) == -1


def test_empty_input_is_a_noop(lib):
    assert lib.svtad_fwd(None, None, None, None, 0, None, None, Z, I64(0), 8, 8, I64(0), 0, None) == 0
    assert lib.svtad_bwd_in(None, None, None, None, None, Z, I64(0), 8, 8, I64(0), 0, None) == 0


def test_workspace_sizes(lib):
    for n, ci, co, dt in [(0, 8, 8, 0), (17248, 192, 192, 1), (13107, 512, 512, 2), (100, 48, 48, 3)]:
        b = lib.svtad_bwd_w_workspace_bytes(I64(n), ci, co, dt)
        acc = 8 if dt == 3 else 4
        assert b >= (9 * ci * co + co) * acc
        # per split: 9 offset partials (10 work units with the large-tile
        # kernel: the center offset in two halves) and two bias partials
        assert b % ((9 * ci * co + 2 * co) * acc) == 0 or b % ((10 * ci * co + 2 * co) * acc) == 0
    assert lib.svtad_dw_bwd_w_workspace_bytes(I64(17248), 192, 1) >= 10 * 192 * 4


def test_fwd_workspace(lib):
    lib.svtad_fwd_workspace_bytes.restype = ctypes.c_size_t
    # f16 / bf16 shapes of the matrix-core forward hold the packed weight
    lib.svtad_bwd_in_workspace_bytes.restype = ctypes.c_size_t
    assert lib.svtad_fwd_workspace_bytes(192, 192, 1) == 9 * 192 * 192 * 2
    # backward-input: the packed weight plus the 256-byte orphan flag block
    assert lib.svtad_bwd_in_workspace_bytes(256, 128, 1) == 9 * 256 * 128 * 2 + 256
    assert lib.svtad_fwd_workspace_bytes(256, 256, 2) == 9 * 256 * 256 * 2
    assert lib.svtad_fwd_workspace_bytes(192, 192, 0) == 0  # f32: VALU kernel, no workspace
    assert lib.svtad_fwd_workspace_bytes(20, 36, 1) == 0
    st = lib.svtad_fwd(None, None, None, None, 0, None, None, Z, I64(10), 192, 192, I64(0), 1, None)
    assert st == -2 and b"workspace" in lib.svtad_last_error()


def test_workspace_too_small_rejected(lib):
    buf = ctypes.create_string_buffer(16)
    st = lib.svtad_bwd_w(None, None, None, buf, None, buf, ctypes.c_size_t(16), I64(0), 8, 8,
                         I64(0), 0, None)
    assert st == -2 and b"workspace" in lib.svtad_last_error()


def test_prune_step_arguments_checked_on_host(lib):
    # last_idx without idx_out, and a table without its mapping workspace
    buf = ctypes.create_string_buffer(64)
    st = lib.svtad_prune_step(buf, I64(1), I64(0), I64(4), I64(16), buf, I64(2), buf, None, None,
                              buf, None, None, None)
    assert st == -1 and b"go together" in lib.svtad_last_error()
    st = lib.svtad_prune_step(buf, I64(1), I64(0), I64(4), I64(16), buf, I64(2), None, buf, None,
                              buf, None, buf, None)
    assert st == -1 and b"go together" in lib.svtad_last_error()
    # nothing kept: the index / table pointers are not needed
    assert lib.svtad_prune_step(None, I64(1), I64(0), I64(4), I64(0), buf, I64(0), buf, None, None,
                                None, None, None, None) == 0
    # more kept than present
    st = lib.svtad_prune_step(buf, I64(1), I64(0), I64(2), I64(16), buf, I64(3), None, None, None,
                              buf, None, None, None)
    assert st == -1 and b"bad sizes" in lib.svtad_last_error()
    # nothing to do
    assert lib.svtad_prune_step(None, I64(0), I64(0), I64(0), I64(16), None, I64(0), None, None,
                                None, None, None, None, None) == 0


def test_adapter_arguments_checked_on_host(lib):
    buf = ctypes.create_string_buffer(256)
    # dtype: the fused adapter GEMMs take f16 / bf16 only
    st = lib.svtad_adapter_down(buf, buf, None, buf, buf, buf, I64(1), I64(4), I64(1), 64, 64, 0, None)
    assert st == -3 and b"f16/bf16" in lib.svtad_last_error()
    # k % 32, n % 64
    st = lib.svtad_adapter_down(buf, buf, None, buf, buf, buf, I64(1), I64(4), I64(1), 48, 64, 1, None)
    assert st == -3
    st = lib.svtad_adapter_up(buf, buf, buf, None, buf, buf, buf, I64(1), I64(4), I64(1), 64, 96, 1, None)
    assert st == -3
    # more special tokens than tokens
    st = lib.svtad_adapter_up(buf, buf, buf, None, buf, buf, buf, I64(1), I64(4), I64(5), 64, 64, 1, None)
    assert st == -1
    # missing gamma / patch output
    st = lib.svtad_adapter_up(buf, buf, buf, None, None, buf, buf, I64(1), I64(4), I64(1), 64, 64, 1, None)
    assert st == -1 and b"null pointer" in lib.svtad_last_error()
    st = lib.svtad_adapter_down(buf, buf, None, buf, buf, None, I64(1), I64(4), I64(1), 64, 64, 2, None)
    assert st == -1 and b"null pointer" in lib.svtad_last_error()
    # nothing to do
    assert lib.svtad_adapter_down(None, None, None, None, None, None, I64(0), I64(4), I64(1), 64, 64, 1,
                                  None) == 0


def test_adapter_backward_arguments_checked_on_host(lib):
    buf = ctypes.create_string_buffer(256)
    # gelu_backward_split: f16/bf16 only, n % 8, n_special <= n_tokens, 2^31 elements
    st = lib.svtad_gelu_backward_split(buf, buf, buf, buf, I64(1), I64(4), I64(1), 64, 0, None)
    assert st == -3 and b"f16/bf16" in lib.svtad_last_error()
    st = lib.svtad_gelu_backward_split(buf, buf, buf, buf, I64(1), I64(4), I64(1), 12, 1, None)
    assert st == -1
    st = lib.svtad_gelu_backward_split(buf, buf, buf, buf, I64(1), I64(4), I64(5), 64, 1, None)
    assert st == -1
    st = lib.svtad_gelu_backward_split(buf, buf, None, buf, I64(1), I64(4), I64(1), 64, 1, None)
    assert st == -1 and b"null pointer" in lib.svtad_last_error()
    st = lib.svtad_gelu_backward_split(buf, buf, buf, buf, I64(1 << 20), I64(1 << 12), I64(1), 1024, 1, None)
    assert st == -3
    assert lib.svtad_gelu_backward_split(None, None, None, None, I64(0), I64(4), I64(1), 64, 1, None) == 0
    # gamma_grad: counts multiples of 8, b and gs together, workspace size
    lib.svtad_gamma_grad_workspace_bytes.restype = ctypes.c_size_t
    wsb = ctypes.c_size_t(lib.svtad_gamma_grad_workspace_bytes())
    assert wsb.value == 256
    N4 = (None, None, None, None)
    st = lib.svtad_gamma_grad(buf, buf, I64(12), None, None, I64(0), buf, *N4, buf, wsb, 1, None)
    assert st == -1
    st = lib.svtad_gamma_grad(buf, buf, I64(16), buf, None, I64(8), buf, *N4, buf, wsb, 1, None)
    assert st == -1 and b"together" in lib.svtad_last_error()
    st = lib.svtad_gamma_grad(buf, buf, I64(16), None, None, I64(0), buf, *N4, buf, wsb, 0, None)
    assert st == -3
    st = lib.svtad_gamma_grad(buf, buf, I64(16), None, None, I64(0), buf, *N4, buf, ctypes.c_size_t(8), 1, None)
    assert st == -2
    # scaled outputs need gamma
    st = lib.svtad_gamma_grad(buf, buf, I64(16), None, None, I64(0), buf, None, buf, None, None, buf, wsb, 1, None)
    assert st == -1 and b"gamma" in lib.svtad_last_error()


def test_heatmap_add_arguments_checked_on_host(lib):
    buf = ctypes.create_string_buffer(256)
    st = lib.svtad_heatmap_add(buf, buf, buf, buf, I64(4), I64(4), 64, 0, None)
    assert st == -3 and b"f16/bf16" in lib.svtad_last_error()
    st = lib.svtad_heatmap_add(buf, buf, buf, buf, I64(4), I64(4), 12, 1, None)
    assert st == -1
    st = lib.svtad_heatmap_add(buf, buf, None, buf, I64(4), I64(4), 64, 2, None)
    assert st == -1 and b"null pointer" in lib.svtad_last_error()
    assert lib.svtad_heatmap_add(None, None, None, None, I64(0), I64(4), 64, 1, None) == 0


def test_adapter_variants_have_the_reference_parameters():
    """Parameter names and shapes of every adapter variant match the reference
    module's (vit_sparse_adapter_poguise.py:93-166), so its state dicts load."""
    from eccv26_tad_amd import SparseConvAdapter

    def shapes(m):
        return {k: tuple(v.shape) for k, v in m.state_dict().items()}

    base = {"down_proj.weight": (256, 768), "down_proj.bias": (256,), "up_proj.weight": (768, 256),
            "up_proj.bias": (768,), "gamma": (1,), "sparse_conv.weight": (9, 256, 256), "sparse_conv.bias": (256,)}
    assert shapes(SparseConvAdapter(768, 0.25)) == base
    assert shapes(SparseConvAdapter(768, 0.25, n_key_tokens=197, heatmap_grid_size=(14, 14))) == {
        **base, "heatmap_gate": (1,)}
    attn = {"attn_norm.weight": (256,), "attn_norm.bias": (256,), "attn_gamma": (1,),
            "down_attn.weight": (128, 256), "down_attn.bias": (128,), "qkv.weight": (384, 128), "qkv.bias": (384,),
            "q_norm.weight": (32,), "q_norm.bias": (32,), "k_norm.weight": (32,), "k_norm.bias": (32,),
            "attn_proj.weight": (256, 128), "attn_proj.bias": (256,)}
    for v in (1, 2, 3):
        m = SparseConvAdapter(768, 0.25, use_attn=v, n_key_tokens=197, heatmap_grid_size=(14, 14))
        assert shapes(m) == {**base, **attn} and m.num_heads == 4
    m = SparseConvAdapter(768, 0.25, use_attn=4)
    t = {"attn_norm.weight": (256,), "attn_norm.bias": (256,), "attn_gamma": (1,), "qkv.weight": (768, 256),
         "attn_proj.weight": (256, 256), "attn_proj.bias": (256,), "attn_mlp.0.weight": (256,),
         "attn_mlp.0.bias": (256,), "attn_mlp.1.weight": (256, 256), "attn_mlp.1.bias": (256,),
         "attn_mlp.3.weight": (256, 256), "attn_mlp.3.bias": (256,)}
    assert shapes(m) == {**base, **t} and m.num_heads == 4
    # the reference's zero-initialised layers and unit gains
    assert float(m.attn_mlp[3].weight.detach().abs().max()) == 0 and float(m.up_proj.weight.detach().abs().max()) == 0
    assert float(m.gamma.detach()) == 1 and float(m.attn_gamma.detach()) == 1
    # hidden width rounds to a power of two (768 * 0.25 -> 256, 384 * 0.25 -> 128, 1024 / 4 -> 256)
    assert SparseConvAdapter(384, 0.25).hidden_dims == 128 and SparseConvAdapter(1024, 0.25).hidden_dims == 256


def test_dw_bwd_arguments_checked_on_host(lib):
    lib.svtad_dw_bwd_workspace_bytes.restype = ctypes.c_size_t
    buf = ctypes.create_string_buffer(256)
    ws = lib.svtad_dw_bwd_workspace_bytes(I64(1000), 64, 1)
    assert ws > lib.svtad_dw_bwd_w_workspace_bytes(I64(1000), 64, 1)  # plus the split flag words
    st = lib.svtad_dw_bwd(buf, buf, buf, buf, buf, buf, None, buf, ctypes.c_size_t(16), I64(1000), 64, I64(0), 1,
                          None)
    assert st == -2 and b"workspace" in lib.svtad_last_error()
    st = lib.svtad_dw_bwd(buf, buf, buf, None, buf, buf, None, buf, ctypes.c_size_t(ws), I64(1000), 64, I64(0), 1,
                          None)
    assert st == -1 and b"null pointer" in lib.svtad_last_error()
    st = lib.svtad_dw_bwd(buf, buf, buf, buf, buf, buf, None, buf, ctypes.c_size_t(ws), I64(1000), 6, I64(0), 1,
                          None)
    assert st != 0


def test_one_launch_table_arguments_checked_on_host(lib):
    buf = ctypes.create_string_buffer(64)
    aligned = ctypes.c_void_p((ctypes.addressof(buf) + 15) & ~15)
    # index width 32 or 64; h*w <= 16384; at most 4 MiB of mask; 16-byte aligned mask
    assert lib.svtad_table_build(aligned, I64(1), 2, 2, I64(4), aligned, 16, None) == -1
    assert lib.svtad_table_build(aligned, I64(1), 200, 200, I64(4), aligned, 32, None) == -3
    st = lib.svtad_table_build(aligned, I64(300), 128, 128, I64(4), aligned, 32, None)
    assert st == -3 and b"4 MiB" in lib.svtad_last_error()
    unaligned = ctypes.c_void_p(aligned.value + 1)
    st = lib.svtad_table_build(unaligned, I64(1), 2, 2, I64(4), aligned, 32, None)
    assert st == -1 and b"aligned" in lib.svtad_last_error()
    assert lib.svtad_table_build(None, I64(1), 2, 2, I64(0), None, 64, None) == 0  # no rows: nothing to do
    assert lib.svtad_table_grid(I64(1), 0, 3, aligned, 32, None) == -1
    assert lib.svtad_table_grid(I64(0), 3, 3, None, 64, None) == 0
    assert lib.svtad_table_to_global(aligned, 32, I64(-1), I64(4), aligned, aligned, None) == -1
    st = lib.svtad_table_to_global(None, 64, I64(3), I64(4), aligned, aligned, None)
    assert st == -1 and b"null pointer" in lib.svtad_last_error()
    assert lib.svtad_table_to_global(None, 32, I64(0), I64(4), None, None, None) == 0


def test_table_limits_rejected(lib):
    st = lib.svtad_table_scan(ctypes.create_string_buffer(8), I64(1), 200, 200,
                              ctypes.create_string_buffer(8), None)
    assert st == -3 and b"16384" in lib.svtad_last_error()


def test_extension_module_api():
    import eccv26_tad_amd  # noqa: F401
    import opentad_sparse_ops as ops

    for name in ("fwd", "bwd_in", "bwd_w", "implicit_gemm_fwd_v2", "implicit_gemm_fwd_v2_chunked"):
        assert hasattr(ops, name)
    for name in ("fwd_bias", "bwd_w_bias", "dw_fwd", "dw_bwd_in", "dw_bwd_w",
                 "build_neighbor_table", "remap_neighbor_table", "transpose_neighbor_table",
                 "validate_neighbor_table", "prune_tokens", "bwd_packed", "adapter_down",
                 "adapter_up", "linear_wgrad", "column_sums", "gelu_backward_split", "gamma_grad", "up_proj_grads",
                 "dw_bwd", "heatmap_add_", "build_neighbor_table_n", "grid_neighbor_table", "table_to_global"):
        assert hasattr(ops, name)
    import torch

    with pytest.raises(RuntimeError, match="GPU tensor"):
        ops.fwd(torch.zeros(4, 8), torch.zeros(4, 9, dtype=torch.int32), torch.zeros(9, 8, 8), 8, 0)


def test_wrapper_module_shapes_and_init():
    import math

    import torch

    from eccv26_tad_amd import SparseConv2d, SparseDepthwiseConv2d

    torch.manual_seed(0)
    m = SparseConv2d(48, 32)
    assert m.weight.shape == (9, 48, 32) and m.bias.shape == (32,)
    bound = 1 / math.sqrt(48 * 9)
    assert float(m.weight.abs().max()) <= bound + 1e-7
    assert float(m.bias.abs().max()) <= bound + 1e-7
    assert set(m.state_dict()) == {"weight", "bias"}
    assert SparseConv2d(16, 16, bias=False).bias is None
    d = SparseDepthwiseConv2d(12)
    assert d.weight.shape == (9, 12)


def test_cin_not_divisible_by_4_raises():
    import torch

    from eccv26_tad_amd import SparseConv2dFunction

    with pytest.raises(ValueError, match="divisible by 4"):
        SparseConv2dFunction.apply(torch.zeros(2, 6), torch.zeros(2, 9, dtype=torch.int32),
                                   torch.zeros(9, 6, 4), None, 0, 0)


def test_packed_weight_cache_off_gpu():
    """The packed-weight cache holds nothing for a CPU weight (the Function
    then packs, which fails loudly without a GPU), and is not module state."""
    import torch

    from eccv26_tad_amd import SparseConv2d

    m = SparseConv2d(16, 16)
    assert m.packed_weight_cache.get(m.weight, m.weight, True) is None
    assert m.packed_weight_cache._packed is None
    assert set(m.state_dict()) == {"weight", "bias"}
    with torch.inference_mode():
        inf = torch.nn.Parameter(torch.zeros(9, 16, 16))
    assert m.packed_weight_cache.get(inf, inf, False) is None


def test_legacy_weight_remap():
    import torch

    from eccv26_tad_amd import remap_legacy_sparse_conv_weights

    legacy = torch.arange(8 * 9 * 4, dtype=torch.float32).view(8, 9, 4)
    sd = {"blk.sparse_conv.weight": legacy, "other": torch.zeros(3)}
    model = {"blk.sparse_conv.weight": torch.zeros(9, 8, 4), "other": torch.zeros(3)}
    out = remap_legacy_sparse_conv_weights(sd, model)
    assert out["blk.sparse_conv.weight"].shape == (9, 8, 4)
    assert torch.equal(out["blk.sparse_conv.weight"][2, 5], legacy[5, 2])


def _fused_plan(lib, n, ci, co, dt):
    a, b, s = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    st = lib.svtad_bwd_fused_plan(I64(n), ci, co, dt, ctypes.byref(a), ctypes.byref(b), ctypes.byref(s))
    return st, (a.value, b.value, s.value)


def test_bwd_fused_plan_at_config_2(lib, monkeypatch):
    """The one-launch backward's choice at config 2 (C = 192 fp16, 256 CUs
    assumed on a host without a GPU): the backward-input tiles and the
    backward-weight units (12 per split: the center offset in four parts)
    fit one workgroup per CU at 10-40 % keep, with splits of at most 2560
    rows whose partials fit the backward-weight workspace; 55 % keep and above
    keep two launches. Other widths than 192 and 256, and f32, never fuse."""
    monkeypatch.delenv("SVTAD_BWD_FUSED", raising=False)
    want = {3136: (1, (3, 1, 4)), 7840: (1, (3, 3, 7)), 12544: (1, (4, 3, 5)),
            17248: (0, (0, 0, 0)), 21952: (0, (0, 0, 0)), 31360: (0, (0, 0, 0))}
    lib.svtad_bwd_w_workspace_bytes.restype = ctypes.c_size_t
    for n, w in want.items():
        st, got = _fused_plan(lib, n, 192, 192, 1)
        assert (st, got) == w, (n, st, got)
        for tr, tc, sp in [got] if st == 1 else []:
            tiles = -(-n // (16 * tr)) * (192 // (64 * tc))
            assert tiles + 12 * sp <= 256  # one workgroup per CU
            need = sp * (12 * 192 * 192 + 4 * 192) * 4
            assert need <= lib.svtad_bwd_w_workspace_bytes(ctypes.c_int64(n), 192, 192, 1)
    assert _fused_plan(lib, 3136, 192, 192, 2)[0] == 1  # bf16
    assert _fused_plan(lib, 3136, 192, 192, 0)[0] == 0  # f32: VALU kernels
    # config 4 (C = 256 bf16): 128-column tiles of three row fragments and 2
    # splits at 10 % keep; two launches at 25 % and 55 %
    assert _fused_plan(lib, 4916, 256, 256, 2) == (1, (3, 2, 2))
    assert _fused_plan(lib, 12288, 256, 256, 2)[0] == 0
    assert _fused_plan(lib, 27034, 256, 256, 2)[0] == 0
    assert _fused_plan(lib, 4916, 512, 512, 2)[0] == 0  # no one-launch configuration at C = 512
    assert _fused_plan(lib, 3136, 192, 128, 1)[0] == 0


def test_bwd_fused_plan_override(lib, monkeypatch):
    monkeypatch.setenv("SVTAD_BWD_FUSED", "off")
    assert _fused_plan(lib, 3136, 192, 192, 1) == (0, (0, 0, 0))
    monkeypatch.setenv("SVTAD_BWD_FUSED", "3x3:4")
    st, (tr, tc, sp) = _fused_plan(lib, 3136, 192, 192, 1)
    assert (st, tr, tc, sp) == (1, 3, 3, 4)
    # without a count: the most splits whose partials the backward-weight
    # workspace holds (sized for 7 splits of 10 units at 3136 rows: 5 of 12)
    monkeypatch.setenv("SVTAD_BWD_FUSED", "4x3")
    assert _fused_plan(lib, 3136, 192, 192, 1) == (1, (4, 3, 5))
    monkeypatch.setenv("SVTAD_BWD_FUSED", "5x3")
    st, _ = _fused_plan(lib, 3136, 192, 192, 1)
    assert st == -1 and b"SVTAD_BWD_FUSED" in lib.svtad_last_error()
    monkeypatch.setenv("SVTAD_BWD_FUSED", "fused")  # unreadable
    st, _ = _fused_plan(lib, 3136, 192, 192, 1)
    assert st == -1 and b"SVTAD_BWD_FUSED" in lib.svtad_last_error()
    monkeypatch.setenv("SVTAD_BWD_FUSED", "3x2")  # the C = 256 shape
    assert _fused_plan(lib, 3136, 192, 192, 1)[0] == -1
    assert _fused_plan(lib, 4916, 256, 256, 2) == (1, (3, 2, 5))  # 5 of 12 units in the workspace of 7 x 10
    # forced split counts are clamped to what the launch accepts: no more than
    # the workspace holds, no split above 4096 rows
    monkeypatch.setenv("SVTAD_BWD_FUSED", "3x3:1000")
    assert _fused_plan(lib, 3136, 192, 192, 1) == (1, (3, 3, 5))
    monkeypatch.setenv("SVTAD_BWD_FUSED", "3x1:1")
    st, (tr, tc, sp) = _fused_plan(lib, 12544, 192, 192, 1)
    assert st == 1 and (tr, tc) == (3, 1) and sp == 4  # 3328 rows each
    monkeypatch.delenv("SVTAD_BWD_FUSED")
    st, _ = _fused_plan(lib, -1, 192, 192, 1)
    assert st == -1


def test_table_flags_checked_on_host(lib):
    buf = ctypes.create_string_buffer(64)
    aligned = ctypes.c_void_p((ctypes.addressof(buf) + 15) & ~15)
    U = ctypes.c_uint
    # unknown bits are rejected before any launch (0 and SVTAD_TABLE_SYMMETRIC = 1 are accepted)
    st = lib.svtad_bwd_in_packed_ex(aligned, aligned, aligned, aligned, aligned, I64(4), 192, 192, I64(0), 1,
                                    U(2), None)
    assert st == -1 and b"table_flags" in lib.svtad_last_error()
    st = lib.svtad_bwd_packed_ex(aligned, aligned, aligned, aligned, aligned, aligned, aligned, None, aligned,
                                 ctypes.c_size_t(1 << 30), I64(4), 192, 192, I64(0), 1, U(0x10), None)
    assert st == -1 and b"table_flags" in lib.svtad_last_error()
    st = lib.svtad_dw_bwd_in_ex(aligned, aligned, aligned, aligned, I64(4), 64, I64(0), 1, U(4), None)
    assert st == -1 and b"table_flags" in lib.svtad_last_error()
    st = lib.svtad_dw_bwd_ex(aligned, aligned, aligned, aligned, aligned, aligned, None, aligned,
                             ctypes.c_size_t(1 << 30), I64(4), 64, I64(0), 1, U(3), None)
    assert st == -1 and b"table_flags" in lib.svtad_last_error()
    st = lib.svtad_bwd_in_gemm(aligned, aligned, aligned, aligned, I64(4), 192, 192, I64(0), 1, U(8), None)
    assert st == -1 and b"table_flags" in lib.svtad_last_error()
    # empty inputs with valid flags are no-ops
    assert lib.svtad_dw_bwd_in_ex(None, None, None, None, I64(0), 64, I64(0), 1, U(1), None) == 0
    assert lib.svtad_bwd_in_packed_ex(None, None, None, None, None, I64(0), 192, 192, I64(0), 1, U(1), None) == 0


def test_symmetric_record_follows_the_tensor_version():
    import torch

    from eccv26_tad_amd import is_symmetric_table, mark_symmetric_table
    from eccv26_tad_amd.neighbor import _keep_symmetric

    t = torch.full((6, 9), -1, dtype=torch.int32)
    assert not is_symmetric_table(t) and not is_symmetric_table(None)
    mark_symmetric_table(t)
    assert is_symmetric_table(t)
    # a change through a view drops it (views share the version counter)
    v = t.view(2, 3, 9)
    assert not is_symmetric_table(v)  # the view object itself carries no record
    v[0, 0, 0] = 3
    assert not is_symmetric_table(t)
    # propagation: only from a recorded, unchanged source
    u = mark_symmetric_table(torch.full((4, 9), -1, dtype=torch.int64))
    w = _keep_symmetric(u, u.reshape(-1, 9).to(torch.int32))
    assert is_symmetric_table(w)
    assert not is_symmetric_table(_keep_symmetric(t, t.clone()))
    # a copy of a recorded table carries nothing (the checked path)
    assert not is_symmetric_table(u.clone())


def test_inference_tensors_get_no_record():
    import torch

    from eccv26_tad_amd import is_symmetric_table, mark_symmetric_table

    with torch.inference_mode():
        t = mark_symmetric_table(torch.full((4, 9), -1, dtype=torch.int32))
        assert not is_symmetric_table(t)
    assert not is_symmetric_table(t)
