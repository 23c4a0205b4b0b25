"""Drop-in SparseConv2d / SparseConv2dFunction over the MI355X extension.

Mirrors opentad/models/bricks/sparse_conv_layer.py of pcr-upm/eccv26_tad:
same constructor, parameter names and layouts (``weight (9, C_in, C_out)``,
``bias (C_out)``), same forward signature, the same ``tokens_per_batch``
heuristic, autocast casting, C_in % 4 check and the same two bias paths. All
arithmetic runs in the ``opentad_sparse_ops`` HIP kernels.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
from torch.autograd import Function

from . import opentad_sparse_ops as _ops
from .neighbor import _keep_symmetric, global_neighbor_table, is_symmetric_table

try:  # torch >= 2.4
    from torch.amp import custom_bwd as _custom_bwd, custom_fwd as _custom_fwd

    custom_fwd = _custom_fwd(device_type="cuda")
    custom_bwd = _custom_bwd(device_type="cuda")
except ImportError:  # pragma: no cover - older torch
    from torch.cuda.amp import custom_bwd, custom_fwd  # type: ignore

# Channel count from which the reference switches to its implicit-GEMM forward,
# whose bias is added in fp32 before rounding (sparse_conv_layer.py:55-75);
# below it the bias is added after rounding (:76-89).
IMPLICIT_GEMM_MIN_CIN = 128

BIAS_NONE, BIAS_FP32, BIAS_AFTER = 0, 1, 2


class PackedWeightCache:
    """The matrix-core layouts of one module's weight (``pack_weight``), kept
    across forwards while the weight is unchanged, so that a recomputed
    forward (activation checkpointing) and inference skip the pack launch.

    An entry is reused when the parameter is the same object at the same
    address with the same version counter (every in-place update made through
    the tensor bumps it: optimizer steps, ``load_state_dict``, ``copy_`` under
    ``no_grad``), the compute dtype (the autocast target) and device match,
    and the current stream is the one the pack ran on. A training step that
    updates the weight therefore packs once per step, as without the cache.
    Writes through ``weight.data`` do not bump the version counter: call
    ``invalidate()`` after them. Inference tensors have no version counter and
    are packed on every call.

    The backward-input layout ends with the orphan flag word (set by the
    backward-input kernel when the table has an entry whose symmetric partner
    is missing, cleared only by a pack): a reused layout keeps a set flag, which
    makes later backward passes run the orphan pass even for a symmetric table.
    That costs one launch and never changes a result."""

    def __init__(self):
        self.invalidate()

    def invalidate(self):
        self._param = None
        self._key = None
        self._packed = None

    def get(self, param, weight, need_bwd):
        """``(packed_fwd, packed_bwd)`` for ``weight``, which is ``param`` or its
        cast to the compute dtype; ``packed_bwd`` is None when not requested.
        None (the caller packs) off the GPU or for an inference tensor."""
        if not weight.is_cuda or param.is_inference():
            return None
        stream = torch.cuda.current_stream(weight.device).cuda_stream
        key = (param.data_ptr(), param._version, weight.dtype, weight.device, stream)
        if param is self._param and key == self._key and (self._packed[1] is not None or not need_bwd):
            return self._packed
        pf, pb = _ops.pack_weight(weight.detach(), True, need_bwd)
        self._param, self._key, self._packed = param, key, (pf, pb if need_bwd else None)
        return self._packed


class SparseConv2dFunction(Function):
    """autograd Function of the sparse 3x3 convolution
    (reference sparse_conv_layer.py:29-123).

    ``packed`` (not in the reference; optional) is ``(packed_fwd,
    packed_bwd)`` from ``pack_weight(weight, True, ...)``, ``packed_bwd`` None
    when it was not requested; without it the weight is packed here. The
    backward skips the partner checks for a table that carries the
    symmetric record of the table builders (``is_symmetric_table``)."""

    @staticmethod
    @custom_fwd
    def forward(ctx, x, neighbor_indices, weight, bias=None, tokens_per_batch=0, chunk_size=0, packed=None):
        _, C_in, C_out = weight.shape
        ctx.symmetric = is_symmetric_table(neighbor_indices)
        if C_in % 4 != 0:
            raise ValueError(f"C_in ({C_in}) must be divisible by 4 for optimized kernel.")
        ctx.C_in = C_in
        ctx.tokens_per_batch = tokens_per_batch
        if bias is None:
            mode = BIAS_NONE
        elif C_in >= IMPLICIT_GEMM_MIN_CIN:
            mode = BIAS_FP32
        else:
            mode = BIAS_AFTER
        # Both matrix-core weight layouts in one launch; the backward-input one
        # is kept for backward (empty tensors where the shape has none).
        need_bwd = bool(ctx.needs_input_grad[0])
        if packed is None or (need_bwd and packed[1] is None):
            packed = _ops.pack_weight(weight, True, need_bwd)
        packed_fwd, packed_bwd = packed
        ctx.save_for_backward(x, neighbor_indices, weight, bias, packed_bwd if need_bwd else None)
        return _ops.fwd_packed(x, neighbor_indices, weight, packed_fwd, bias, tokens_per_batch, mode)

    @staticmethod
    @custom_bwd
    def backward(ctx, grad_output):
        x, neighbor_indices, weight, bias, packed_bwd = ctx.saved_tensors
        C_in = ctx.C_in
        tpb = ctx.tokens_per_batch
        go = grad_output.contiguous()
        grad_input = grad_weight = grad_bias = None
        need_b = bias is not None and ctx.needs_input_grad[3]
        if ctx.needs_input_grad[0] and ctx.needs_input_grad[2]:
            # both gradients in one call (the same kernels as the two calls
            # below, with one launch less)
            gi, gw, gb = _ops.bwd_packed(go, x, neighbor_indices, weight, packed_bwd, C_in, tpb, need_b,
                                         symmetric=ctx.symmetric)
            grad_input = gi.view(x.shape) if x.dim() == 3 else gi
            grad_weight = gw
            grad_bias = gb if need_b else None
            return grad_input, None, grad_weight, grad_bias, None, None, None
        if ctx.needs_input_grad[0]:
            grad_input = _ops.bwd_in_packed(go, neighbor_indices, weight, packed_bwd,
                                            x.numel() // x.shape[-1], C_in, tpb, symmetric=ctx.symmetric)
            if x.dim() == 3:
                grad_input = grad_input.view(x.shape)
        if ctx.needs_input_grad[2] or need_b:
            gw, gb = _ops.bwd_w_bias(go, x, neighbor_indices, C_in, tpb, need_b)
            if ctx.needs_input_grad[2]:
                grad_weight = gw
            if need_b:
                grad_bias = gb
        return grad_input, None, grad_weight, grad_bias, None, None, None


def _table_and_tpb(x, neighbor_indices, tokens_per_batch):
    """The int32 ``[rows, 9]`` table and tokens_per_batch for the kernels.

    For a 3D input without an explicit ``tokens_per_batch`` this is the
    reference heuristic (sparse_conv_layer.py:170-177: local per-sample
    indices when the table's max is < N), evaluated on the device by
    ``global_neighbor_table``: the table comes back global, so the kernels run
    with tokens_per_batch = 0, and there is no host synchronisation (the
    reference reads ``max()`` back). The table keeps the input's symmetric
    record."""
    if x.dim() == 3 and tokens_per_batch is None:
        return global_neighbor_table(neighbor_indices, x.shape[1]), 0
    nbr = neighbor_indices.reshape(-1, 9)
    if nbr.dtype != torch.int32:
        nbr = nbr.to(torch.int32)
    return _keep_symmetric(neighbor_indices, nbr), (tokens_per_batch or 0)


def _autocast_cast(x, weight, bias):
    """Dtype policy of sparse_conv_layer.py:191-202."""
    if torch.is_autocast_enabled("cuda"):
        target = torch.get_autocast_dtype("cuda")
        if x.dtype != target:
            x = x.to(target)
        if weight.dtype != target:
            weight = weight.to(target)
        if bias is not None and bias.dtype != target:
            bias = bias.to(target)
    elif x.dtype != weight.dtype:
        weight = weight.to(x.dtype)
        if bias is not None:
            bias = bias.to(x.dtype)
    return x, weight, bias


class SparseConv2d(nn.Module):
    """3x3 convolution over a pruned token set (reference sparse_conv_layer.py:126-211).

    ``forward(x, neighbor_indices)``: x is ``[N, C_in]`` or ``[B, N, C_in]``;
    neighbor_indices ``[N, 9]`` / ``[B, N, 9]`` (int32 or int64, -1 = missing).
    ``tokens_per_batch`` may be passed to skip the reference's ``max()``
    heuristic; ``None`` keeps it, evaluated on the device (no host sync).

    ``packed_weight_cache`` (a ``PackedWeightCache``; not in the reference)
    keeps the weight's matrix-core layouts between forwards while the weight
    is unchanged; set it to None to pack on every forward.
    """

    def __init__(self, in_channels, out_channels, bias=True, chunk_size=4096):
        super().__init__()
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.chunk_size = chunk_size  # accepted for API compatibility; not needed
        self.weight = nn.Parameter(torch.Tensor(9, in_channels, out_channels))
        if bias:
            self.bias = nn.Parameter(torch.Tensor(out_channels))
        else:
            self.register_parameter("bias", None)
        self.packed_weight_cache = PackedWeightCache()
        self.reset_parameters()

    def reset_parameters(self):
        # Kaiming-uniform(a=sqrt(5)) on the standard (C_out, C_in, 3, 3) layout,
        # re-laid out to (9, C_in, C_out) (sparse_conv_layer.py:145-161).
        temp = torch.empty(self.out_channels, self.in_channels, 3, 3)
        nn.init.kaiming_uniform_(temp, a=math.sqrt(5))
        with torch.no_grad():
            self.weight.copy_(temp.view(self.out_channels, self.in_channels, 9).permute(2, 1, 0))
        if self.bias is not None:
            fan_in, _ = nn.init._calculate_fan_in_and_fan_out(temp)
            bound = 1 / math.sqrt(fan_in)
            nn.init.uniform_(self.bias, -bound, bound)

    def forward(self, x, neighbor_indices, tokens_per_batch=None):
        is_batched = x.dim() == 3
        nbr, tpb = _table_and_tpb(x, neighbor_indices, tokens_per_batch)
        if is_batched:
            B, N, C = x.shape
            x = x.reshape(-1, C)
        x, weight, bias = _autocast_cast(x, self.weight, self.bias)
        cache = self.packed_weight_cache
        packed = None
        if cache is not None:
            packed = cache.get(self.weight, weight, torch.is_grad_enabled() and x.requires_grad)
        out = SparseConv2dFunction.apply(x, nbr, weight, bias, tpb, self.chunk_size, packed)
        if is_batched:
            out = out.view(B, N, -1)
        return out


class SparseDepthwiseConv2dFunction(Function):
    """Depthwise (groups = C) sparse 3x3 convolution; weight (9, C). Not in the
    reference; same index semantics as SparseConv2dFunction."""

    @staticmethod
    @custom_fwd
    def forward(ctx, x, neighbor_indices, weight, bias=None, tokens_per_batch=0):
        ctx.save_for_backward(x, neighbor_indices, weight, bias)
        ctx.tokens_per_batch = tokens_per_batch
        ctx.symmetric = is_symmetric_table(neighbor_indices)
        return _ops.dw_fwd(x, neighbor_indices, weight, bias, tokens_per_batch)

    @staticmethod
    @custom_bwd
    def backward(ctx, grad_output):
        x, neighbor_indices, weight, bias = ctx.saved_tensors
        tpb = ctx.tokens_per_batch
        go = grad_output.contiguous()
        grad_input = grad_weight = grad_bias = None
        need_b = bias is not None and ctx.needs_input_grad[3]
        if ctx.needs_input_grad[0] and ctx.needs_input_grad[2]:
            # all gradients in one pass over the rows plus one reduction
            gi, gw, gb = _ops.dw_bwd(go, x, neighbor_indices, weight, tpb, need_b, symmetric=ctx.symmetric)
            return gi.view(x.shape), None, gw, gb if need_b else None, None
        if ctx.needs_input_grad[0]:
            grad_input = _ops.dw_bwd_in(go, neighbor_indices, weight, tpb, symmetric=ctx.symmetric).view(x.shape)
        if ctx.needs_input_grad[2] or need_b:
            gw, gb = _ops.dw_bwd_w(go, x, neighbor_indices, tpb, need_b)
            grad_weight = gw if ctx.needs_input_grad[2] else None
            grad_bias = gb if need_b else None
        return grad_input, None, grad_weight, grad_bias, None


class SparseDepthwiseConv2d(nn.Module):
    """Depthwise sparse 3x3 convolution, weight ``(9, C)`` with k = ky*3 + kx."""

    def __init__(self, channels, bias=True):
        super().__init__()
        self.channels = channels
        self.weight = nn.Parameter(torch.Tensor(9, channels))
        if bias:
            self.bias = nn.Parameter(torch.Tensor(channels))
        else:
            self.register_parameter("bias", None)
        self.reset_parameters()

    def reset_parameters(self):
        temp = torch.empty(self.channels, 1, 3, 3)
        nn.init.kaiming_uniform_(temp, a=math.sqrt(5))
        with torch.no_grad():
            self.weight.copy_(temp.view(self.channels, 9).t())
        if self.bias is not None:
            bound = 1 / math.sqrt(9)
            nn.init.uniform_(self.bias, -bound, bound)

    def forward(self, x, neighbor_indices, tokens_per_batch=None):
        is_batched = x.dim() == 3
        nbr, tpb = _table_and_tpb(x, neighbor_indices, tokens_per_batch)
        if is_batched:
            B, N, C = x.shape
            x = x.reshape(-1, C)
        x, weight, bias = _autocast_cast(x, self.weight, self.bias)
        out = SparseDepthwiseConv2dFunction.apply(x, nbr, weight, bias, tpb)
        if is_batched:
            out = out.view(B, N, -1)
        return out


def remap_legacy_sparse_conv_weights(state_dict, model_state_dict):
    """Permute legacy ``(C_in, 9, C_out)`` ``sparse_conv.weight`` entries to the
    ``(9, C_in, C_out)`` layout when the model expects it
    (reference opentad/utils/checkpoint.py:42-55)."""
    for key, param in list(state_dict.items()):
        if key.endswith("sparse_conv.weight") and key in model_state_dict:
            target = model_state_dict[key].shape
            if param.shape != target and param.dim() == 3:
                permuted = param.permute(1, 0, 2).contiguous()
                if permuted.shape == target:
                    state_dict[key] = permuted
    return state_dict
