"""MI355X-native SparseConv2D for SV-TAD (pcr-upm/eccv26_tad).

Importing the package loads the in-tree native extension ``opentad_sparse_ops``
(built by ``python eccv26_tad_amd/build.py``) and registers it under its
top-level name, so reference code doing ``import opentad_sparse_ops`` gets
this build. There is no CPU or Python fallback: a missing extension raises.
"""
from __future__ import annotations

import importlib.util
import os
import sys

_PKG = os.path.dirname(os.path.abspath(__file__))


def _load_extension():
    import sysconfig

    import torch  # noqa: F401  (loads the HIP runtime the extension binds to)

    path = os.path.join(_PKG, "opentad_sparse_ops" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))
    if not os.path.exists(path):
        raise ImportError(
            f"eccv26_tad_amd: native extension not built ({path} missing); "
            "run `python eccv26_tad_amd/build.py`")
    spec = importlib.util.spec_from_file_location("opentad_sparse_ops", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    sys.modules.setdefault("opentad_sparse_ops", mod)
    return mod


opentad_sparse_ops = _load_extension()
ops = opentad_sparse_ops

from .neighbor import (  # noqa: E402
    build_neighbor_table,
    get_initial_neighbor_indices,
    global_neighbor_table,
    is_symmetric_table,
    mark_symmetric_table,
    prune_tokens,
    set_debug_sparse,
    remap_neighbor_table,
    transpose_neighbor_table,
    validate_neighbor_table,
)
from .adapter import (AdapterDownFunction, AdapterUpFunction, SparseConvAdapter,  # noqa: E402
                      SparseConvAdapterFunction)
from .dense_path import (  # noqa: E402
    conv2d_weight_from_sparse,
    dense_conv_tokens,
    keep_mask_from_indices,
    sparse_weight_from_conv2d,
)
from .sparse_conv_layer import (  # noqa: E402
    SparseConv2d,
    SparseConv2dFunction,
    SparseDepthwiseConv2d,
    SparseDepthwiseConv2dFunction,
    remap_legacy_sparse_conv_weights,
)

LIB_PATH = os.path.join(_PKG, "libsvtad_sparse.so")

__all__ = [
    "opentad_sparse_ops", "ops", "SparseConv2d", "SparseConv2dFunction",
    "SparseDepthwiseConv2d", "SparseDepthwiseConv2dFunction",
    "build_neighbor_table", "get_initial_neighbor_indices", "prune_tokens", "remap_neighbor_table",
    "transpose_neighbor_table", "validate_neighbor_table", "global_neighbor_table", "set_debug_sparse",
    "is_symmetric_table", "mark_symmetric_table",
    "remap_legacy_sparse_conv_weights",
    "dense_conv_tokens", "keep_mask_from_indices", "sparse_weight_from_conv2d",
    "conv2d_weight_from_sparse", "SparseConvAdapter", "AdapterDownFunction", "AdapterUpFunction", "SparseConvAdapterFunction",
    "LIB_PATH",
]
