"""MI355X (gfx950) fused Qwen3 SwiGLU MLP: ``out = residual + down(silu(gate(x)) * up(x))``.

Host code for ``libqwen_mlp.so`` (hand-written HIP kernels behind the C ABI in
``include/qwen_mlp.h``).  The public surface mirrors the reference module
``docker/qwen-c2-graft/graft/mlp.py``: ``Qwen36MLP``, ``MLPWeights``, ``load_mlp_weights``.
"""
from ._lib import FMT_BF4, FMT_BF16, FMT_BFP8, LIB_PATH, QmlpError, lib
from .mlp import (
    MATRIX_FORMATS,
    WEIGHT_FORMATS,
    MLPWeights,
    PackedWeight,
    Qwen36MLP,
    WorkspacePool,
    dequantize,
    load_mlp_weights,
    matrix_formats,
    mlp_forward,
    mlp_forward_rmsnorm,
    new_workspace,
    pack_canonical,
    pack_canonical_bfp8,
    pack_weight,
    quantize_bf4,
    quantize_bfp8,
    unpack_bfp8,
    unpack_canonical,
    workspace_bytes,
    workspace_pool,
)

__all__ = [
    "FMT_BF4", "FMT_BF16", "FMT_BFP8", "LIB_PATH", "QmlpError", "lib", "MATRIX_FORMATS", "WEIGHT_FORMATS",
    "MLPWeights", "PackedWeight", "Qwen36MLP", "dequantize", "load_mlp_weights", "matrix_formats", "mlp_forward",
    "mlp_forward_rmsnorm", "new_workspace", "pack_canonical", "pack_canonical_bfp8", "pack_weight", "quantize_bf4",
    "quantize_bfp8", "unpack_bfp8", "unpack_canonical", "workspace_bytes", "WorkspacePool", "workspace_pool",
]
