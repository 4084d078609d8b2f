"""breadv2_amd — MI355X (gfx950) MoE feed-forward hot path of BREAD.

The compute lives in libbread_moe.so (HIP kernels behind the C ABI in
include/bread_moe.h); this package is its Python host layer.  Importing it
without the built library raises: there is no CPU fallback.
"""
from ._lib import BreadError, MoeLayer, MoeShape, lib, status_str  # noqa: F401
from .api import (  # noqa: F401
    Arena,
    Gguf,
    LayerTensors,
    MoeContext,
    argmax_f16,
    bread_dequant_rows,
    bread_matvec,
    bread_matvec_f32,
    bread_rmsnorm_f32,
    layer_seeds,
    row_bytes,
    shape,
    shape_bytes,
    spec_accept,
    synth_layer_tensors,
)
