"""nativebit_amd -- MI355X (gfx950) packed-weight decode path for NativeBit.

The packed NativeBit linear layer (3-bit indices + per-block fp32 codebooks)
and its fused dequant-GEMV, running on hand-written HIP kernels in
libnativebit_amd.so behind a C ABI (include/nativebit_amd.h).

    from nativebit_amd import PackedLinear
    layer = PackedLinear.from_packed(indices_np, codebook_np, (out, in), "cuda")
    y = layer(x)            # x (..., in) float32/bfloat16 on the GPU -> float32
"""
from .linear import BS, NE, PackedLinear  # noqa: F401
from ._lib import NativeBitError  # noqa: F401

__all__ = ["PackedLinear", "NativeBitError", "BS", "NE"]
