"""Function-level mirror of the reference's packed-operator entry points.

The reference exposes (inference/triton_kernel.py, inference/cuda_kernel.py):

    dequant_matvec(x, indices, codebook, N, K)          uint8 indices, K4
    dequant_matvec_3bit(x, packed_indices, codebook, N, K)   Triton K2
    dequant_matvec_3bit_cuda(x, packed, codebook, N, K)      CUDA K1
    pack_indices_to_3bit(indices_uint8)
    PackedLinear

Here all of them run on the gfx950 kernels of libnativebit_amd.so, with the
same argument meaning and the same float32 (N,) result.  The reference's
``tile_n`` tuning argument is accepted and ignored (the launch shape is chosen
by the library).
"""
from __future__ import annotations

import torch

from . import ops
from .linear import BS, NE, PackedLinear  # noqa: F401


def _as_gemv_input(x: torch.Tensor) -> torch.Tensor:
    """x as fp32 on the device, whatever float type it arrives in: the
    reference's kernels multiply x read as fp32 by the exact fp32 codebook
    values (triton_kernel.py:46, 174-183; the CUDA kernel takes fp32 x only,
    cuda_kernel.py:74-77, 97), so these entry points compute exactly that
    (the fp32 kernels of nb_gemv) for bf16 and fp16 x too."""
    x = x.reshape(-1)
    return x if x.dtype == torch.float32 else x.to(torch.float32)


def dequant_matvec_3bit(x: torch.Tensor, packed_indices: torch.Tensor,
                        codebook: torch.Tensor, N: int, K: int, tile_n=None) -> torch.Tensor:
    """y = W @ x for a 3-bit packed W (N x K), block 128; x (K,) -> y (N,) fp32."""
    return ops.gemv(_as_gemv_input(x), packed_indices.reshape(-1), codebook.reshape(-1, NE),
                    int(N), int(K), bits=3, block_size=BS)


def dequant_matvec_3bit_cuda(x, packed, codebook, N, K):
    """Same contract as the reference's CUDA entry (inference/cuda_kernel.py:133-136)."""
    return dequant_matvec_3bit(x, packed, codebook, N, K)


def dequant_matvec(x: torch.Tensor, indices: torch.Tensor, codebook: torch.Tensor,
                   N: int, K: int, tile_n=None) -> torch.Tensor:
    """Unpacked-index variant: indices (num_blocks, BS) uint8, one byte each.

    One byte per index is an 8-bit LSB-first stream, so this is the same
    GEMV with bits = 8.
    """
    idx = indices.reshape(-1)
    if idx.dtype != torch.uint8:
        idx = idx.to(torch.uint8)
    return ops.gemv(_as_gemv_input(x), idx.contiguous(), codebook.reshape(-1, codebook.shape[-1]),
                    int(N), int(K), bits=8, block_size=BS)


def pack_indices_to_3bit(indices_uint8: torch.Tensor) -> torch.Tensor:
    """8 indices -> 3 bytes on the device (inference/triton_kernel.py:199-220)."""
    return ops.pack(indices_uint8, 3)
