"""torch-tensor wrappers over the C ABI (device memory and streams come from
PyTorch-ROCm; all arithmetic runs in libnativebit_amd.so's gfx950 kernels).

Every wrapper checks devices, dtypes and shapes on the host, enqueues on
torch's current stream and raises NativeBitError on a non-zero status.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _lib

_DT = {torch.float32: _lib.NB_F32, torch.bfloat16: _lib.NB_BF16}


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    """torch's current stream on t's device, as the ABI's hipStream_t."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _require_cuda(name: str, t: torch.Tensor):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a ROCm GPU (got {t.device}); "
                         "this path has no CPU implementation")


def _same_device(*ts):
    dev = ts[0].device
    for t in ts[1:]:
        if t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")


def bits_for_entries(n_entries: int) -> int:
    """ceil(log2(n_entries)), as nativebit/pack.py:230."""
    if n_entries < 1:
        raise ValueError("n_entries must be >= 1")
    return max(1, math.ceil(math.log2(n_entries)))


def packed_nbytes(count: int, bits: int) -> int:
    return int(_lib.load().nb_packed_nbytes(int(count), int(bits)))


def gemv(x: torch.Tensor, packed: torch.Tensor, codebook: torch.Tensor, N: int,
         K: int, bits: int = 3, block_size: int = 128,
         out_dtype: torch.dtype = torch.float32, out: torch.Tensor | None = None):
    """y = x @ W.T for a packed W (N x K); x is (M, K) or (K,), M <= 16."""
    _require_cuda("x", x)
    _require_cuda("packed", packed)
    _require_cuda("codebook", codebook)
    _same_device(x, packed, codebook)
    squeeze = x.dim() == 1
    x2 = x.reshape(1, -1) if squeeze else x
    if x2.dim() != 2 or x2.shape[1] != K:
        raise ValueError(f"x must be (M, {K}) or ({K},), got {tuple(x.shape)}")
    if x2.dtype not in _DT:
        raise TypeError(f"x dtype {x2.dtype} not supported (float32 or bfloat16)")
    if x2.stride(1) != 1:
        x2 = x2.contiguous()
    if packed.dtype != torch.uint8 or not packed.is_contiguous():
        raise TypeError("packed must be a contiguous uint8 tensor")
    if codebook.dtype != torch.float32 or codebook.dim() != 2 or not codebook.is_contiguous():
        raise TypeError("codebook must be a contiguous float32 (num_blocks, n_entries) tensor")
    n_entries = codebook.shape[1]
    num_blocks = -(-N * K // block_size) if N * K else 0
    if codebook.shape[0] < num_blocks:
        raise ValueError(f"codebook has {codebook.shape[0]} blocks, {num_blocks} needed")
    need = packed_nbytes(N * K, bits)
    if packed.numel() < need:
        raise ValueError(f"packed has {packed.numel()} bytes, {need} needed")
    M = x2.shape[0]
    if out_dtype not in _DT:
        raise TypeError(f"out_dtype {out_dtype} not supported")
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=x.device)
    elif out.shape != (M, N) or out.dtype != out_dtype or out.stride(1) != 1:
        raise ValueError("out must be (M, N), row-contiguous, of out_dtype")
    lib = _lib.load()
    _lib.check(lib.nb_gemv(
        x2.data_ptr(), _DT[x2.dtype], x2.stride(0) if M > 1 else K,
        packed.data_ptr(), codebook.data_ptr(),
        out.data_ptr(), _DT[out_dtype], out.stride(0) if M > 1 else N,
        M, N, K, bits, n_entries, block_size, _stream(x)))
    return out.reshape(N) if squeeze else out


def unpack(packed: torch.Tensor, count: int, bits: int) -> torch.Tensor:
    """uint8 indices from an LSB-first stream (device)."""
    _require_cuda("packed", packed)
    if packed.dtype != torch.uint8 or not packed.is_contiguous():
        raise TypeError("packed must be a contiguous uint8 tensor")
    if packed.numel() * 8 < count * bits:
        raise ValueError("packed stream shorter than count * bits")
    out = torch.empty(count, dtype=torch.uint8, device=packed.device)
    _lib.check(_lib.load().nb_unpack(packed.data_ptr(), out.data_ptr(), count, bits,
                                     _stream(packed)))
    return out


def pack(indices: torch.Tensor, bits: int) -> torch.Tensor:
    """LSB-first stream of uint8 indices (device), zero padded."""
    _require_cuda("indices", indices)
    idx = indices.reshape(-1)
    if idx.dtype != torch.uint8:
        idx = idx.to(torch.uint8)
    idx = idx.contiguous()
    out = torch.empty(packed_nbytes(idx.numel(), bits), dtype=torch.uint8, device=idx.device)
    _lib.check(_lib.load().nb_pack(idx.data_ptr(), out.data_ptr(), idx.numel(), bits,
                                   _stream(idx)))
    return out


def dequant(packed: torch.Tensor, codebook: torch.Tensor, total: int, bits: int,
            block_size: int, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Flat W[:total] = codebook[i // block_size][index i] (device)."""
    _require_cuda("packed", packed)
    _require_cuda("codebook", codebook)
    _same_device(packed, codebook)
    if codebook.dtype != torch.float32 or codebook.dim() != 2 or not codebook.is_contiguous():
        raise TypeError("codebook must be a contiguous float32 (num_blocks, n_entries) tensor")
    if packed.dtype != torch.uint8 or not packed.is_contiguous():
        raise TypeError("packed must be a contiguous uint8 tensor")
    if packed.numel() < packed_nbytes(total, bits):
        raise ValueError("packed stream too short for total weights")
    if out_dtype not in _DT:
        raise TypeError(f"out_dtype {out_dtype} not supported")
    w = torch.empty(total, dtype=out_dtype, device=packed.device)
    _lib.check(_lib.load().nb_dequant(
        packed.data_ptr(), codebook.data_ptr(), w.data_ptr(), _DT[out_dtype], total,
        codebook.shape[0], bits, codebook.shape[1], block_size, _stream(packed)))
    return w
