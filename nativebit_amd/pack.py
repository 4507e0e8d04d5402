"""Host-side packed format: the reference's CPU packers, vectorised.

Function names and results follow nativebit/pack.py and inference/pack.py;
all widths share one rule (index i occupies bits [i*b, (i+1)*b) of an
LSB-first little-endian stream) and are vectorised with numpy bit
operations, so the generic 2/5/6/7-bit paths that the reference runs as
per-bit Python loops (nativebit/pack.py:109-115, 129-137) take milliseconds
instead of hours on 2.2B-shape layers.

These are load/export-time utilities that run on host arrays.  The hot path
never uses them: device-side packing, unpacking and dequantization are the
nb_pack / nb_unpack / nb_dequant kernels (nativebit_amd.ops).
"""
from __future__ import annotations

import math

import numpy as np
import torch

FORMAT_VERSION = 1  # nativebit/pack.py:14


def packed_nbytes(count: int, bits: int) -> int:
    """3-bit pads to whole 24-bit groups, other widths to whole bytes."""
    if bits == 3:
        return 3 * ((count + 7) // 8)
    return (count * bits + 7) // 8


def _as_np_u8(indices) -> np.ndarray:
    if isinstance(indices, torch.Tensor):
        if indices.device.type != "cpu":
            raise ValueError("host packers take CPU tensors; use nativebit_amd.ops.pack on GPU")
        indices = indices.numpy()
    return np.ascontiguousarray(np.asarray(indices).reshape(-1).astype(np.uint8, copy=False))


def pack_bits_np(indices, bits: int) -> np.ndarray:
    """LSB-first stream of the low `bits` bits of each index (numpy uint8)."""
    idx = _as_np_u8(indices)
    n = idx.size
    nbytes = packed_nbytes(n, bits)
    if n == 0:
        return np.zeros(0, dtype=np.uint8)
    planes = (idx[:, None] >> np.arange(bits, dtype=np.uint8)[None, :]) & 1   # (n, bits)
    stream = planes.reshape(-1)
    pad = nbytes * 8 - stream.size
    if pad:
        stream = np.concatenate([stream, np.zeros(pad, dtype=np.uint8)])
    return np.packbits(stream, bitorder="little")


def unpack_bits_np(packed, count: int, bits: int) -> np.ndarray:
    """Inverse of pack_bits_np: `count` uint8 indices."""
    p = _as_np_u8(packed)
    if p.size * 8 < count * bits:
        raise ValueError(f"stream of {p.size} bytes holds fewer than {count} {bits}-bit fields")
    stream = np.unpackbits(p, bitorder="little")[: count * bits].reshape(count, bits)
    weights = (1 << np.arange(bits, dtype=np.uint16)).astype(np.uint16)
    return (stream.astype(np.uint16) @ weights).astype(np.uint8)


def _to_torch(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a))


# --- nativebit/pack.py names -------------------------------------------------

def pack_3bit(indices: torch.Tensor) -> torch.Tensor:
    """8 indices -> 3 bytes (nativebit/pack.py:21-41)."""
    return _to_torch(pack_bits_np(indices, 3))


def unpack_3bit(packed: torch.Tensor, count: int) -> torch.Tensor:
    """(nativebit/pack.py:44-68)."""
    return _to_torch(unpack_bits_np(packed, count, 3))


def pack_4bit(indices: torch.Tensor) -> torch.Tensor:
    """2 indices per byte, low nibble first (nativebit/pack.py:75-82)."""
    return _to_torch(pack_bits_np(indices, 4))


def unpack_4bit(packed: torch.Tensor, count: int) -> torch.Tensor:
    """(nativebit/pack.py:85-90)."""
    return _to_torch(unpack_bits_np(packed, count, 4))


def pack_nbits(indices: torch.Tensor, bits: int) -> torch.Tensor:
    """Any width 1..8 (nativebit/pack.py:97-116)."""
    if not 1 <= bits <= 8:
        raise ValueError(f"bits={bits} outside 1..8")
    return _to_torch(pack_bits_np(indices, bits))


def unpack_nbits(packed: torch.Tensor, count: int, bits: int) -> torch.Tensor:
    """(nativebit/pack.py:119-138)."""
    if not 1 <= bits <= 8:
        raise ValueError(f"bits={bits} outside 1..8")
    return _to_torch(unpack_bits_np(packed, count, bits))


def reconstruct_weight(indices: torch.Tensor, codebook: torch.Tensor, shape: tuple,
                       block_size: int, total_weights: int) -> torch.Tensor:
    """Gather W from indices + codebook (nativebit/pack.py:145-169)."""
    num_blocks = codebook.shape[0]
    idx = indices.reshape(num_blocks, block_size).long()
    w = torch.gather(codebook, 1, idx)
    return w.reshape(-1)[:total_weights].reshape(shape)


def bits_for_entries(n_entries: int) -> int:
    """ceil(log2(n_entries)) (nativebit/pack.py:230)."""
    return max(1, math.ceil(math.log2(n_entries)))


# --- inference/pack.py names -------------------------------------------------

def quantize_weight(weight: np.ndarray, codebook: np.ndarray) -> np.ndarray:
    """Nearest entry by squared distance, first on ties (inference/pack.py:21-35).

    Returns uint8 (num_blocks, block_size).  Processed in chunks of blocks so
    a 2.2B-shape layer does not materialise a multi-GB distance tensor.
    """
    num_blocks, n_entries = codebook.shape
    total = weight.size
    block_size = math.ceil(total / num_blocks)
    padded = num_blocks * block_size
    w = np.asarray(weight, dtype=np.float32).reshape(-1)
    if padded > total:
        w = np.pad(w, (0, padded - total))
    w = w.reshape(num_blocks, block_size)
    cb = np.asarray(codebook, dtype=np.float32)
    out = np.empty((num_blocks, block_size), dtype=np.uint8)
    step = max(1, (1 << 22) // max(1, block_size * n_entries))
    for b0 in range(0, num_blocks, step):
        b1 = min(num_blocks, b0 + step)
        d = (w[b0:b1, :, None] - cb[b0:b1, None, :]) ** 2
        out[b0:b1] = np.argmin(d, axis=-1).astype(np.uint8)
    return out


def pack_indices_3bit(indices) -> bytes:
    """uint8 indices -> 3-bit stream bytes (inference/pack.py:38-57)."""
    return pack_bits_np(indices, 3).tobytes()
