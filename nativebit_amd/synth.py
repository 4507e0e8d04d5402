"""Seeded synthetic packed layers, as the benchmark configurations define them.

A layer of shape (N, K) is built the way the reference initialises and packs
a NativeBitLinear:

* latent weights W ~ N(0, std^2) fp32 from ``torch.Generator(seed)``;
* per-block codebook = ``torch.quantile(block, linspace(0, 1, NE))`` over the
  block's real weights (nativebit/codebook_utils.py:6-22 applied per block as
  nativebit/layers.py:72-76 does), computed in chunks because torch.quantile
  rejects inputs above 2^24 elements;
* indices = nearest entry by squared distance, first on ties, on the
  zero-padded flat weights (nativebit/layers.py:78-94, inference/pack.py:21-35);
* packed LSB-first at ceil(log2 NE) bits.

All of it is torch and runs on whatever device it is given (the benchmark
generates its 182 layers on the GPU).  This is input generation only.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import pack as host_pack

# 2.2B shape (configs/tpu.py:137-183): 26 layers, hidden 2560, FFN 6912.
N_LAYERS = 26
HIDDEN = 2560
FFN = 6912
# Per-layer packed matmuls as (name, out_features, in_features).
LAYER_SHAPES = (
    ("q", HIDDEN, HIDDEN), ("k", HIDDEN, HIDDEN), ("v", HIDDEN, HIDDEN),
    ("o", HIDDEN, HIDDEN), ("gate", FFN, HIDDEN), ("up", FFN, HIDDEN),
    ("down", HIDDEN, FFN),
)

_QUANTILE_LIMIT = 1 << 24


@dataclass
class PackedLayer:
    out_features: int
    in_features: int
    n_entries: int
    block_size: int
    bits: int
    codebook: torch.Tensor   # (num_blocks, n_entries) fp32
    packed: torch.Tensor     # flat uint8 stream
    indices: torch.Tensor | None = None  # (num_blocks * block_size,) uint8, if kept


def block_codebooks(w_flat: torch.Tensor, total: int, n_entries: int,
                    block_size: int) -> torch.Tensor:
    """Per-block quantile codebooks over each block's real weights."""
    num_blocks = -(-total // block_size)
    q = torch.linspace(0, 1, n_entries, device=w_flat.device)
    cb = torch.empty(num_blocks, n_entries, dtype=torch.float32, device=w_flat.device)
    full = total // block_size
    if full:
        blocks = w_flat[: full * block_size].reshape(full, block_size).float()
        step = max(1, _QUANTILE_LIMIT // block_size - 1)
        for b0 in range(0, full, step):
            b1 = min(full, b0 + step)
            cb[b0:b1] = torch.quantile(blocks[b0:b1], q, dim=1).T
    if full < num_blocks:  # tail block: quantiles of the weights that exist
        cb[full] = torch.quantile(w_flat[full * block_size: total].float(), q)
    return cb


def nearest_indices(w_flat: torch.Tensor, total: int, codebook: torch.Tensor,
                    block_size: int) -> torch.Tensor:
    """uint8 (num_blocks * block_size,) nearest-entry indices, padded tail = 0.0."""
    num_blocks, n_entries = codebook.shape
    padded = num_blocks * block_size
    w = w_flat[:total].float()
    if padded > total:
        w = torch.nn.functional.pad(w, (0, padded - total))
    w = w.reshape(num_blocks, block_size)
    out = torch.empty(num_blocks, block_size, dtype=torch.uint8, device=w.device)
    step = max(1, (1 << 24) // (block_size * n_entries))
    for b0 in range(0, num_blocks, step):
        b1 = min(num_blocks, b0 + step)
        d = (w[b0:b1, :, None] - codebook[b0:b1, None, :]).square()
        out[b0:b1] = d.argmin(dim=-1).to(torch.uint8)
    return out.reshape(-1)


def make_layer(out_features: int, in_features: int, n_entries: int = 8,
               block_size: int = 128, seed: int = 0, device="cpu",
               std: float = 0.02, keep_indices: bool = False) -> PackedLayer:
    device = torch.device(device)
    gen = torch.Generator(device=device).manual_seed(int(seed))
    total = out_features * in_features
    w = torch.randn(total, generator=gen, device=device, dtype=torch.float32) * std
    cb = block_codebooks(w, total, n_entries, block_size)
    idx = nearest_indices(w, total, cb, block_size)
    del w
    bits = host_pack.bits_for_entries(n_entries)
    if device.type == "cuda":
        from . import ops
        packed = ops.pack(idx, bits)
    else:
        packed = host_pack.pack_nbits(idx, bits)
    return PackedLayer(out_features, in_features, n_entries, block_size, bits,
                       cb.contiguous(), packed, idx if keep_indices else None)


def make_random_layer(out_features: int, in_features: int, n_entries: int = 8,
                      block_size: int = 128, seed: int = 0, device="cpu",
                      std: float = 0.02) -> PackedLayer:
    """A layer of the same format with uniformly random index bytes and
    N(0, std^2) codebooks -- no quantile or argmin pass, so it is cheap to
    make on a profiled device (the kernels do the same work for any bytes)."""
    device = torch.device(device)
    gen = torch.Generator(device=device).manual_seed(int(seed))
    total = out_features * in_features
    nb = -(-total // block_size)
    bits = host_pack.bits_for_entries(n_entries)
    packed = torch.randint(0, 256, (host_pack.packed_nbytes(nb * block_size, bits),),
                           generator=gen, device=device, dtype=torch.uint8)
    cb = torch.randn(nb, n_entries, generator=gen, device=device) * std
    return PackedLayer(out_features, in_features, n_entries, block_size, bits, cb, packed, None)


def make_activation(k: int, m: int = 1, seed: int = 1000, device="cpu",
                    dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """x ~ N(0, 1) of shape (m, k), drawn in fp32 then cast."""
    gen = torch.Generator(device=torch.device(device)).manual_seed(int(seed))
    return torch.randn(m, k, generator=gen, device=device, dtype=torch.float32).to(dtype)


def layer_bytes(n: int, k: int, n_entries: int, block_size: int, m: int = 1,
                x_bytes: int = 2, y_bytes: int = 4) -> int:
    """Algorithmic HBM bytes of one GEMV: packed stream + codebooks + x + y."""
    bits = host_pack.bits_for_entries(n_entries)
    total = n * k
    num_blocks = math.ceil(total / block_size)
    return (host_pack.packed_nbytes(num_blocks * block_size, bits)
            + num_blocks * n_entries * 4 + m * k * x_bytes + m * n * y_bytes)
