"""PackedLinear: drop-in for the reference's packed NativeBit linear layer.

Mirrors inference/triton_kernel.py:223-286: the same buffers
(``packed_indices`` flat uint8 stream, ``codebook`` (num_blocks, n_entries)
float32), the same ``out_features`` / ``in_features`` attributes, the same
``from_packed(indices_np, codebook_np, weight_shape, device)`` constructor and
a ``forward`` that takes any leading dimensions and returns float32 by
default.  Differences, all deliberate:

* up to 16 rows run the fused dequant-GEMV kernels with x read as fp32 and
  the exact fp32 codebook values (the reference's batch-1 arithmetic, for
  bf16 and fp16 x too); more rows of bf16 activations run the packed MFMA
  prefill kernels (bf16-rounded codebook values, the reference's bf16 path
  of eval_ppl.py:149-174 -- its fp32 batched branch rejects bf16 x); more
  rows of fp32 x run the same MFMA kernels in three bf16 passes over the hi
  and lo parts of x and W (fp32-level products); other formats gather W on
  the device with the format kernel and multiply it densely, as the
  reference's batched branch does; nothing falls back silently -- a failure raises
  NativeBitError (the reference swallows every exception,
  triton_kernel.py:252);
* bit width, entries per block and block size are attributes (defaults 3, 8
  and 128, the reference's constants, triton_kernel.py:18-19);
* ``out_dtype`` may be bfloat16 for callers that keep activations in bf16.
"""
from __future__ import annotations

import numpy as np
import torch

from . import ops

BS = 128  # weights per codebook block (inference/triton_kernel.py:18)
NE = 8    # codebook entries per block (inference/triton_kernel.py:19)

MAX_GEMV_ROWS = 16


class PackedLinear(torch.nn.Module):
    """y = x @ W.T with W held as packed indices + per-block codebooks."""

    def __init__(self, packed_indices: torch.Tensor, codebook: torch.Tensor,
                 out_features: int, in_features: int, block_size: int = BS,
                 bits: int | None = None, out_dtype: torch.dtype = torch.float32):
        super().__init__()
        self.register_buffer("packed_indices", packed_indices)  # flat uint8 stream
        self.register_buffer("codebook", codebook)              # (num_blocks, n_entries)
        self.out_features = int(out_features)
        self.in_features = int(in_features)
        self.block_size = int(block_size)
        self.n_entries = int(codebook.shape[1])
        self.bits = int(bits) if bits is not None else ops.bits_for_entries(self.n_entries)
        self.out_dtype = out_dtype
        total = self.out_features * self.in_features
        need_blocks = -(-total // self.block_size)
        if codebook.shape[0] != need_blocks:
            raise ValueError(f"codebook has {codebook.shape[0]} blocks; "
                             f"{self.out_features}x{self.in_features} at block "
                             f"{self.block_size} needs {need_blocks}")
        # the kernels read the stream of every (zero-padded) block
        need = ops.packed_nbytes(need_blocks * self.block_size, self.bits)
        if packed_indices.numel() < need:
            raise ValueError(f"packed_indices has {packed_indices.numel()} bytes, "
                             f"{need} needed")

    def _standard(self) -> bool:
        """The format of the MFMA prefill kernels: 3-bit, 8 entries, blocks of
        128 along whole rows."""
        return (self.bits == 3 and self.n_entries == NE and self.block_size == BS
                and self.in_features % BS == 0)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        if x.dim() == 0 or shape[-1] != self.in_features:
            raise ValueError(f"x last dim must be {self.in_features}, got {tuple(shape)}")
        x_flat = x.reshape(-1, self.in_features)
        M = x_flat.shape[0]
        if x_flat.dtype != torch.float32 and (M <= MAX_GEMV_ROWS or
                                              x_flat.dtype != torch.bfloat16):
            # up to 16 rows, any float type is read as fp32 against the exact
            # fp32 codebook values, as the reference's batch-1 kernels compute
            # (.to(tl.float32), triton_kernel.py:46, 174-183)
            x_flat = x_flat.to(torch.float32)
        N, K = self.out_features, self.in_features
        if M <= MAX_GEMV_ROWS:
            y = ops.gemv(x_flat, self.packed_indices, self.codebook, N, K, bits=self.bits,
                         block_size=self.block_size, out_dtype=self.out_dtype)
        elif x_flat.dtype == torch.bfloat16 and self._standard():
            # the bf16 batched form (eval_ppl.py:149-174): the packed MFMA kernels
            y = ops.gemm_prefill(x_flat, self.packed_indices, self.codebook, N, K,
                                 out_dtype=self.out_dtype)
        elif self._standard():
            # the reference's fp32 batched branch (triton_kernel.py:258-275) on
            # the packed MFMA kernels: three bf16 passes over the hi / lo parts
            # of x and of the exact fp32 weights, W never materialised
            y = ops.gemm_prefill_f32(x_flat.contiguous(), self.packed_indices, self.codebook,
                                     N, K).to(self.out_dtype)
        else:
            # the reference's batched branch as it computes it (triton_kernel.py:
            # 258-275): W gathered on the device at x's precision by the format
            # kernel (exact fp32 copies of the codebook entries, or their bf16
            # rounding), then one dense GEMM
            w = ops.dequant(self.packed_indices, self.codebook, N * K, self.bits,
                            self.block_size, x_flat.dtype).view(N, K)
            y = (x_flat @ w.T).to(self.out_dtype)
        return y.reshape(*shape[:-1], N)

    @staticmethod
    def from_packed(indices_np, codebook_np, weight_shape, device="cuda",
                    block_size: int = BS) -> "PackedLinear":
        """Build from unpacked uint8 indices (as read from a .nbpack.npz).

        Like the reference (triton_kernel.py:277-286) the indices are moved to
        the device and packed there (nb_pack kernel).
        """
        idx = torch.from_numpy(np.ascontiguousarray(indices_np, dtype=np.uint8)).to(device)
        cb = torch.from_numpy(np.ascontiguousarray(codebook_np, dtype=np.float32)).to(device)
        bits = ops.bits_for_entries(cb.shape[1])
        packed = ops.pack(idx, bits)
        return PackedLinear(packed, cb, int(weight_shape[0]), int(weight_shape[1]),
                            block_size=block_size, bits=bits)

    @staticmethod
    def from_stream(packed_np, codebook_np, weight_shape, device="cuda",
                    block_size: int = BS, bits: int | None = None) -> "PackedLinear":
        """Build directly from an already-packed stream (no unpack/repack)."""
        packed = torch.from_numpy(np.ascontiguousarray(packed_np, dtype=np.uint8)).to(device)
        cb = torch.from_numpy(np.ascontiguousarray(codebook_np, dtype=np.float32)).to(device)
        return PackedLinear(packed, cb, int(weight_shape[0]), int(weight_shape[1]),
                            block_size=block_size, bits=bits)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bits={self.bits}, n_entries={self.n_entries}, block_size={self.block_size}")
