"""CPU oracle for NativeBit's packed-weight path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker.  The product
(``nativebit_amd``) never imports it: its kernels run on the GPU or raise.

Two layers:

* ``liboracle.so`` (``nb_oracle.c``): per-bit bitstream pack/unpack, the
  3-bit group packer, the exact gather dequant, fp64 brute-force matmul, the
  reference CUDA kernel's fp32 accumulation order, and nearest-entry
  quantization.  Built by ``make -C oracle``.
* torch-on-CPU restatements of the reference's two dequant+matmul paths,
  used as the CPU baseline and as a second GEMV reference:
    - ``torch_packed_linear_f32``: PackedLinear's batched branch
      (inference/triton_kernel.py:258-275) generalised to any bit width via
      the LSB-first stream.
    - ``torch_packed_linear_bf16``: the bf16 evaluation path
      (inference/eval_ppl.py:149-174): gather, ``.to(torch.bfloat16)``, bf16
      ``F.linear``.

How each function is pinned is listed in tests/test_oracle.py.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        raise RuntimeError(
            f"{_LIB_PATH} is missing: build it with `make -C oracle` "
            "(or __graft_entry__.build())")
    lib = ctypes.CDLL(_LIB_PATH)
    P = ctypes.c_void_p
    S = ctypes.c_size_t
    I = ctypes.c_int
    lib.oracle_packed_nbytes.argtypes = [S, I]
    lib.oracle_packed_nbytes.restype = S
    lib.oracle_pack.argtypes = [P, S, I, P]
    lib.oracle_unpack.argtypes = [P, S, I, P]
    lib.oracle_pack3_groups.argtypes = [P, S, P]
    lib.oracle_dequant.argtypes = [P, P, S, I, I, S, P]
    lib.oracle_round_bf16.argtypes = [ctypes.c_float]
    lib.oracle_round_bf16.restype = ctypes.c_float
    lib.oracle_matmul_f64.argtypes = [P, I, I, P, I, P]
    lib.oracle_matvec_3bit_k1.argtypes = [P, P, P, I, I, P]
    lib.oracle_quantize.argtypes = [P, S, P, S, I, I, P]
    _lib = lib
    return lib


def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


def packed_nbytes(count: int, bits: int) -> int:
    return int(_load().oracle_packed_nbytes(count, bits))


def pack(indices, bits: int) -> np.ndarray:
    """LSB-first bitstream of ``indices`` (uint8), zero padded."""
    idx = np.ascontiguousarray(np.asarray(indices, dtype=np.uint8).reshape(-1))
    out = np.zeros(max(packed_nbytes(idx.size, bits), 1), dtype=np.uint8)
    _load().oracle_pack(_ptr(idx), idx.size, bits, _ptr(out))
    return out[:packed_nbytes(idx.size, bits)]


def pack3_groups(indices) -> np.ndarray:
    """The 3-bit packer in the reference's bits24 form."""
    idx = np.ascontiguousarray(np.asarray(indices, dtype=np.uint8).reshape(-1))
    out = np.zeros(max(packed_nbytes(idx.size, 3), 1), dtype=np.uint8)
    _load().oracle_pack3_groups(_ptr(idx), idx.size, _ptr(out))
    return out[:packed_nbytes(idx.size, 3)]


def unpack(packed, count: int, bits: int) -> np.ndarray:
    p = np.ascontiguousarray(np.asarray(packed, dtype=np.uint8).reshape(-1))
    if p.size * 8 < count * bits:
        raise ValueError("packed buffer too short")
    out = np.zeros(max(count, 1), dtype=np.uint8)
    _load().oracle_unpack(_ptr(p), count, bits, _ptr(out))
    return out[:count]


def dequant(indices, codebook, block_size: int, total: int) -> np.ndarray:
    """Exact gather ``w[i] = cb[i // block_size][idx[i]]`` (fp32)."""
    idx = np.ascontiguousarray(np.asarray(indices, dtype=np.uint8).reshape(-1))
    cb = np.ascontiguousarray(np.asarray(codebook, dtype=np.float32))
    nb, ne = cb.shape
    if idx.size < total:
        raise ValueError("fewer indices than weights")
    if int(idx[:total].max(initial=0)) >= ne:
        raise ValueError("index out of codebook range")
    w = np.zeros(max(total, 1), dtype=np.float32)
    _load().oracle_dequant(_ptr(idx), _ptr(cb), nb, ne, block_size, total, _ptr(w))
    return w[:total]


def round_bf16(a) -> np.ndarray:
    """torch-style float32 -> bfloat16 (RNE) -> float32, element by element."""
    a = np.asarray(a, dtype=np.float32)
    f = _load().oracle_round_bf16
    return np.array([f(float(v)) for v in a.reshape(-1)], dtype=np.float32).reshape(a.shape)


def matmul_f64(x, w) -> np.ndarray:
    """``y = x @ w.T`` with every product and sum in fp64."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    w = np.ascontiguousarray(np.asarray(w, dtype=np.float32))
    if x.ndim == 1:
        x = x[None]
    M, K = x.shape
    N, K2 = w.shape
    assert K == K2
    y = np.zeros((M, N), dtype=np.float64)
    _load().oracle_matmul_f64(_ptr(x), M, K, _ptr(w), N, _ptr(y))
    return y


def matvec_3bit_k1(x, packed, codebook, N: int, K: int) -> np.ndarray:
    """The reference CUDA kernel's fp32 arithmetic in its own order."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32).reshape(-1))
    p = np.ascontiguousarray(np.asarray(packed, dtype=np.uint8).reshape(-1))
    cb = np.ascontiguousarray(np.asarray(codebook, dtype=np.float32))
    assert K % 128 == 0 and x.size == K and cb.shape[1] == 8
    y = np.zeros(N, dtype=np.float32)
    _load().oracle_matvec_3bit_k1(_ptr(x), _ptr(p), _ptr(cb), N, K, _ptr(y))
    return y


def quantize(weight, codebook, block_size: int) -> np.ndarray:
    """Squared-distance nearest entry per weight, first index on ties."""
    w = np.ascontiguousarray(np.asarray(weight, dtype=np.float32).reshape(-1))
    cb = np.ascontiguousarray(np.asarray(codebook, dtype=np.float32))
    nb, ne = cb.shape
    idx = np.zeros(nb * block_size, dtype=np.uint8)
    _load().oracle_quantize(_ptr(w), w.size, _ptr(cb), nb, ne, block_size, _ptr(idx))
    return idx


# ---------------------------------------------------------------------------
# torch-on-CPU restatements of the reference's dequant + matmul
# ---------------------------------------------------------------------------

def torch_unpack_indices(packed, num_blocks: int, block_size: int, bits: int):
    """Unpack to int64 ``(num_blocks, block_size)`` with torch ops.

    For 3 bits this is the reference's own sequence
    (inference/triton_kernel.py:262-269): bytes -> bits24 -> 8 shifts.  For
    other widths the same LSB-first stream is read with a per-bit gather.
    """
    import torch
    packed = torch.as_tensor(packed).reshape(-1).to(torch.int32)
    total_idx = num_blocks * block_size
    if bits == 3:
        n_groups = packed.shape[0] // 3
        g = packed[: n_groups * 3].reshape(n_groups, 3)
        bits24 = g[:, 0] | (g[:, 1] << 8) | (g[:, 2] << 16)
        idx = torch.zeros(n_groups, 8, dtype=torch.int64)
        for j in range(8):
            idx[:, j] = (bits24 >> (j * 3)) & 0x7
        return idx.reshape(-1)[:total_idx].reshape(num_blocks, block_size)
    pos = torch.arange(total_idx, dtype=torch.int64) * bits
    idx = torch.zeros(total_idx, dtype=torch.int64)
    for b in range(bits):
        p = pos + b
        bit = (packed[p // 8].to(torch.int64) >> (p % 8)) & 1
        idx |= bit << b
    return idx.reshape(num_blocks, block_size)


def torch_dequant(packed, codebook, out_features: int, in_features: int,
                  block_size: int, bits: int):
    """``codebook[block_idx, indices]`` trimmed to (out, in), fp32."""
    import torch
    codebook = torch.as_tensor(codebook)
    num_blocks = codebook.shape[0]
    idx = torch_unpack_indices(packed, num_blocks, block_size, bits)
    block_idx = torch.arange(num_blocks).unsqueeze(1)
    total = out_features * in_features
    w = codebook[block_idx, idx].reshape(-1)[:total]
    return w.reshape(out_features, in_features)


def torch_packed_linear_f32(x, packed, codebook, out_features: int,
                            in_features: int, block_size: int = 128, bits: int = 3):
    """PackedLinear's batched branch on CPU (triton_kernel.py:258-275)."""
    import torch
    w = torch_dequant(packed, codebook, out_features, in_features, block_size, bits)
    x = torch.as_tensor(x)
    x_flat = x.reshape(-1, in_features).to(torch.float32)
    return (x_flat @ w.T).reshape(*x.shape[:-1], out_features)


def torch_packed_linear_bf16(x, packed, codebook, out_features: int,
                             in_features: int, block_size: int = 128, bits: int = 3):
    """The bf16 evaluation path (inference/eval_ppl.py:149-174)."""
    import torch
    w = torch_dequant(packed, codebook, out_features, in_features, block_size, bits)
    w = w.to(torch.bfloat16)
    x = torch.as_tensor(x).to(torch.bfloat16)
    return torch.nn.functional.linear(x, w)
