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
from . import pack as host_pack

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


def block_codebooks(w: torch.Tensor, n_entries: int, block_size: int) -> torch.Tensor:
    """Per-block quantile codebooks of the flat weights ``w``:
    (ceil(total / block_size), n_entries) fp32, torch.quantile(w_block,
    linspace(0, 1, n_entries)) per block (nativebit/codebook_utils.py:6-22,
    nativebit/layers.py:76), the last block over the weights that exist."""
    _require_cuda("w", w)
    if w.dtype != torch.float32:
        raise TypeError("w must be float32")
    w = w.contiguous().reshape(-1)
    nb = -(-w.numel() // block_size)
    out = torch.empty(nb, n_entries, dtype=torch.float32, device=w.device)
    _lib.check(_lib.load().nb_block_codebooks(w.data_ptr(), w.numel(), block_size, n_entries,
                                              out.data_ptr(), _stream(w)))
    return out


def quantize_pack(w: torch.Tensor, codebook: torch.Tensor, block_size: int,
                  bits: int | None = None) -> torch.Tensor:
    """Nearest-entry indices of the flat weights ``w`` against per-block
    ``codebook`` (num_blocks, n_entries), first entry on ties, packed
    LSB-first (quantize_weight + pack_indices_3bit, inference/pack.py:21-57)
    by one kernel: uint8 stream of packed_nbytes(num_blocks * block_size,
    bits) bytes."""
    for name, t in (("w", w), ("codebook", codebook)):
        _require_cuda(name, t)
    _same_device(w, codebook)
    if w.dtype != torch.float32 or codebook.dtype != torch.float32:
        raise TypeError("w and codebook must be float32")
    if codebook.dim() != 2:
        raise ValueError("codebook must be (num_blocks, n_entries)")
    w = w.contiguous().reshape(-1)
    codebook = codebook.contiguous()
    num_blocks, n_entries = codebook.shape
    if bits is None:
        bits = host_pack.bits_for_entries(n_entries)
    out = torch.empty(packed_nbytes(num_blocks * block_size, bits), dtype=torch.uint8,
                      device=w.device)
    _lib.check(_lib.load().nb_quantize_pack(w.data_ptr(), w.numel(), codebook.data_ptr(),
                                            num_blocks, n_entries, block_size, bits,
                                            out.data_ptr(), _stream(w)))
    return out


class GemvBatch:
    """Many independent 3-bit GEMVs in one launch.

    items: sequence of (x, packed, codebook, y, N, K) or (x, packed,
    codebook, y, N, K, form), packed/codebook a 3-bit / 8-entry / block-128
    layer and y an (N,) float32 or bfloat16 output.  ``form`` (a dict, all
    keys optional) selects the fused activation and output forms of
    nb_batch_item:

    * ``x``: "bf16" (default; x is (K,) bfloat16), ("rmsnorm", w, eps) (x is
      the (K,) float32 residual stream, the activations are
      bf16((x / sqrt(mean(x^2) + eps)) * w), generate_torch.py:29-38) or
      "silu_mul" (x is the (2K,) float32 gate | up vector, the activations
      are bf16(silu(gate) * up), generate_torch.py:116-117);
    * ``y``: "store" (default), "add" (y += result, float32 y; the
      residual add, generate_torch.py:128-132) or "silu_pairs" (rows
      alternate gate and up: y is the (N/2,) bfloat16 vector
      silu(gate) * up, generate_torch.py:116-117; one item per batch).

    ``m`` > 1 (up to 16) makes every item a skinny GEMM over m activation
    rows (nb_gemm_skinny_batched): x is an (m, K) bfloat16 matrix and y an
    (m, N) matrix, both contiguous; only the plain bf16 activation form is
    available then (the output may still be "add").

    ``layout="quad"`` (m <= 4, K >= 2048): every item's packed / codebook
    are the row-quad layout of its layer (``quad_layout``), run by
    nb_gemm_skinny_quad_batched.  ``layout="tile"`` (m > 1): every item's
    packed / codebook are the tile layout of its layer (``tile_layout``),
    run by nb_gemm_skinny_tile_batched.  ``layout="sel"`` (m == 1): every
    item's packed is the selector-ordered unit layout of its stream
    (``stream_layout``; codebook unchanged), run by nb_gemv_batched_sel with
    every activation and output form.

    The device table is built once here; each run() enqueues one launch on
    torch's current stream (graph-capturable).  The tensors are referenced
    by pointer: keep them alive and in place.
    """

    def __init__(self, items, m: int = 1, layout: str = "rows"):
        if not 1 <= m <= 16:
            raise ValueError(f"m={m} outside 1..16")
        if layout not in ("rows", "quad", "tile", "sel"):
            raise ValueError(f"unknown layout {layout!r}")
        if layout == "sel" and m != 1:
            raise ValueError("the selector-ordered layout is for m == 1 (nb_gemv_batched_sel)")
        if layout == "quad" and m > 4:
            raise ValueError(f"the row-quad kernel takes m <= 4 (got {m})")
        if layout == "tile" and m < 2:
            raise ValueError("the tile layout is for m > 1 (the skinny kernel)")
        self.m = int(m)
        self.layout = layout
        self.items = list(items)
        n = len(self.items)
        self._arr = (_lib.BatchItem * max(n, 1))()
        self._keep = []
        y_dt = None
        for i, item in enumerate(self.items):
            x, packed, cb, y, N, K = item[:6]
            form = item[6] if len(item) > 6 else {}
            for name, t in (("x", x), ("packed", packed), ("codebook", cb), ("y", y)):
                _require_cuda(name, t)
            xf = form.get("x", "bf16")
            if m > 1 and xf != "bf16":
                raise ValueError(f"item {i}: m > 1 takes bf16 activations only")
            norm_w, eps = None, 0.0
            if xf == "bf16":
                x_mode, x_dt, x_n = _lib.NB_X_BF16, torch.bfloat16, K
            elif xf == "silu_mul":
                x_mode, x_dt, x_n = _lib.NB_X_SILU_MUL, torch.float32, 2 * K
            elif isinstance(xf, tuple) and xf[0] == "rmsnorm":
                x_mode, x_dt, x_n = _lib.NB_X_RMSNORM, torch.float32, K
                norm_w, eps = xf[1], float(xf[2])
                _require_cuda("norm weight", norm_w)
                if norm_w.dtype != torch.float32 or norm_w.numel() != K or \
                        not norm_w.is_contiguous():
                    raise TypeError(f"item {i}: norm weight must be a contiguous ({K},) float32 tensor")
                self._keep.append(norm_w)
            else:
                raise ValueError(f"item {i}: unknown activation form {xf!r}")
            if x.dtype != x_dt or x.numel() != m * x_n or not x.is_contiguous():
                shape = f"({m}, {x_n})" if m > 1 else f"({x_n},)"
                raise TypeError(f"item {i}: x must be a contiguous {shape} {x_dt} tensor")
            yf = form.get("y", "store")
            if yf not in ("store", "add", "silu_pairs"):
                raise ValueError(f"item {i}: unknown output form {yf!r}")
            y_mode = {"store": _lib.NB_Y_STORE, "add": _lib.NB_Y_ADD,
                      "silu_pairs": _lib.NB_Y_SILU_PAIRS}[yf]
            if yf == "add" and y.dtype != torch.float32:
                raise TypeError(f"item {i}: y += result needs a float32 y")
            if yf == "silu_pairs":
                if m != 1 or len(self.items) != 1:
                    raise ValueError("the silu_pairs output form takes one item of one row")
                if y.dtype != torch.bfloat16 or y.numel() * 2 != N or not y.is_contiguous():
                    raise ValueError(f"item {i}: silu_pairs writes a contiguous ({N // 2},) "
                                     "bfloat16 y")
            if packed.dtype != torch.uint8 or cb.dtype != torch.float32:
                raise TypeError(f"item {i}: packed must be uint8 and codebook float32")
            if layout == "tile":
                nblk = (N + 15) // 16 * 16 * ((K // 128 + 3) // 4 * 4)
            else:
                nblk = ((N + 3) // 4 * 4 if layout == "quad" else N) * K // 128
            if cb.shape != (nblk, 8) or packed.numel() < nblk * 48:
                what = {"quad": "row-quad layout of a", "tile": "tile layout of a"}.get(layout, "a")
                raise ValueError(f"item {i}: not {what} 3-bit / 8-entry / block-128 {N}x{K} "
                                 "layer")
            if layout == "quad" and K < 2048:
                raise ValueError(f"item {i}: the row-quad kernel needs K >= 2048 (got {K})")
            if yf != "silu_pairs" and (y.numel() != m * N or y.dtype not in _DT or
                                       not y.is_contiguous()):
                shape = f"({m}, {N})" if m > 1 else f"({N},)"
                raise ValueError(f"item {i}: y must be a contiguous {shape} float32/bfloat16 tensor")
            if y_dt is None:
                y_dt = y.dtype
            elif y.dtype != y_dt:
                raise TypeError("all outputs of a batch share one dtype")
            self._arr[i] = _lib.BatchItem(x.data_ptr(), packed.data_ptr(), cb.data_ptr(),
                                          y.data_ptr(), int(N), int(K), x_mode, y_mode,
                                          norm_w.data_ptr() if norm_w is not None else None,
                                          eps, 0)
        self.y_dtype = y_dt or torch.float32
        lib = _lib.load()
        nbytes = int(lib.nb_gemv_batch_table_bytes(n))
        host = torch.zeros(max(nbytes, 8), dtype=torch.uint8)
        _lib.check(lib.nb_gemv_batch_plan(self._arr, n, host.data_ptr(), nbytes))
        dev = self.items[0][0].device if n else torch.device("cuda")
        self.table = host.to(dev)
        self.count = n

    def run(self):
        stream = ctypes.c_void_p(torch.cuda.current_stream(self.table.device).cuda_stream)
        lib = _lib.load()
        if self.layout == "quad":
            _lib.check(lib.nb_gemm_skinny_quad_batched(self._arr, self.table.data_ptr(),
                                                       self.count, self.m, _DT[self.y_dtype],
                                                       stream))
        elif self.layout == "tile":
            _lib.check(lib.nb_gemm_skinny_tile_batched(self._arr, self.table.data_ptr(),
                                                       self.count, self.m, _DT[self.y_dtype],
                                                       stream))
        elif self.layout == "sel":
            _lib.check(lib.nb_gemv_batched_sel(self._arr, self.table.data_ptr(), self.count,
                                               _DT[self.y_dtype], stream))
        elif self.m == 1:
            _lib.check(lib.nb_gemv_batched(self._arr, self.table.data_ptr(), self.count,
                                           _DT[self.y_dtype], stream))
        else:
            _lib.check(lib.nb_gemm_skinny_batched(self._arr, self.table.data_ptr(), self.count,
                                                  self.m, _DT[self.y_dtype], stream))


def quad_layout(packed: torch.Tensor, codebook: torch.Tensor, N: int, K: int):
    """The row-quad layout of a 3-bit / 8-entry / block-128 N x K layer
    (nb_quad_layout): the same blocks, rows taken four at a time (N rounded
    up with zero blocks), the four rows' blocks of one column block side by
    side.  Returns (qpacked uint8, qcodebook (ceil(N/4)*4*K/128, 8) float32)
    on the layer's device, for GemvBatch(..., layout="quad")."""
    for name, t in (("packed", packed), ("codebook", codebook)):
        _require_cuda(name, t)
    _same_device(packed, codebook)
    if packed.dtype != torch.uint8 or codebook.dtype != torch.float32:
        raise TypeError("packed must be uint8 and codebook float32")
    if K % 128 or codebook.shape != (N * K // 128, 8) or \
            packed.numel() < packed_nbytes(N * K, 3):
        raise ValueError(f"not a 3-bit / 8-entry / block-128 {N}x{K} layer")
    if not packed.is_contiguous() or not codebook.is_contiguous():
        raise ValueError("packed and codebook must be contiguous")
    rows = (N + 3) // 4 * 4
    lib = _lib.load()
    qp = torch.empty(int(lib.nb_quad_layout_bytes(N, K)), dtype=torch.uint8, device=packed.device)
    qc = torch.empty((rows * K // 128, 8), dtype=torch.float32, device=packed.device)
    _lib.check(lib.nb_quad_layout(packed.data_ptr(), codebook.data_ptr(), N, K, qp.data_ptr(),
                                  qc.data_ptr(), _stream(packed)))
    return qp, qc


def tile_layout(packed: torch.Tensor, codebook: torch.Tensor, N: int, K: int):
    """The tile layout of a 3-bit / 8-entry / block-128 N x K layer
    (nb_tile_layout): tiles of 16 rows x 4 column blocks (rows and column
    blocks padded with zero blocks), each stored as the skinny kernel's LDS
    slot holds it, indices in selector order.  Returns (tpacked uint8,
    tcodebook (tiles * 64, 8) float32) on the layer's device, for
    GemvBatch(..., layout="tile")."""
    for name, t in (("packed", packed), ("codebook", codebook)):
        _require_cuda(name, t)
    _same_device(packed, codebook)
    if packed.dtype != torch.uint8 or codebook.dtype != torch.float32:
        raise TypeError("packed must be uint8 and codebook float32")
    if N < 0 or K <= 0 or K % 128 or codebook.shape != (N * K // 128, 8) or \
            packed.numel() < packed_nbytes(N * K, 3):
        raise ValueError(f"not a 3-bit / 8-entry / block-128 {N}x{K} layer")
    if not packed.is_contiguous() or not codebook.is_contiguous():
        raise ValueError("packed and codebook must be contiguous")
    lib = _lib.load()
    nbytes = int(lib.nb_tile_layout_bytes(N, K))
    tp = torch.empty(nbytes, dtype=torch.uint8, device=packed.device)
    tc = torch.empty((nbytes // 48, 8), dtype=torch.float32, device=packed.device)
    _lib.check(lib.nb_tile_layout(packed.data_ptr(), codebook.data_ptr(), N, K, tp.data_ptr(),
                                  tc.data_ptr(), _stream(packed)))
    return tp, tc


def stream_layout(packed: torch.Tensor, N: int, K: int, out: torch.Tensor | None = None):
    """The selector-ordered unit layout of the 3-bit stream of an N x K layer
    (nb_stream_layout): the same N*K*3/8 bytes, each 12-byte unit's bits
    placed so that the batched kernels take its selectors with one shift and
    one mask each.  The codebook is unchanged.  Returns the new uint8 stream
    (``out`` if given; ``out`` may be ``packed`` itself), for
    GemvBatch(..., layout="sel")."""
    _require_cuda("packed", packed)
    if packed.dtype != torch.uint8 or not packed.is_contiguous():
        raise TypeError("packed must be a contiguous uint8 tensor")
    if N < 0 or K <= 0 or K % 128:
        raise ValueError(f"N={N}, K={K}: K must be a positive multiple of 128")
    nbytes = N * K * 3 // 8
    if packed.numel() < nbytes:
        raise ValueError(f"packed has {packed.numel()} bytes, {nbytes} needed")
    if out is None:
        out = torch.empty(nbytes, dtype=torch.uint8, device=packed.device)
    elif (out.dtype != torch.uint8 or not out.is_contiguous() or out.numel() < nbytes or
          out.device != packed.device):
        raise ValueError(f"out must be a contiguous uint8 tensor of >= {nbytes} bytes on "
                         f"{packed.device}")
    lib = _lib.load()
    _lib.check(lib.nb_stream_layout(packed.data_ptr(), out.data_ptr(), N, K, _stream(packed)))
    return out


def gemm_prefill(x: torch.Tensor, packed: torch.Tensor, codebook: torch.Tensor, N: int,
                 K: int, out_dtype: torch.dtype = torch.bfloat16,
                 out: torch.Tensor | None = None, path: str = "auto") -> torch.Tensor:
    """y = x @ bf16(W).T for a 3-bit / 8-entry / block-128 packed W (N x K);
    x (M, K) bfloat16, row-contiguous, fp32 accumulation.

    ``path``: "auto" (nb_gemm_prefill_split: the hand-written MFMA kernel,
    the packed weight dequantized into LDS tiles; a layer whose tile grid
    would leave CUs idle -- few tokens, narrow layers -- is split over K
    ranges, with fp32 partial products in a workspace taken from torch's
    allocator and one reduction launch) or "fused" (nb_gemm_prefill: the same
    kernel in one launch over all of K, no workspace)."""
    for name, t in (("x", x), ("packed", packed), ("codebook", codebook)):
        _require_cuda(name, t)
    _same_device(x, packed, codebook)
    if x.dim() != 2 or x.shape[1] != K or x.dtype != torch.bfloat16 or x.stride(1) != 1:
        raise ValueError(f"x must be a row-contiguous (M, {K}) bfloat16 tensor")
    if x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    if codebook.shape != (N * K // 128, 8) or codebook.dtype != torch.float32:
        raise ValueError("codebook must be (N*K/128, 8) float32")
    if packed.dtype != torch.uint8 or packed.numel() < packed_nbytes(N * K, 3):
        raise ValueError("packed must hold the 3-bit stream of N*K indices")
    M = x.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=x.device)
    elif out.shape != (M, N) or out.dtype not in _DT or out.stride(1) != 1:
        raise ValueError("out must be (M, N), row-contiguous")
    if path not in ("auto", "fused"):
        raise ValueError(f"unknown prefill path {path!r}")
    lib = _lib.load()
    if path == "auto":
        nbytes = int(lib.nb_gemm_prefill_split_ws_bytes(M, N, K))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device) if nbytes else None
        _lib.check(lib.nb_gemm_prefill_split(
            x.data_ptr(), x.stride(0), packed.data_ptr(), codebook.data_ptr(), out.data_ptr(),
            _DT[out.dtype], out.stride(0), M, N, K, ws.data_ptr() if nbytes else None, nbytes,
            _stream(x)))
        return out
    _lib.check(lib.nb_gemm_prefill(
        x.data_ptr(), x.stride(0), packed.data_ptr(), codebook.data_ptr(), out.data_ptr(),
        _DT[out.dtype], out.stride(0), M, N, K, _stream(x)))
    return out



def gemm_prefill_f32(x: torch.Tensor, packed: torch.Tensor, codebook: torch.Tensor, N: int,
                     K: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """y = x @ W.T for fp32 x (M, K) against the exact fp32 codebook values of
    a 3-bit / 8-entry / block-128 packed W (N x K), y fp32 (M, N):
    nb_gemm_prefill_f32, three bf16 MFMA passes over the hi / lo parts of x
    and W (each product to within 2^-16 of its size), the packed weight
    dequantized into LDS tiles, never materialised; a workspace from torch's
    allocator."""
    for name, t in (("x", x), ("packed", packed), ("codebook", codebook)):
        _require_cuda(name, t)
    _same_device(x, packed, codebook)
    if x.dim() != 2 or x.shape[1] != K or x.dtype != torch.float32 or x.stride(1) != 1:
        raise ValueError(f"x must be a row-contiguous (M, {K}) float32 tensor")
    if codebook.shape != (N * K // 128, 8) or codebook.dtype != torch.float32:
        raise ValueError("codebook must be (N*K/128, 8) float32")
    if packed.dtype != torch.uint8 or packed.numel() < packed_nbytes(N * K, 3):
        raise ValueError("packed must hold the 3-bit stream of N*K indices")
    M = x.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=x.device)
    elif out.shape != (M, N) or out.dtype != torch.float32 or out.stride(1) != 1:
        raise ValueError("out must be (M, N) float32, row-contiguous")
    lib = _lib.load()
    nbytes = int(lib.nb_gemm_prefill_f32_ws_bytes(M, N, K))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
    _lib.check(lib.nb_gemm_prefill_f32(
        x.data_ptr(), x.stride(0), packed.data_ptr(), codebook.data_ptr(), out.data_ptr(),
        out.stride(0), M, N, K, ws.data_ptr(), nbytes, _stream(x)))
    return out

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
            block_size: int, out_dtype: torch.dtype = torch.float32,
            out: torch.Tensor | None = None) -> torch.Tensor:
    """Flat W[:total] = codebook[i // block_size][index i] (device); into
    ``out`` (contiguous, >= total elements of out_dtype) when given."""
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
    if out is None:
        w = torch.empty(total, dtype=out_dtype, device=packed.device)
    else:
        if (out.dtype != out_dtype or not out.is_contiguous() or out.numel() < total
                or out.device != packed.device):
            raise ValueError(f"out must be a contiguous {out_dtype} tensor of >= {total} "
                             "elements on the stream's device")
        w = out
    _lib.check(_lib.load().nb_dequant(
        packed.data_ptr(), codebook.data_ptr(), w.data_ptr(), _DT[out_dtype], total,
        codebook.shape[0], bits, codebook.shape[1], block_size, _stream(packed)))
    return w
