"""GPU parity of the gfx950 kernels against the CPU oracle (run with -m gpu).

Bars (from the north star):
* unpack / pack / dequant: bit-exact (torch.equal / byte equality);
* GEMV: ||y - y_ref|| / ||y_ref|| <= 1e-3 against the fp64 brute force for
  fp32 arithmetic, <= 1e-2 against the reference's bf16 path (weights cast to
  bf16, inference/eval_ppl.py:149-174) for bf16 activations; golden cases
  with fp32-exact answers must match exactly.
"""
import ctypes

import numpy as np
import pytest
import torch

from nativebit_amd import PackedLinear, _lib, kernels, ops, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu

REL_F32 = 1e-3
REL_BF16 = 1e-2


def rel(a, b):
    a = np.asarray(a, dtype=np.float64).reshape(-1)
    b = np.asarray(b, dtype=np.float64).reshape(-1)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def note(msg):
    print(f"[case] {msg}", flush=True)


def random_layer(N, K, bits, ne, bs, seed):
    rng = np.random.default_rng(seed)
    total = N * K
    nb = -(-total // bs)
    idx = rng.integers(0, ne, nb * bs, dtype=np.uint8)
    cb = (rng.standard_normal((nb, ne)) * 0.02).astype(np.float32)
    return idx, O.pack(idx, bits), cb


# --------------------------------------------------------------------------
# bit-exact format kernels
# --------------------------------------------------------------------------

@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("n", [1, 7, 10, 1001, 100_003])
def test_unpack_pack_bit_exact(dev, bits, n):
    note(f"unpack/pack bits={bits} n={n}")
    rng = np.random.default_rng(bits * 7 + n)
    idx = rng.integers(0, 1 << bits, n, dtype=np.uint8)
    ref = O.pack(idx, bits)
    got = ops.pack(torch.from_numpy(idx).to(dev), bits)
    assert np.array_equal(got.cpu().numpy(), ref)
    back = ops.unpack(torch.from_numpy(ref).to(dev), n, bits)
    assert np.array_equal(back.cpu().numpy(), idx)


def test_golden_streams_on_gpu(dev, golden):
    for v in golden["bitstream"]:
        note(f"golden stream {v['name']}")
        got = ops.pack(torch.tensor(v["indices"], dtype=torch.uint8, device=dev), v["bits"])
        assert bytes(got.cpu().numpy()).hex() == v["hex"], v["name"]
        p = torch.from_numpy(np.frombuffer(bytes.fromhex(v["hex"]), np.uint8).copy()).to(dev)
        assert ops.unpack(p, len(v["indices"]), v["bits"]).tolist() == v["indices"]


@pytest.mark.parametrize("bits", [1, 3, 5, 8])
def test_codec_unaligned_pointers(dev, bits):
    """Streams and index arrays that start at an odd byte address (the
    per-element kernels) give the same bytes as aligned ones (the chunk
    kernels), tails included."""
    n = 32 * 37 + 11
    note(f"unaligned codec bits={bits} n={n}")
    rng = np.random.default_rng(bits)
    idx = rng.integers(0, 1 << bits, n, dtype=np.uint8)
    ref = O.pack(idx, bits)
    buf = torch.zeros(n + 1, dtype=torch.uint8, device=dev)
    buf[1:] = torch.from_numpy(idx).to(dev)
    assert np.array_equal(ops.pack(buf[1:], bits).cpu().numpy(), ref)
    sbuf = torch.zeros(ref.size + 1, dtype=torch.uint8, device=dev)
    sbuf[1:] = torch.from_numpy(ref).to(dev)
    assert np.array_equal(ops.unpack(sbuf[1:], n, bits).cpu().numpy(), idx)
    ne = 1 << bits
    cb = rng.standard_normal((-(-n // 64), ne)).astype(np.float32)
    w = ops.dequant(sbuf[1:], torch.from_numpy(cb).to(dev), n, bits, 64)
    assert np.array_equal(w.cpu().numpy(), O.dequant(idx, cb, 64, n))


@pytest.mark.parametrize("N,K,bits,ne,bs", [
    (6912, 2560, 3, 8, 128), (2560, 6912, 3, 8, 128), (100, 37, 3, 8, 128),
    (64, 512, 2, 4, 64), (64, 512, 4, 16, 256), (33, 65, 5, 20, 16), (17, 9, 3, 5, 8),
    (48, 640, 5, 20, 64), (40, 96, 8, 200, 32), (3, 100, 1, 2, 32), (7, 160, 6, 64, 96),
])
def test_dequant_bit_exact(dev, N, K, bits, ne, bs):
    note(f"dequant N={N} K={K} bits={bits} ne={ne} bs={bs}")
    idx, p, cb = random_layer(N, K, bits, ne, bs, N + K)
    ref = O.dequant(idx, cb, bs, N * K)
    pt, ct = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
    w32 = ops.dequant(pt, ct, N * K, bits, bs, torch.float32)
    assert np.array_equal(w32.cpu().numpy(), ref)
    w16 = ops.dequant(pt, ct, N * K, bits, bs, torch.bfloat16)
    assert torch.equal(w16.cpu(), torch.from_numpy(ref).to(torch.bfloat16))


@pytest.mark.parametrize("total,ne,bs,bits", [
    (6912 * 2560, 8, 128, 3), (1000, 8, 125, 3), (1001, 8, 128, 3), (777, 4, 64, 2),
    (4096, 16, 256, 4), (333, 5, 7, 3), (100, 2, 10, 1), (515, 200, 64, 8), (64, 8, 128, 3),
])
def test_quantize_pack_bit_exact(dev, total, ne, bs, bits):
    """GPU quantize-at-pack equals the oracle's quantize_weight restatement
    packed by the oracle, byte for byte -- with planted exact ties (weights
    at the midpoint of two entries, and equal entries) that must take the
    first index, and a padded tail block."""
    note(f"quantize_pack total={total} ne={ne} bs={bs} bits={bits}")
    rng = np.random.default_rng(total + ne)
    nb = -(-total // bs)
    w = (rng.standard_normal(total) * 0.02).astype(np.float32)
    cb = np.sort((rng.standard_normal((nb, ne)) * 0.02).astype(np.float32), axis=1)
    if ne >= 3:
        cb[::3, 1] = cb[::3, 2]                      # duplicate entries: first wins
    # midpoints of entries 0 and 1, exactly representable distance ties
    for i in range(0, total, 17):
        b = i // bs
        lo, hi = np.float32(cb[b, 0]), np.float32(cb[b, 1])
        w[i] = np.float32((lo + hi) / np.float32(2))
    ref = O.pack(O.quantize(w, cb, bs), bits)
    got = ops.quantize_pack(torch.from_numpy(w).to(dev), torch.from_numpy(cb).to(dev), bs, bits)
    assert got.numel() == ref.size
    assert np.array_equal(got.cpu().numpy(), ref)


@pytest.mark.parametrize("total,ne,bs", [
    (6912 * 2560, 8, 128), (1000, 8, 128), (777, 4, 64), (4096 + 17, 16, 256), (3000, 8, 1000),
    (55, 3, 5), (300, 1, 128), (1024, 256, 128), (2, 8, 128), (640, 2, 1024),
])
def test_block_codebooks_equal_torch_quantile(dev, total, ne, bs):
    """GPU per-block quantile codebooks equal torch.quantile on the CPU over
    the same blocks (the reference's init_codebook_percentile per block,
    codebook_utils.py:6-22, layers.py:76), bit for bit, tail block over the
    weights that exist; repeated values included."""
    note(f"block_codebooks total={total} ne={ne} bs={bs}")
    g = torch.Generator().manual_seed(total + ne)
    w = torch.randn(total, generator=g) * 0.02
    w[::7] = w[total // 2]                           # repeated values
    ref = synth.block_codebooks(w, total, ne, bs)
    got = ops.block_codebooks(w.to(dev), ne, bs).cpu()
    assert got.shape == ref.shape
    assert torch.equal(got, ref), int((got != ref).sum())


def test_quantize_pack_roundtrip_synth(dev):
    """The synthetic generator's torch quantization (squared distance argmin,
    per-block quantile codebooks) packed by nb_pack equals nb_quantize_pack
    on the same weights and codebooks."""
    N, K = 2560, 2560
    g = torch.Generator(device=dev).manual_seed(5)
    w = torch.randn(N * K, generator=g, device=dev) * 0.02
    cb = synth.block_codebooks(w, N * K, 8, 128)
    idx = synth.nearest_indices(w, N * K, cb, 128)
    assert torch.equal(ops.quantize_pack(w, cb, 128), ops.pack(idx, 3))


def test_reference_gather_equals_dequant(dev):
    """The reference's own torch unpack+gather (restated) equals nb_dequant."""
    N, K = 300, 2560
    idx, p, cb = random_layer(N, K, 3, 8, 128, 5)
    ref = O.torch_dequant(torch.from_numpy(p), torch.from_numpy(cb), N, K, 128, 3)
    got = ops.dequant(torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev), N * K, 3, 128)
    assert torch.equal(got.cpu().reshape(N, K), ref)


# --------------------------------------------------------------------------
# GEMV
# --------------------------------------------------------------------------

def run_gemv(dev, x, p, cb, N, K, bits, bs, out_dtype=torch.float32):
    return ops.gemv(x.to(dev), torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev),
                    N, K, bits=bits, block_size=bs, out_dtype=out_dtype)


def ref_weights(idx, cb, bs, N, K, xdt):
    """Dequantized W as the GEMV contract defines it: exact fp32 for fp32 x,
    rounded to bf16 (torch's cast, pinned in tests/test_oracle.py) for bf16 x."""
    w = O.dequant(idx, cb, bs, N * K).reshape(N, K)
    if xdt == torch.bfloat16:
        w = torch.from_numpy(w).to(torch.bfloat16).float().numpy()
    return w


def ref_gemv(x, idx, cb, bs, N, K):
    """fp64 brute force over exactly the operands the kernel multiplies."""
    w = ref_weights(idx, cb, bs, N, K, x.dtype)
    return O.matmul_f64(x.float().reshape(-1, K).numpy(), w)


def test_golden_gemv_exact(dev, golden):
    for g in golden["gemv"]:
        p = np.frombuffer(bytes.fromhex(g["packed_hex"]), np.uint8).copy()
        cb = np.array(g["codebook"], np.float32)
        for xdt in (torch.float32, torch.bfloat16):
            note(f"golden gemv {g['name']} x={xdt}")
            x = torch.tensor(g["x"], dtype=torch.float32).to(xdt)
            y = run_gemv(dev, x, p, cb, g["N"], g["K"], g["bits"], g["block_size"])
            assert y.cpu().tolist() == g["y"], (g["name"], xdt)


@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("N,K", [(6912, 2560), (2560, 6912), (2560, 2560), (7680, 2560)])
def test_gemv_3bit_2p2b_shapes(dev, N, K, xdt):
    note(f"gemv 3-bit N={N} K={K} x={xdt}")
    idx, p, cb = random_layer(N, K, 3, 8, 128, N * 3 + K)
    x = torch.randn(K, generator=torch.Generator().manual_seed(N)).to(xdt)
    y = run_gemv(dev, x, p, cb, N, K, 3, 128).cpu().numpy()
    ref = ref_gemv(x, idx, cb, 128, N, K)[0]
    assert rel(y, ref) <= REL_F32, rel(y, ref)
    # the reference kernel's own fp32 arithmetic (cuda_kernel.py:53-81) ...
    k1 = O.matvec_3bit_k1(x.float().numpy(), p, cb, N, K)
    if xdt == torch.bfloat16:
        # ... and the reference's bf16 path (eval_ppl.py:149-174) agree
        ref16 = O.torch_packed_linear_bf16(x, torch.from_numpy(p), torch.from_numpy(cb), N, K)
        assert rel(y, ref16.float().numpy()) <= REL_BF16
        assert rel(y, k1) <= REL_BF16
    else:
        assert rel(y, k1) <= REL_F32


@pytest.mark.parametrize("M", [2, 3, 4, 5, 8, 16])
@pytest.mark.parametrize("N,K", [(2560, 2560), (6912, 2560), (2560, 6912)])
def test_gemv_skinny_bf16(dev, M, N, K):
    """Config 2: M activation rows share one pass over the packed weights."""
    note(f"skinny gemv M={M} N={N} K={K}")
    idx, p, cb = random_layer(N, K, 3, 8, 128, M * 7 + N + K)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16)
    y = run_gemv(dev, x, p, cb, N, K, 3, 128).cpu().numpy()
    ref = ref_gemv(x, idx, cb, 128, N, K)
    assert y.shape == (M, N)
    for m in range(M):
        assert rel(y[m], ref[m]) <= REL_F32, (m, rel(y[m], ref[m]))


def test_gemv_strided_rows_bf16(dev):
    """x rows with a stride larger than K (a view into a wider buffer)."""
    N, K, M = 1000, 2560, 6
    idx, p, cb = random_layer(N, K, 3, 8, 128, 77)
    big = torch.randn(M, K + 64, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    x = big[:, :K]
    y = ops.gemv(x.to(dev), torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev), N, K)
    xv = big.to(dev)[:, :K]
    assert xv.stride(0) == K + 64
    y2 = ops.gemv(xv, torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev), N, K)
    ref = ref_gemv(x.contiguous(), idx, cb, 128, N, K)
    assert rel(y.cpu(), ref) <= REL_F32 and rel(y2.cpu(), ref) <= REL_F32


@pytest.mark.parametrize("M", [1, 4, 16])
def test_mfma_and_generic_agree_bf16(dev, M):
    """The MFMA kernel and the generic kernel (reached through a misaligned x)
    compute the same bf16-weight product."""
    N, K = 2560, 6912
    idx, p, cb = random_layer(N, K, 3, 8, 128, 500 + M)
    pt, ct = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16).to(dev)
    buf = torch.empty(M * K + 1, dtype=torch.bfloat16, device=dev)
    x_mis = buf[1:].view(M, K)
    x_mis.copy_(x)
    y_mfma = ops.gemv(x, pt, ct, N, K)
    y_gen = ops.gemv(x_mis, pt, ct, N, K)
    assert rel(y_gen.cpu(), y_mfma.cpu()) <= 1e-5


@pytest.mark.parametrize("ne,bs", [(4, 64), (4, 128), (4, 256), (8, 64), (8, 128),
                                   (8, 256), (16, 64), (16, 128), (16, 256)])
@pytest.mark.parametrize("N,K", [(6912, 2560), (2560, 6912)])
def test_gemv_bits_block_sweep(dev, ne, bs, N, K):
    bits = {4: 2, 8: 3, 16: 4}[ne]
    note(f"gemv sweep ne={ne} bs={bs} N={N} K={K}")
    idx, p, cb = random_layer(N, K, bits, ne, bs, ne * 1000 + bs + N)
    x = torch.randn(K, generator=torch.Generator().manual_seed(ne + bs)).to(torch.bfloat16)
    y = run_gemv(dev, x, p, cb, N, K, bits, bs).cpu().numpy()
    ref = ref_gemv(x, idx, cb, bs, N, K)[0]
    assert rel(y, ref) <= REL_F32


@pytest.mark.parametrize("N,K,bits,ne,bs,M", [
    (100, 37, 3, 8, 128, 1),     # ragged: blocks straddle rows
    (61, 300, 3, 8, 16, 3),
    (257, 1000, 4, 16, 64, 16),
    (64, 512, 3, 6, 128, 2),     # fewer entries than 2^bits
    (33, 65, 5, 20, 16, 5),
    (128, 256, 8, 256, 128, 1),  # unpacked uint8 indices
    (3000, 2560, 3, 8, 128, 4),
    (5, 8448, 3, 8, 128, 1),     # K above the fast kernel's limit
])
def test_gemv_generic_shapes(dev, N, K, bits, ne, bs, M):
    note(f"gemv generic N={N} K={K} bits={bits} ne={ne} bs={bs} M={M}")
    idx, p, cb = random_layer(N, K, bits, ne, bs, N * 13 + K)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(K))
    y = run_gemv(dev, x, p, cb, N, K, bits, bs).cpu().numpy()
    ref = O.matmul_f64(x.numpy(), O.dequant(idx, cb, bs, N * K).reshape(N, K))
    assert rel(y, ref) <= REL_F32


def test_fast_and_generic_agree(dev):
    """Same problem through both kernels: an x view misaligned to 16 bytes
    routes the 6912x2560 case to the generic kernel."""
    N, K = 6912, 2560
    idx, p, cb = random_layer(N, K, 3, 8, 128, 99)
    pt, ct = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
    x_fast = torch.randn(K, generator=torch.Generator().manual_seed(1)).to(dev)
    x_mis = torch.empty(K + 1, device=dev)
    x_mis[1:] = x_fast
    y_fast = ops.gemv(x_fast, pt, ct, N, K)
    y_slow = ops.gemv(x_mis[1:], pt, ct, N, K)       # 4-byte offset -> generic
    assert rel(y_slow.cpu(), y_fast.cpu()) <= 1e-5


def test_gemv_deterministic(dev):
    N, K = 6912, 2560
    idx, p, cb = random_layer(N, K, 3, 8, 128, 7)
    x = torch.randn(K).to(torch.bfloat16)
    a = run_gemv(dev, x, p, cb, N, K, 3, 128)
    b = run_gemv(dev, x, p, cb, N, K, 3, 128)
    assert torch.equal(a, b)


def test_gemv_bf16_output(dev):
    N, K = 2560, 2560
    idx, p, cb = random_layer(N, K, 3, 8, 128, 8)
    x = torch.randn(K)
    y32 = run_gemv(dev, x, p, cb, N, K, 3, 128, torch.float32)
    y16 = run_gemv(dev, x, p, cb, N, K, 3, 128, torch.bfloat16)
    assert torch.equal(y16.cpu(), y32.cpu().to(torch.bfloat16))


def test_gemv_k_zero_writes_zeros(dev):
    y = torch.full((4,), 7.0, device=dev)
    ops.gemv(torch.zeros(0, device=dev), torch.zeros(1, dtype=torch.uint8, device=dev),
             torch.zeros(0, 8, device=dev), 4, 0, out=y.reshape(1, 4))
    assert y.cpu().tolist() == [0.0] * 4


# --------------------------------------------------------------------------
# operator API (PackedLinear and the function-level mirror)
# --------------------------------------------------------------------------

def test_packed_linear_api(dev):
    N, K = 768, 2560
    idx, p, cb = random_layer(N, K, 3, 8, 128, 21)
    layer = PackedLinear.from_packed(idx.reshape(-1, 128), cb, (N, K), device=dev)
    assert torch.equal(layer.packed_indices.cpu(), torch.from_numpy(p))
    assert layer.out_features == N and layer.in_features == K
    # up to 16 rows: the GEMV kernels; more: the MFMA prefill kernels (bf16 x)
    # or the device gather + dense GEMM (fp32 x, the reference's batched branch)
    for xdt in (torch.float32, torch.bfloat16, torch.float16):
        for shape in [(K,), (1, K), (1, 1, K), (3, K), (2, 5, K), (40, K), (300, K),
                      (4, 100, K)]:
            note(f"PackedLinear x{shape} {xdt}")
            x = torch.randn(*shape, generator=torch.Generator().manual_seed(len(shape))).to(xdt)
            y = layer(x.to(dev))
            assert y.dtype == torch.float32 and y.shape == (*shape[:-1], N)
            # up to 16 rows every x is read as fp32 against the exact fp32
            # codebook values (the reference's batch-1 kernels); more rows of
            # bf16 x take the bf16 path, fp16 x is read as fp32
            rows = x.numel() // K
            xr = x if (xdt == torch.bfloat16 and rows > 16) else x.float()
            ref = ref_gemv(xr.reshape(-1, K), idx, cb, 128, N, K)
            assert rel(y.cpu().reshape(-1, N), ref) <= REL_F32


def test_packed_linear_other_format_batched(dev):
    """A 4-bit / 16-entry / block-64 layer with many rows: the device gather
    and a dense fp32 GEMM, equal to the fp64 brute force."""
    N, K, M = 300, 640, 70
    idx, p, cb = random_layer(N, K, 4, 16, 64, 41)
    layer = PackedLinear(torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev), N, K,
                         block_size=64)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(3))
    y = layer(x.to(dev))
    ref = O.matmul_f64(x.numpy(), O.dequant(idx, cb, 64, N * K).reshape(N, K))
    assert rel(y.cpu(), ref) <= REL_F32


def test_kernels_mirror(dev):
    N, K = 512, 2560
    idx, p, cb = random_layer(N, K, 3, 8, 128, 31)
    x = torch.randn(K)
    ref = O.matmul_f64(x.numpy(), O.dequant(idx, cb, 128, N * K).reshape(N, K))[0]
    pt, ct = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
    for fn in (kernels.dequant_matvec_3bit, kernels.dequant_matvec_3bit_cuda):
        y = fn(x.to(dev), pt, ct, N, K)
        assert y.shape == (N,) and rel(y.cpu(), ref) <= REL_F32
    # bf16 x: the reference's runtime arithmetic (x read as fp32, exact fp32
    # codebook values) -- within 1e-3 of the CUDA kernel's own fp32 order
    xb = x.to(torch.bfloat16)
    k1 = O.matvec_3bit_k1(xb.float().numpy(), p, cb, N, K)
    refb = O.matmul_f64(xb.float().numpy(), O.dequant(idx, cb, 128, N * K).reshape(N, K))[0]
    for fn in (kernels.dequant_matvec_3bit, kernels.dequant_matvec_3bit_cuda):
        yb = fn(xb.to(dev), pt, ct, N, K)
        assert yb.dtype == torch.float32
        assert rel(yb.cpu(), k1) <= 1e-3 and rel(yb.cpu(), refb) <= REL_F32
    # fp16 x is read as fp32, as the reference's Triton kernels do
    x16 = x.to(torch.float16)
    ref16 = O.matmul_f64(x16.float().numpy(), O.dequant(idx, cb, 128, N * K).reshape(N, K))[0]
    y16 = kernels.dequant_matvec_3bit(x16.to(dev), pt, ct, N, K)
    assert y16.dtype == torch.float32 and rel(y16.cpu(), ref16) <= REL_F32
    y8 = kernels.dequant_matvec(x.to(dev), torch.from_numpy(idx.reshape(-1, 128)).to(dev), ct, N, K)
    assert rel(y8.cpu(), ref) <= REL_F32
    assert torch.equal(kernels.pack_indices_to_3bit(torch.from_numpy(idx).to(dev)).cpu(),
                       torch.from_numpy(p))


def test_errors_raise_not_fallback(dev):
    from nativebit_amd import NativeBitError
    N, K = 64, 256
    idx, p, cb = random_layer(N, K, 3, 8, 128, 1)
    layer = PackedLinear.from_packed(idx, cb, (N, K), device=dev)
    with pytest.raises(ValueError):
        layer(torch.randn(3, K + 1, device=dev))
    with pytest.raises(ValueError):
        layer(torch.randn(3, K))                       # CPU tensor
    with pytest.raises(NativeBitError):
        ops.gemv(torch.randn(K, device=dev), layer.packed_indices, layer.codebook, N, K,
                 bits=9)


# --------------------------------------------------------------------------
# full 2.2B shape: all seven matmul shapes of a layer from the synthetic
# generator, and size-independent properties over the whole 26-layer model
# --------------------------------------------------------------------------

def test_synth_layer_all_shapes_vs_f64(dev):
    for j, (name, N, K) in enumerate(synth.LAYER_SHAPES):
        note(f"synth layer {name} {N}x{K}")
        lay = synth.make_layer(N, K, seed=100 + j, device=dev, keep_indices=True)
        x = synth.make_activation(K, seed=1000 + j, device=dev, dtype=torch.bfloat16)
        y = ops.gemv(x[0], lay.packed, lay.codebook, N, K).cpu().numpy()
        idx = lay.indices.cpu().numpy()
        cb = lay.codebook.cpu().numpy()
        assert np.array_equal(lay.packed.cpu().numpy(), O.pack(idx, 3))
        ref = ref_gemv(x.cpu(), idx, cb, 128, N, K)[0]
        assert rel(y, ref) <= REL_F32


def test_full_model_properties(dev):
    """26 layers x 7 matmuls at full size: unpack->pack round trip is the
    identity on every stream, and each GEMV is linear in x."""
    for layer in range(synth.N_LAYERS):
        for j, (name, N, K) in enumerate(synth.LAYER_SHAPES):
            lay = synth.make_layer(N, K, seed=layer * 7 + j, device=dev)
            idx = ops.unpack(lay.packed, N * K, 3)
            assert torch.equal(ops.pack(idx, 3), lay.packed)
            if name in ("q", "down"):
                note(f"linearity layer {layer} {name}")
                x1 = synth.make_activation(K, seed=layer, device=dev)[0]
                x2 = synth.make_activation(K, seed=layer + 500, device=dev)[0]
                y1 = ops.gemv(x1, lay.packed, lay.codebook, N, K)
                y2 = ops.gemv(x2, lay.packed, lay.codebook, N, K)
                y12 = ops.gemv(x1 + x2, lay.packed, lay.codebook, N, K)
                assert rel(y12.cpu(), (y1 + y2).cpu()) <= 1e-5


# --------------------------------------------------------------------------
# batched streaming GEMV (nb_gemv_batched)
# --------------------------------------------------------------------------

def test_batched_matches_single_and_f64(dev):
    """Mixed shapes, ragged N, an empty item, bf16 output: every item equals
    its own fp64 reference and the single-call nb_gemv."""
    shapes = [(2560, 2560), (100, 2560), (6912, 2560), (0, 2560), (2560, 6912), (17, 128),
              (1000, 6912), (16, 256)]
    items, refs, singles = [], [], []
    for i, (N, K) in enumerate(shapes):
        note(f"batched item {i} {N}x{K}")
        idx, p, cb = random_layer(max(N, 1), K, 3, 8, 128, 900 + i)
        x = torch.randn(K, generator=torch.Generator().manual_seed(i)).to(torch.bfloat16)
        pt, ct = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
        if N == 0:
            pt, ct = pt[:16].clone(), ct[:0].reshape(0, 8).contiguous()
        y = torch.full((N,), float("nan"), device=dev)
        items.append((x.to(dev), pt, ct, y, N, K))
        refs.append(ref_gemv(x, idx, cb, 128, N, K)[0] if N else None)
        singles.append(ops.gemv(x.to(dev), pt, ct, N, K) if N else None)
    batch = ops.GemvBatch(items)
    batch.run()
    for i, (x, pt, ct, y, N, K) in enumerate(items):
        if N == 0:
            continue
        assert rel(y.cpu(), refs[i]) <= REL_F32, (i, rel(y.cpu(), refs[i]))
        assert rel(y.cpu(), singles[i].cpu()) <= 1e-5
    # bf16 outputs and a second run over the same table are stable
    ys16 = [torch.empty(N, dtype=torch.bfloat16, device=dev) for (_, _, _, _, N, _) in items]
    b16 = ops.GemvBatch([(x, p, c, y16, N, K) for (x, p, c, _, N, K), y16 in zip(items, ys16)])
    b16.run()
    b16.run()
    for (x, p, c, y, N, K), y16 in zip(items, ys16):
        if N:
            assert torch.equal(y16.cpu(), y.cpu().to(torch.bfloat16))


def test_batched_full_model_layer(dev):
    """One layer's seven matmuls from the synthetic generator in one batch."""
    mats = []
    for j, (name, N, K) in enumerate(synth.LAYER_SHAPES):
        lay = synth.make_layer(N, K, seed=700 + j, device=dev, keep_indices=True)
        x = synth.make_activation(K, seed=800 + j, device=dev, dtype=torch.bfloat16)[0].contiguous()
        mats.append((lay, x, torch.empty(N, device=dev)))
    ops.GemvBatch([(x, l.packed, l.codebook, y, l.out_features, l.in_features)
                   for l, x, y in mats]).run()
    for l, x, y in mats:
        ref = ref_gemv(x.cpu(), l.indices.cpu().numpy(), l.codebook.cpu().numpy(), 128,
                       l.out_features, l.in_features)[0]
        assert rel(y.cpu(), ref) <= REL_F32


def _fused_activations(mode, x, w=None, eps=0.0):
    """bf16 activations of an x_mode, formed on the CPU in fp32 by the
    reference's expressions (RMSNorm: generate_torch.py:35-38; SwiGLU:
    116-117)."""
    x = x.detach().cpu().float()
    if mode == "rmsnorm":
        norm = torch.sqrt(x.pow(2).mean(-1, keepdim=True) + eps)
        a = x / norm * w.detach().cpu().float()
    else:
        K = x.numel() // 2
        a = torch.nn.functional.silu(x[:K]) * x[K:]
    return a.to(torch.bfloat16)


def test_batched_fused_forms(dev):
    """x_mode RMSNorm / SiLU*up and y_mode add in one launch, ragged N: each
    item equals the unfused sequence (activations formed by torch on the CPU,
    plain batched GEMV, residual add by torch) and the fp64 brute force over
    those activations.  Rounding the activations to bf16 may flip a few
    last bits where the sum of squares is accumulated in another order, so
    the fused-vs-unfused bar is rel 1e-3, not equality."""
    g = torch.Generator().manual_seed(77)
    eps = 1e-6
    cases = [("rmsnorm", 2560, 2560, "store"), ("silu_mul", 2560, 6912, "add"),
             ("rmsnorm", 6912, 2560, "add"), ("silu_mul", 100, 256, "store"),
             ("bf16", 1000, 2560, "add")]
    items, plain, refs, adds = [], [], [], []
    for i, (mode, N, K, yf) in enumerate(cases):
        note(f"fused item {i} {mode} {N}x{K} y={yf}")
        idx, p, cb = random_layer(N, K, 3, 8, 128, 1300 + i)
        pt, ct = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
        form = {"y": yf}
        if mode == "rmsnorm":
            x = torch.randn(K, generator=g) * 3
            w = 1 + 0.1 * torch.randn(K, generator=g)
            form["x"] = ("rmsnorm", w.to(dev), eps)
            a = _fused_activations(mode, x, w, eps)
        elif mode == "silu_mul":
            x = torch.randn(2 * K, generator=g) * 2
            form["x"] = "silu_mul"
            a = _fused_activations(mode, x)
        else:
            x = torch.randn(K, generator=g).to(torch.bfloat16)
            a = x
        y0 = torch.randn(N, generator=g) if yf == "add" else torch.zeros(N)
        y = y0.clone().to(dev) if yf == "add" else torch.full((N,), float("nan"), device=dev)
        items.append((x.to(dev), pt, ct, y, N, K, form))
        yp = torch.empty(N, device=dev)
        plain.append((a.to(dev), pt, ct, yp, N, K))
        refs.append(ref_gemv(a, idx, cb, 128, N, K)[0] + y0.double().numpy())
        adds.append(y0)
    ops.GemvBatch(items).run()
    ops.GemvBatch(plain).run()
    for i, (item, pl) in enumerate(zip(items, plain)):
        y, yp = item[3], pl[3]
        unfused = yp.cpu() + adds[i]
        assert rel(y.cpu(), unfused) <= 1e-3, (i, rel(y.cpu(), unfused))
        assert rel(y.cpu(), refs[i]) <= REL_F32, (i, rel(y.cpu(), refs[i]))


@pytest.mark.parametrize("N,K", [(2560, 2560), (7680, 2560), (13824, 2560), (2560, 6912),
                                 (1, 128), (5, 128), (1000, 384), (71, 8192), (333, 1280)])
@pytest.mark.parametrize("mode,yf", [("bf16", "store"), ("rmsnorm", "store"), ("bf16", "add"),
                                     ("silu_mul", "add"), ("rmsnorm", "add")])
def test_single_item_rows_kernel(dev, N, K, mode, yf):
    """A batch of one item runs the whole-row kernel (nb_gemv_rows.hip):
    every activation form and output form, chunks of 64 / bpr rows with a
    partial last chunk, K from one block to 64 blocks per row -- against
    the fp64 brute force over the bf16 activations formed on the CPU, and
    against the same item in a two-item batch (the 64-block-chunk kernel)."""
    note(f"rows kernel {N}x{K} x={mode} y={yf}")
    g = torch.Generator().manual_seed(N * 7 + K)
    eps = 1e-6
    idx, p, cb = random_layer(N, K, 3, 8, 128, N + K)
    pt, ct = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
    form = {"y": yf}
    if mode == "rmsnorm":
        x = torch.randn(K, generator=g) * 3
        w = 1 + 0.1 * torch.randn(K, generator=g)
        form["x"] = ("rmsnorm", w.to(dev), eps)
        a = _fused_activations(mode, x, w, eps)
    elif mode == "silu_mul":
        x = torch.randn(2 * K, generator=g) * 2
        form["x"] = "silu_mul"
        a = _fused_activations(mode, x)
    else:
        x = torch.randn(K, generator=g).to(torch.bfloat16)
        a = x
    y0 = torch.randn(N, generator=g) if yf == "add" else torch.zeros(N)
    xd = x.to(dev)

    def out():
        return y0.clone().to(dev) if yf == "add" else torch.full((N,), float("nan"), device=dev)
    y1, y2 = out(), out()
    ops.GemvBatch([(xd, pt, ct, y1, N, K, form)]).run()
    # the same item beside a one-row dummy item: the batched (64-block chunk) kernel
    didx, dp, dcb = random_layer(1, 128, 3, 8, 128, 5)
    dummy = (torch.zeros(128, dtype=torch.bfloat16, device=dev), torch.from_numpy(dp).to(dev),
             torch.from_numpy(dcb).to(dev), torch.empty(1, device=dev), 1, 128)
    ops.GemvBatch([(xd, pt, ct, y2, N, K, form), dummy]).run()
    ref = ref_gemv(a, idx, cb, 128, N, K)[0] + y0.double().numpy()
    assert np.isfinite(y1.cpu().numpy()).all()
    assert rel(y1.cpu(), ref) <= REL_F32, rel(y1.cpu(), ref)
    assert rel(y1.cpu(), y2.cpu()) <= 1e-3, rel(y1.cpu(), y2.cpu())


@pytest.mark.parametrize("F,K", [(6912, 2560), (64, 128), (300, 384), (21, 2560)])
def test_single_item_silu_pairs(dev, F, K):
    """NB_Y_SILU_PAIRS: a gate|up layer whose rows alternate gate row i, up
    row i writes act[i] = bf16(silu(gate_i . a) * (up_i . a)) -- the SwiGLU
    product of generate_torch.py:116-117 -- equal to forming it on the CPU
    from the fp64 brute-force rows (bf16 bar: 1e-2), and to the stacked
    gate|up GEMV followed by the silu_mul activation form up to bf16
    rounding of a few values."""
    note(f"silu pairs F={F} K={K}")
    g = torch.Generator().manual_seed(F + K)
    eps = 1e-6
    gi, gp, gcb = random_layer(F, K, 3, 8, 128, F)
    ui, up, ucb = random_layer(F, K, 3, 8, 128, F + 1)
    # interleave rows on the host: row 2i = gate i, row 2i+1 = up i
    bpr = K // 128
    gidx, uidx = gi.reshape(F, bpr * 128), ui.reshape(F, bpr * 128)
    iidx = np.stack([gidx, uidx], axis=1).reshape(-1)
    icb = np.stack([gcb.reshape(F, bpr, 8), ucb.reshape(F, bpr, 8)], axis=1).reshape(-1, 8)
    ipk = torch.from_numpy(O.pack(iidx, 3)).to(dev)
    icbt = torch.from_numpy(np.ascontiguousarray(icb)).to(dev)
    x = torch.randn(K, generator=g) * 3
    w = 1 + 0.1 * torch.randn(K, generator=g)
    wd = w.to(dev)
    act = torch.full((F,), float("nan"), dtype=torch.bfloat16, device=dev)
    ops.GemvBatch([(x.to(dev), ipk, icbt, act, 2 * F, K,
                    {"x": ("rmsnorm", wd, eps), "y": "silu_pairs"})]).run()
    a = _fused_activations("rmsnorm", x, w, eps)
    r = ref_gemv(a, iidx, icb, 128, 2 * F, K)[0]
    gate, upv = torch.from_numpy(r[0::2]), torch.from_numpy(r[1::2])
    ref = torch.nn.functional.silu(gate) * upv
    got = act.float().cpu()
    assert torch.isfinite(got).all()
    assert rel(got, ref) <= REL_BF16, rel(got, ref)
    # the unfused route: stacked gate|up rows (fp32 out), then silu(gate) * up
    spk = torch.from_numpy(O.pack(np.concatenate([gi, ui]), 3)).to(dev)
    scb = torch.from_numpy(np.concatenate([gcb, ucb])).to(dev)
    gu = torch.empty(2 * F, device=dev)
    ops.GemvBatch([(x.to(dev), spk, scb, gu, 2 * F, K, {"x": ("rmsnorm", wd, eps)})]).run()
    gu = gu.cpu()
    unfused = (torch.nn.functional.silu(gu[:F]) * gu[F:]).to(torch.bfloat16).float()
    assert rel(got, unfused) <= 4e-3, rel(got, unfused)


def test_batched_many_small_fused_items(dev):
    """Many small items, so one workgroup forms several problems'
    activations (each RMSNorm with its own barriers) and takes chunks of
    several problems: every item equals its unfused sequence."""
    g = torch.Generator().manual_seed(99)
    eps = 1e-6
    items, plain, adds = [], [], []
    for i in range(40):
        N, K = (17 + 13 * i) % 300 + 1, 128 * (1 + i % 5)
        mode = ("rmsnorm", "silu_mul", "bf16")[i % 3]
        yf = "add" if i % 2 else "store"
        idx, p, cb = random_layer(N, K, 3, 8, 128, 2000 + i)
        pt, ct = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
        form = {"y": yf}
        if mode == "rmsnorm":
            x = torch.randn(K, generator=g)
            w = 1 + 0.1 * torch.randn(K, generator=g)
            form["x"] = ("rmsnorm", w.to(dev), eps)
            a = _fused_activations(mode, x, w, eps)
        elif mode == "silu_mul":
            x = torch.randn(2 * K, generator=g)
            form["x"] = "silu_mul"
            a = _fused_activations(mode, x)
        else:
            x = torch.randn(K, generator=g).to(torch.bfloat16)
            a = x
        y0 = torch.randn(N, generator=g) if yf == "add" else torch.zeros(N)
        y = y0.clone().to(dev) if yf == "add" else torch.full((N,), float("nan"), device=dev)
        items.append((x.to(dev), pt, ct, y, N, K, form))
        plain.append((a.to(dev), pt, ct, torch.empty(N, device=dev), N, K))
        adds.append(y0)
    note("40 small fused items in one batch")
    ops.GemvBatch(items).run()
    ops.GemvBatch(plain).run()
    for i, (item, pl) in enumerate(zip(items, plain)):
        unfused = pl[3].cpu() + adds[i]
        assert rel(item[3].cpu(), unfused) <= 1e-3, (i, rel(item[3].cpu(), unfused))


def test_skinny_batched_more_items_than_one_launch(dev):
    """More items than one skinny launch takes (512): the launcher splits
    the table; every item still equals its own GEMV."""
    M, n = 3, 600
    items, refs = [], []
    for i in range(n):
        N, K = 1 + (i * 37) % 200, 128 * (1 + i % 3)
        idx, p, cb = random_layer(N, K, 3, 8, 128, 3000 + i)
        x = torch.randn(M, K, generator=torch.Generator().manual_seed(i)).to(torch.bfloat16)
        items.append((x.to(dev), torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev),
                      torch.full((M, N), float("nan"), device=dev), N, K))
        refs.append((idx, cb, x))
    note(f"skinny M={M} with {n} items")
    ops.GemvBatch(items, m=M).run()
    torch.cuda.synchronize()
    for i in range(0, n, 7):  # a spread sample against the fp64 brute force
        idx, cb, x = refs[i]
        N, K = items[i][4], items[i][5]
        ref = ref_gemv(x, idx, cb, 128, N, K)
        assert rel(items[i][3].cpu(), ref) <= REL_F32, (i, N, K)
    assert all(torch.isfinite(it[3]).all().item() for it in items)


@pytest.mark.parametrize("M", [5, 14])
def test_skinny_batched_task_runs_cross_items(dev, M):
    """Workgroups walk contiguous task runs that cross item boundaries (here
    every workgroup holds several small items, some with a partial last
    slice and ragged rows), with three x buffers (M <= 13) or two; every item
    equals the fp64 brute force, and a y += item adds."""
    n = 400
    items, refs = [], []
    for i in range(n):
        N, K = 1 + (i * 53) % 300, 128 * (1 + i % 7)
        idx, p, cb = random_layer(N, K, 3, 8, 128, 7000 + i)
        x = torch.randn(M, K, generator=torch.Generator().manual_seed(900 + i)).to(torch.bfloat16)
        y0 = torch.randn(M, N, generator=torch.Generator().manual_seed(5 + i))
        add = i % 5 == 0
        y = (y0.clone() if add else torch.full((M, N), float("nan"))).to(dev)
        item = (x.to(dev), torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev), y, N, K)
        items.append(item + (({"y": "add"},) if add else ()))
        refs.append((idx, cb, x, y0 if add else None))
    note(f"skinny M={M} with {n} small items")
    ops.GemvBatch(items, m=M).run()
    torch.cuda.synchronize()
    for i in range(0, n, 3):
        idx, cb, x, y0 = refs[i]
        N, K = items[i][4], items[i][5]
        ref = ref_gemv(x, idx, cb, 128, N, K)
        got = items[i][3].cpu()
        if y0 is not None:
            got = got - y0  # (an overwrite instead of an add would leave -y0 here)
        assert rel(got, ref) <= REL_F32, (i, N, K, y0 is not None)


def test_batched_add_twice_accumulates(dev):
    """y_mode add reads y each launch: two runs add the product twice."""
    N, K = 2560, 2560
    idx, p, cb = random_layer(N, K, 3, 8, 128, 4343)
    pt, ct = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
    x = torch.randn(K, device=dev).to(torch.bfloat16)
    y0 = torch.randn(N, device=dev)
    y = y0.clone()
    b = ops.GemvBatch([(x, pt, ct, y, N, K, {"y": "add"})])
    b.run()
    once = y.clone()
    b.run()
    yp = ops.gemv(x, pt, ct, N, K)
    assert rel((once - y0).cpu(), yp.cpu()) <= 1e-5
    assert rel((y - y0).cpu(), (2 * yp).cpu()) <= 1e-5


@pytest.mark.parametrize("M", [1, 2, 3, 4, 8, 13, 14, 16])
def test_skinny_batched_vs_f64(dev, M):
    """nb_gemm_skinny_batched over mixed shapes (ragged N, K with a partial
    last 512-slice, an empty item) equals the fp64 brute force on the
    bf16-rounded weights for every activation row."""
    shapes = [(2560, 2560), (100, 384), (0, 2560), (1000, 6912), (17, 128), (300, 2688)]
    items, refs = [], []
    for i, (N, K) in enumerate(shapes):
        note(f"skinny M={M} item {i} {N}x{K}")
        idx, p, cb = random_layer(max(N, 1), K, 3, 8, 128, 1500 + 10 * M + i)
        x = torch.randn(M, K, generator=torch.Generator().manual_seed(i + M)).to(torch.bfloat16)
        pt, ct = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
        if N == 0:
            pt, ct = pt[:16].clone(), ct[:0].reshape(0, 8).contiguous()
        y = torch.full((M, N), float("nan"), device=dev)
        items.append((x.to(dev).contiguous(), pt, ct, y, N, K))
        refs.append(ref_gemv(x, idx, cb, 128, N, K) if N else None)
    b = ops.GemvBatch(items, m=M)
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    # the skinny kernel itself, also at M = 1 (GemvBatch(m=1) streams)
    _lib.check(lib.nb_gemm_skinny_batched(b._arr, b.table.data_ptr(), b.count, M, _lib.NB_F32,
                                          stream))
    torch.cuda.synchronize()
    for i, (x, pt, ct, y, N, K) in enumerate(items):
        if N:
            assert rel(y.cpu(), refs[i]) <= REL_F32, (i, rel(y.cpu(), refs[i]))
    if M > 1:
        y1 = [t[3].clone() for t in items]
        b.run()
        for (x, pt, ct, y, N, K), ya in zip(items, y1):
            assert torch.equal(y, ya)  # deterministic


def test_skinny_batched_forms(dev):
    """bf16 outputs are the rounded fp32 outputs; y_mode add adds."""
    M, N, K = 4, 2560, 6912
    idx, p, cb = random_layer(N, K, 3, 8, 128, 1777)
    pt, ct = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
    x = torch.randn(M, K, device=dev).to(torch.bfloat16)
    y32 = torch.empty(M, N, device=dev)
    ops.GemvBatch([(x, pt, ct, y32, N, K)], m=M).run()
    y16 = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    ops.GemvBatch([(x, pt, ct, y16, N, K)], m=M).run()
    assert torch.equal(y16, y32.to(torch.bfloat16))
    y0 = torch.randn(M, N, device=dev)
    ya = y0.clone()
    ops.GemvBatch([(x, pt, ct, ya, N, K, {"y": "add"})], m=M).run()
    assert rel((ya - y0).cpu(), y32.cpu()) <= 1e-5
    # row m of a skinny product is the M = 1 GEMV of x[m]
    for m in range(M):
        assert rel(y32[m].cpu(), ops.gemv(x[m].contiguous(), pt, ct, N, K).cpu()) <= 1e-5


@pytest.mark.parametrize("M", [1, 4])
def test_batched_graph_replay(dev, M):
    """Captured in a HIP graph and replayed several times, with eager work in
    between, every replay reproduces the eager result (M = 1: the streaming
    kernel; M = 4: the skinny kernel)."""
    N, K = 2560, 2560
    idx, p, cb = random_layer(N, K, 3, 8, 128, 4242)
    pt, ct = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
    x = torch.randn(K, device=dev).to(torch.bfloat16) if M == 1 else \
        torch.randn(M, K, device=dev).to(torch.bfloat16)
    y = torch.empty(N, device=dev) if M == 1 else torch.empty(M, N, device=dev)
    b = ops.GemvBatch([(x, pt, ct, y, N, K)], m=M)
    b.run()
    torch.cuda.synchronize()
    eager = y.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        b.run()
    for _ in range(3):
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
