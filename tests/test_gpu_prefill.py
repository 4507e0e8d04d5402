"""GPU parity of the prefill kernel (nb_gemm_prefill, run with -m gpu).

y = x @ bf16(W).T against the fp64 brute force of the oracle on the same
bf16-rounded codebook entries and bf16 activations (the reference's bf16
path, inference/eval_ppl.py:149-174): rel <= 1e-3 for fp32 output (fp32
accumulation), <= 1e-2 for bf16 output; ragged M and N, every 2.2B layer
shape, and agreement with the batched GEMV on shared rows.
"""
import numpy as np
import pytest
import torch

from nativebit_amd import _lib, ops, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def note(msg):
    print(f"[case] {msg}", flush=True)


def rel(a, b):
    a = np.asarray(a, dtype=np.float64).reshape(-1)
    b = np.asarray(b, dtype=np.float64).reshape(-1)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def layer(N, K, seed):
    rng = np.random.default_rng(seed)
    nb = N * K // 128
    idx = rng.integers(0, 8, nb * 128, dtype=np.uint8)
    cb = (rng.standard_normal((nb, 8)) * 0.02).astype(np.float32)
    return idx, O.pack(idx, 3), cb


@pytest.mark.parametrize("M,N,K", [(128, 128, 128), (200, 300, 384), (1, 100, 128),
                                   (17, 2560, 2560), (512, 2560, 2560), (300, 7680, 2560),
                                   (64, 2560, 6912)])
@pytest.mark.parametrize("ydt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("path", ["auto", "fused"])
def test_prefill_vs_f64(dev, M, N, K, ydt, path):
    note(f"prefill M={M} N={N} K={K} {ydt} {path}")
    idx, p, cb = layer(N, K, M * 7 + N)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(M + N)).to(torch.bfloat16)
    xd, pd, cd = x.to(dev), torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
    y = ops.gemm_prefill(xd, pd, cd, N, K, out_dtype=ydt, path=path)
    w = O.dequant(idx, cb, 128, N * K).reshape(N, K)
    w = torch.from_numpy(w).to(torch.bfloat16).float().numpy()
    # fp64 brute force on row subsets for the large shapes (keeps the CPU time short)
    rows = np.arange(M) if M * N * K <= 2e8 else np.unique(np.linspace(0, M - 1, 24).astype(int))
    ref = O.matmul_f64(x.float().numpy()[rows], w)
    got = y.float().cpu().numpy()[rows]
    assert rel(got, ref) <= (1e-3 if ydt == torch.float32 else 1e-2), rel(got, ref)


@pytest.mark.parametrize("path", ["fused", "auto"])
def test_prefill_strided_x_and_out(dev, path):
    M, N, K = 96, 256, 512
    idx, p, cb = layer(N, K, 5)
    big = torch.randn(M, K + 64).to(torch.bfloat16).to(dev)
    x = big[:, :K]                      # row stride K + 64 (a multiple of 8)
    out = torch.full((M, N + 8), float("nan"), device=dev)[:, :N]
    ops.gemm_prefill(x, torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev), N, K,
                     out=out, path=path)
    w = torch.from_numpy(O.dequant(idx, cb, 128, N * K).reshape(N, K)).to(torch.bfloat16).float()
    ref = x.float().cpu() @ w.T
    assert rel(out.cpu(), ref) <= 1e-5


# Shapes the K split takes (nb_gemm_prefill_split, path "auto"): few tokens
# on every 2.2B layer shape, the 512-token narrow layers, and a ragged
# shape whose N is not a multiple of 4 (scalar partial stores and sums).
SPLIT_CASES = [(128, 7680, 2560), (128, 2560, 2560), (128, 13824, 2560), (128, 2560, 6912),
               (512, 2560, 2560), (512, 2560, 6912), (100, 1998, 6912), (40, 2560, 6912)]


@pytest.mark.parametrize("M,N,K", SPLIT_CASES)
def test_prefill_split_vs_f64(dev, M, N, K):
    """The split path against the fp64 brute force, deterministic over two
    calls, and equal to the one-launch kernel up to fp32 summation order."""
    from nativebit_amd import _lib
    ws = _lib.load().nb_gemm_prefill_split_ws_bytes(M, N, K)
    note(f"prefill split M={M} N={N} K={K} ws={ws}")
    assert ws > 0
    idx, p, cb = layer(N, K, 31 * M + N)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(M + K)).to(torch.bfloat16)
    xd, pd, cd = x.to(dev), torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
    a = ops.gemm_prefill(xd, pd, cd, N, K, out_dtype=torch.float32, path="auto")
    b = ops.gemm_prefill(xd, pd, cd, N, K, out_dtype=torch.float32, path="auto")
    assert torch.equal(a, b)
    one = ops.gemm_prefill(xd, pd, cd, N, K, out_dtype=torch.float32, path="fused")
    assert rel(a.cpu(), one.cpu()) <= 1e-5, rel(a.cpu(), one.cpu())
    y16 = ops.gemm_prefill(xd, pd, cd, N, K, out_dtype=torch.bfloat16, path="auto")
    assert torch.equal(y16, a.to(torch.bfloat16))   # the sum, rounded once
    w = O.dequant(idx, cb, 128, N * K).reshape(N, K)
    w = torch.from_numpy(w).to(torch.bfloat16).float().numpy()
    rows = np.unique(np.linspace(0, M - 1, 16).astype(int))
    ref = O.matmul_f64(x.float().numpy()[rows], w)
    assert rel(a.cpu().numpy()[rows], ref) <= 1e-3, rel(a.cpu().numpy()[rows], ref)


def test_prefill_split_strided_out_and_graph(dev):
    """A split into a strided output (row stride N + 8) inside a HIP graph:
    the workspace comes from the graph's pool, and every replay (eager work
    in between) reproduces the eager result."""
    M, N, K = 128, 2560, 2560
    idx, p, cb = layer(N, K, 77)
    x = torch.randn(M, K).to(torch.bfloat16).to(dev)
    pd, cd = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
    note("prefill split strided out + graph")
    out = torch.full((M, N + 8), float("nan"), device=dev)[:, :N]
    ops.gemm_prefill(x, pd, cd, N, K, out=out, path="auto")
    torch.cuda.synchronize()
    eager = out.clone()
    w = torch.from_numpy(O.dequant(idx, cb, 128, N * K).reshape(N, K)).to(torch.bfloat16).float()
    assert rel(eager.cpu(), x.float().cpu() @ w.T) <= 1e-5
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.gemm_prefill(x, pd, cd, N, K, out=out, path="auto")
    for _ in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_prefill_matches_batched_gemv(dev):
    """Row 0 of a prefill equals the single-token GEMV of the same layer."""
    lay = synth.make_layer(6912, 2560, seed=11, device=dev)
    x = synth.make_activation(2560, m=33, seed=12, device=dev, dtype=torch.bfloat16)
    y = ops.gemm_prefill(x, lay.packed, lay.codebook, 6912, 2560, out_dtype=torch.float32)
    for m in (0, 17, 32):
        yv = torch.empty(6912, device=dev)
        ops.GemvBatch([(x[m].contiguous(), lay.packed, lay.codebook, yv, 6912, 2560)]).run()
        assert rel(y[m].cpu(), yv.cpu()) <= 1e-5


def test_prefill_deterministic(dev):
    idx, p, cb = layer(2560, 2560, 9)
    x = torch.randn(256, 2560).to(torch.bfloat16).to(dev)
    pd, cd = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
    a = ops.gemm_prefill(x, pd, cd, 2560, 2560, out_dtype=torch.float32, path="fused")
    b = ops.gemm_prefill(x, pd, cd, 2560, 2560, out_dtype=torch.float32, path="fused")
    assert torch.equal(a, b)


def test_prefill_matches_expanded_weight(dev):
    """The fused kernel and the reference's order of work on the GPU (W
    gathered by the format kernel at bf16, then a dense fp32 product of the
    same bf16 operands, eval_ppl.py:149-174) agree to fp32 summation-order
    differences."""
    lay = synth.make_layer(2560, 6912, seed=13, device=dev)
    x = synth.make_activation(6912, m=512, seed=14, device=dev, dtype=torch.bfloat16)
    a = ops.gemm_prefill(x, lay.packed, lay.codebook, 2560, 6912, out_dtype=torch.float32,
                         path="fused")
    w = ops.dequant(lay.packed, lay.codebook, 2560 * 6912, 3, 128, torch.bfloat16)
    b = x.float() @ w.view(2560, 6912).float().T
    assert rel(a.cpu(), b.cpu()) <= 1e-5, rel(a.cpu(), b.cpu())


@pytest.mark.parametrize("ydt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("path", ["fused", "auto"])
def test_prefill_output_view_at_odd_offset(dev, path, ydt):
    """y a view that starts one element into its storage (aligned to its
    dtype only) and has an odd row stride: every store takes the scalar
    form where the vector one would be misaligned; results are those of a
    fresh output."""
    M, N, K = 130, 260, 2560
    note(f"prefill odd-offset output {path} {ydt}")
    idx, p, cb = layer(N, K, 21)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(dev)
    pd, cd = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
    want = ops.gemm_prefill(x, pd, cd, N, K, out_dtype=ydt, path=path)
    store = torch.full((M * (N + 3) + 1,), float("nan"), dtype=ydt, device=dev)
    out = store[1:].view(M, N + 3)[:, :N]
    assert out.data_ptr() % 8 != 0
    ops.gemm_prefill(x, pd, cd, N, K, out=out, path=path)
    assert torch.equal(out, want)
    assert torch.isnan(store[0]) and torch.isnan(store[1:].view(M, N + 3)[:, N:]).all()


# Config 4a: M = 2048 tokens on the four matmul shapes of a 2.2B layer
# (q|k|v, o, gate|up, down), every path, against the fp64 brute force on 24
# rows spread over M.
PREFILL_2P2B = {"qkv": (7680, 2560), "o": (2560, 2560), "gate|up": (13824, 2560),
                "down": (2560, 6912)}
_LAYER_CACHE = {}


def _layer_2p2b(name):
    if name not in _LAYER_CACHE:
        N, K = PREFILL_2P2B[name]
        idx, p, cb = layer(N, K, 4242 + N + K)
        w = O.dequant(idx, cb, 128, N * K).reshape(N, K)
        w = torch.from_numpy(w).to(torch.bfloat16).float().numpy()
        _LAYER_CACHE.clear()  # one shape at a time (the 13824 x 2560 weight is 142 MB)
        _LAYER_CACHE[name] = (p, cb, w)
    return _LAYER_CACHE[name]


@pytest.mark.parametrize("ydt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("path", ["auto", "fused"])
@pytest.mark.parametrize("name", list(PREFILL_2P2B))
def test_prefill_m2048_2p2b(dev, name, path, ydt):
    M = 2048
    N, K = PREFILL_2P2B[name]
    note(f"prefill M={M} {name} {N}x{K} {path} {ydt}")
    p, cb, w = _layer_2p2b(name)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(N + K)).to(torch.bfloat16)
    y = ops.gemm_prefill(x.to(dev), torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev),
                         N, K, out_dtype=ydt, path=path)
    rows = np.unique(np.linspace(0, M - 1, 24).astype(int))
    ref = O.matmul_f64(x.float().numpy()[rows], w)
    got = y.float().cpu().numpy()[rows]
    assert np.isfinite(got).all()
    assert rel(got, ref) <= (1e-3 if ydt == torch.float32 else 1e-2), rel(got, ref)


# fp32 activations against the exact fp32 codebook values (nb_gemm_prefill_f32:
# three bf16 passes over the hi / lo parts of x and W).  Each product is x.W to
# within 2^-16 of its size, so the sums stay within 1e-5 of the fp64 brute
# force on the exact weights (the north star's fp32 bar is 1e-3).
F32_CASES = [(17, 128, 128), (40, 300, 384), (200, 2560, 2560), (512, 7680, 2560),
             (128, 2560, 6912), (100, 1998, 6912), (2048, 2560, 2560)]


@pytest.mark.parametrize("M,N,K", F32_CASES)
def test_prefill_f32_vs_f64(dev, M, N, K):
    note(f"prefill f32 M={M} N={N} K={K}")
    idx, p, cb = layer(N, K, M + 3 * N)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(M * 5 + K))
    pd, cd = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
    y = ops.gemm_prefill_f32(x.to(dev), pd, cd, N, K)
    w = O.dequant(idx, cb, 128, N * K).reshape(N, K)        # exact fp32 weights
    rows = np.arange(M) if M * N * K <= 2e8 else np.unique(np.linspace(0, M - 1, 24).astype(int))
    ref = O.matmul_f64(x.numpy()[rows], w)
    got = y.cpu().numpy()[rows]
    assert np.isfinite(got).all()
    assert rel(got, ref) <= 1e-5, rel(got, ref)
    # the bf16 path on the same x differs by the bf16 roundings (~1e-3): the
    # fp32 path is the more exact one
    yb = ops.gemm_prefill(x.to(torch.bfloat16).to(dev), pd, cd, N, K, out_dtype=torch.float32)
    assert rel(yb.cpu().numpy()[rows], ref) > 10 * rel(got, ref)


def test_prefill_f32_strided_and_deterministic(dev):
    M, N, K = 96, 260, 640
    idx, p, cb = layer(N, K, 77)
    pd, cd = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
    big = torch.randn(M, K + 3, generator=torch.Generator().manual_seed(8)).to(dev)
    x = big[:, 1:K + 1]                                      # odd offset, row stride K + 3
    out = torch.full((M, N + 5), float("nan"), device=dev)[:, 2:N + 2]
    lib = _lib.load()
    nbytes = int(lib.nb_gemm_prefill_f32_ws_bytes(M, N, K))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    for _ in range(2):
        _lib.check(lib.nb_gemm_prefill_f32(x.data_ptr(), x.stride(0), pd.data_ptr(), cd.data_ptr(),
                                           out.data_ptr(), out.stride(0), M, N, K, ws.data_ptr(),
                                           nbytes, s))
        first = out.clone() if _ == 0 else first
    assert torch.equal(out, first)
    w = O.dequant(idx, cb, 128, N * K).reshape(N, K)
    ref = O.matmul_f64(x.cpu().numpy(), w)
    assert rel(out.cpu().numpy(), ref) <= 1e-5


def test_packed_linear_f32_batched_uses_exact_weights(dev):
    """PackedLinear with fp32 x and more than 16 rows: the fp32 MFMA path."""
    from nativebit_amd import PackedLinear
    N, K, M = 640, 2560, 300
    idx, p, cb = layer(N, K, 5)
    lin = PackedLinear(torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev), N, K)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(6))
    y = lin(x.to(dev))
    ref = O.matmul_f64(x.numpy(), O.dequant(idx, cb, 128, N * K).reshape(N, K))
    assert y.dtype == torch.float32 and rel(y.cpu().numpy(), ref) <= 1e-5
