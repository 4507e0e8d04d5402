"""GPU parity of the row-quad layout (nb_quad_layout) and the M <= 4
skinny kernel on it (nb_gemm_skinny_quad_batched), run with -m gpu.

Bars: the layout is byte-exact against a numpy re-ordering of the
reference layout's blocks with every 12-byte unit in the selector-ordered
unit layout (tests/test_stream_layout.py); the products are within 1e-3 (relative L2) of
the fp64 brute force on the bf16-rounded weights (the reference's bf16
path, inference/eval_ppl.py:149-174), deterministic, and a bf16 output is
the RNE rounding of the fp32 one."""
import numpy as np
import pytest
import torch

from nativebit_amd import ops

from oracle import oracle as O
from test_gpu_parity import REL_F32, note, random_layer, ref_gemv, rel
from test_stream_layout import sel_layout_np

pytestmark = pytest.mark.gpu


def quad_order_np(p, cb, N, K):
    """The row-quad layout by array re-shaping: blocks [N, bpr] -> rows
    padded to a multiple of 4 with zero blocks -> [nq, 4, bpr] -> [nq, bpr, 4],
    then every 12-byte unit in the selector-ordered unit layout."""
    bpr = K // 128
    nq = -(-N // 4)
    ib = np.zeros((nq * 4, bpr, 48), np.uint8)
    ib[:N] = np.frombuffer(p[: N * bpr * 48].tobytes(), np.uint8).reshape(N, bpr, 48)
    c = np.zeros((nq * 4, bpr, 8), np.float32)
    c[:N] = cb.reshape(N, bpr, 8)
    ib = ib.reshape(nq, 4, bpr, 48).transpose(0, 2, 1, 3).reshape(-1)
    c = c.reshape(nq, 4, bpr, 8).transpose(0, 2, 1, 3).reshape(-1, 8)
    return sel_layout_np(O.unpack(ib, ib.size * 8 // 3, 3)), c


@pytest.mark.parametrize("N,K", [(8, 2048), (2560, 2560), (1001, 6912), (3, 128), (6, 8192)])
def test_quad_layout_bytes(dev, N, K):
    note(f"quad layout {N}x{K}")
    idx, p, cb = random_layer(N, K, 3, 8, 128, 60 + N)
    qp, qc = ops.quad_layout(torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev), N, K)
    ib, c = quad_order_np(p, cb, N, K)
    assert np.array_equal(qp.cpu().numpy(), ib)
    assert np.array_equal(qc.cpu().numpy(), c)


def _items(dev, shapes, M, seed, add_every=0):
    items, refs = [], []
    for i, (N, K) in enumerate(shapes):
        idx, p, cb = random_layer(max(N, 1), K, 3, 8, 128, seed + i)
        pt, ct = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
        if N:
            qp, qc = ops.quad_layout(pt, ct, N, K)
        else:
            qp, qc = pt[:16].clone(), ct[:0].reshape(0, 8).contiguous()
        x = torch.randn(M, K, generator=torch.Generator().manual_seed(seed + 7 * i))
        x = x.to(torch.bfloat16)
        add = add_every and i % add_every == 0
        y0 = torch.randn(M, N, generator=torch.Generator().manual_seed(seed + 11 * i))
        y = (y0.clone() if add else torch.full((M, N), float("nan"))).to(dev)
        item = (x.to(dev), qp, qc, y, N, K)
        items.append(item + (({"y": "add"},) if add else ()))
        refs.append((idx, cb, x, y0 if add else None))
    return items, refs


@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_quad_skinny_vs_f64(dev, M):
    """Mixed shapes in one batch (ragged N: quads with padded rows; K from
    2048 to 8192; an empty item) against the fp64 brute force, and
    deterministic over two runs."""
    shapes = [(2560, 2560), (1001, 6912), (0, 2560), (2563, 2048), (6, 8192), (7680, 2560)]
    items, refs = _items(dev, shapes, M, 2100 + 10 * M)
    for i, (N, K) in enumerate(shapes):
        note(f"quad skinny M={M} item {i} {N}x{K}")
    b = ops.GemvBatch(items, m=M, layout="quad")
    b.run()
    torch.cuda.synchronize()
    for i, (N, K) in enumerate(shapes):
        if N:
            idx, cb, x, _ = refs[i]
            ref = ref_gemv(x, idx, cb, 128, N, K)
            assert rel(items[i][3].cpu(), ref) <= REL_F32, (i, N, K, rel(items[i][3].cpu(), ref))
    first = [it[3].clone() for it in items]
    b.run()
    for it, y1 in zip(items, first):
        assert torch.equal(it[3], y1)  # deterministic


@pytest.mark.parametrize("M", [2, 4])
def test_quad_skinny_many_items(dev, M):
    """More problems than one launch takes (256) and workgroup / wave runs
    that cross item boundaries, with y += on every fifth item."""
    n = 300
    shapes = [(1 + (i * 53) % 300, 128 * (16 + i % 3 * 19)) for i in range(n)]
    items, refs = _items(dev, shapes, M, 9000, add_every=5)
    note(f"quad skinny M={M} with {n} items")
    ops.GemvBatch(items, m=M, layout="quad").run()
    torch.cuda.synchronize()
    for i in range(0, n, 3):
        idx, cb, x, y0 = refs[i]
        N, K = shapes[i]
        ref = ref_gemv(x, idx, cb, 128, N, K)
        got = items[i][3].cpu()
        if y0 is not None:
            got = got - y0
        assert rel(got, ref) <= REL_F32, (i, N, K, y0 is not None)


def test_quad_skinny_forms_and_rows_kernel(dev):
    """bf16 outputs are the rounded fp32 outputs, y += adds, and the results
    agree with the row-layout skinny kernel on the same layer."""
    M, N, K = 4, 2560, 6912
    idx, p, cb = random_layer(N, K, 3, 8, 128, 1778)
    pt, ct = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
    qp, qc = ops.quad_layout(pt, ct, N, K)
    x = torch.randn(M, K, device=dev).to(torch.bfloat16)
    note("quad skinny forms")
    y32 = torch.empty(M, N, device=dev)
    ops.GemvBatch([(x, qp, qc, y32, N, K)], m=M, layout="quad").run()
    y16 = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    ops.GemvBatch([(x, qp, qc, y16, N, K)], m=M, layout="quad").run()
    assert torch.equal(y16, y32.to(torch.bfloat16))
    y0 = torch.randn(M, N, device=dev)
    ya = y0.clone()
    ops.GemvBatch([(x, qp, qc, ya, N, K, {"y": "add"})], m=M, layout="quad").run()
    assert rel((ya - y0).cpu(), y32.cpu()) <= 1e-5
    yr = torch.empty(M, N, device=dev)
    ops.GemvBatch([(x, pt, ct, yr, N, K)], m=M).run()
    assert rel(y32.cpu(), yr.cpu()) <= 1e-5


def test_quad_skinny_graph_replay(dev):
    """Captured in a HIP graph, every replay (with eager work between)
    reproduces the eager result."""
    M, N, K = 3, 2560, 2560
    idx, p, cb = random_layer(N, K, 3, 8, 128, 4243)
    qp, qc = ops.quad_layout(torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev), N, K)
    x = torch.randn(M, K, device=dev).to(torch.bfloat16)
    y = torch.empty(M, N, device=dev)
    note("quad skinny graph replay")
    b = ops.GemvBatch([(x, qp, qc, y, N, K)], m=M, layout="quad")
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
