"""GPU parity of the tile layout (nb_tile_layout) and the skinny kernel on it
(nb_gemm_skinny_tile_batched), run with -m gpu.

Bars: the layout is byte-exact against a numpy construction from the
unpacked indices (tiles of 16 rows x 4 column blocks; every 32-index unit
the selector-ordered unit (tests/test_stream_layout.py) whose selector s
holds indices 4s .. 4s + 3, i.e. the unit of the indices placed at
positions o(s) + 8t, o = (0, 1, 3, 4, 6, 7, 2, 5); row
r's blocks at block place (b + ((r >> 1) & 3) + (r >> 3)) & 3, its codebook
pieces p at place (p + ((r & 6) | ((r ^ (r >> 3)) & 1))) & 7; zeros past
the layer); the products are bit-identical to
nb_gemm_skinny_batched on the reference layout (the same MFMAs in the same
order), within 1e-3 of the fp64 brute force on the bf16-rounded weights
(the reference's bf16 path, inference/eval_ppl.py:149-174), and a bf16
output is the RNE rounding of the fp32 one."""
import numpy as np
import pytest
import torch

from nativebit_amd import ops
from oracle import oracle as O

from test_gpu_parity import REL_F32, note, random_layer, ref_gemv, rel
from test_stream_layout import sel_layout_np

pytestmark = pytest.mark.gpu

SEL_OFFSET = (0, 1, 3, 4, 6, 7, 2, 5)


def tile_layout_np(idx, cb, N, K):
    """(tpacked, tcodebook) of the tile layout, built from the natural
    indices and codebook by array operations."""
    bpr = K // 128
    ng, ns = -(-N // 16), -(-bpr // 4)
    # selector order inside every 32-index unit, then repack per block
    u = np.asarray(idx[: N * K], np.uint8).reshape(-1, 32)
    so = np.empty_like(u)
    for i in range(32):
        so[:, SEL_OFFSET[i >> 2] + 8 * (i & 3)] = u[:, i]
    blocks = sel_layout_np(so.reshape(-1)).reshape(N, bpr, 48)
    ib = np.zeros((ng * 16, ns * 4, 48), np.uint8)
    ib[:N, :bpr] = blocks
    c = np.zeros((ng * 16, ns * 4, 8), np.float32)
    c[:N, :bpr] = cb.reshape(N, bpr, 8)
    tp = np.zeros((ng, ns, 16, 4, 48), np.uint8)
    tc = np.zeros((ng, ns, 16, 8, 4), np.float32)
    for r in range(16):
        idx_rot, cb_rot = ((r >> 1) & 3) + (r >> 3), (r & 6) | ((r ^ (r >> 3)) & 1)
        for b in range(4):
            tp[:, :, r, (b + idx_rot) & 3] = ib[r::16].reshape(ng, ns, 4, 48)[:, :, b]
            for h in range(2):
                p = 2 * b + h
                tc[:, :, r, (p + cb_rot) & 7] = \
                    c[r::16].reshape(ng, ns, 4, 8)[:, :, b, 4 * h:4 * h + 4]
    return tp.reshape(-1), tc.reshape(-1, 8)


def test_sel_positions_are_a_permutation():
    pos = sorted(SEL_OFFSET[i >> 2] + 8 * (i & 3) for i in range(32))
    assert pos == list(range(32))


def test_slot_reads_are_bank_conflict_free():
    """Every ds_read_b128 of a slot or an x buffer: the 16 lanes (q, r) of
    one block q reach 16 different 4-bank groups of 64 banks, and each 8 of
    them 8 different groups of 32 banks."""
    def groups(addr_of, banks):
        return [(addr_of(r) // 4 // 4) % (banks // 4) for r in range(16)]
    for q in range(4):
        for j in range(3):  # index pieces
            f = lambda r: r * 192 + ((q + ((r >> 1) & 3) + (r >> 3)) & 3) * 48 + 16 * j
            assert len(set(groups(f, 64))) == 16
            g = groups(f, 32)
            assert len(set(g[:8])) == 8 and len(set(g[8:])) == 8
        for h in range(2):  # codebook pieces
            f = lambda r: 3072 + r * 128 + \
                ((2 * q + h + ((r & 6) | ((r ^ (r >> 3)) & 1))) & 7) * 16
            assert len(set(groups(f, 64))) == 16
            g = groups(f, 32)
            assert len(set(g[:8])) == 8 and len(set(g[8:])) == 8
        for J in range(16):  # x pieces, M = 16
            f = lambda r: r * 1024 + 16 * ((16 * q + J) ^ (r & 15))
            assert len(set(groups(f, 64))) == 16
            g = groups(f, 32)
            assert len(set(g[:8])) == 8 and len(set(g[8:])) == 8


@pytest.mark.parametrize("N,K", [(16, 2048), (2560, 2560), (1001, 6912), (3, 128), (37, 384)])
def test_tile_layout_bytes(dev, N, K):
    note(f"tile layout {N}x{K}")
    idx, p, cb = random_layer(N, K, 3, 8, 128, 90 + N)
    tp, tc = ops.tile_layout(torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev), N, K)
    ep, ec = tile_layout_np(idx, cb, N, K)
    assert np.array_equal(tp.cpu().numpy(), ep)
    assert np.array_equal(tc.cpu().numpy(), ec)


SHAPES = [(2560, 2560), (100, 384), (0, 2560), (1000, 6912), (17, 128), (300, 2688),
          (2563, 2048)]


@pytest.mark.parametrize("M", [2, 5, 8, 13, 14, 16])
def test_tile_skinny_equals_rows_layout(dev, M):
    """Mixed shapes (ragged N, K with a partial last 512-slice, an empty
    item, rows past N inside a 128-row task) in one batch: the tile kernel
    gives the reference-layout kernel's bits and is within the fp64 bar; a
    second run repeats them."""
    rows, tiles, refs = [], [], []
    for i, (N, K) in enumerate(SHAPES):
        note(f"tile skinny M={M} item {i} {N}x{K}")
        idx, p, cb = random_layer(max(N, 1), K, 3, 8, 128, 4400 + 10 * M + i)
        x = torch.randn(M, K, generator=torch.Generator().manual_seed(31 * i + M))
        x = x.to(torch.bfloat16).to(dev)
        pt, ct = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
        if N == 0:
            pt, ct = pt[:16].clone(), ct[:0].reshape(0, 8).contiguous()
            tp, tc = pt.clone(), ct.clone()
        else:
            tp, tc = ops.tile_layout(pt, ct, N, K)
        rows.append((x, pt, ct, torch.full((M, N), float("nan"), device=dev), N, K))
        tiles.append((x, tp, tc, torch.full((M, N), float("nan"), device=dev), N, K))
        refs.append(ref_gemv(x.cpu(), idx, cb, 128, N, K) if N else None)
    ops.GemvBatch(rows, m=M).run()
    b = ops.GemvBatch(tiles, m=M, layout="tile")
    b.run()
    torch.cuda.synchronize()
    for i, (N, K) in enumerate(SHAPES):
        if N:
            assert torch.equal(tiles[i][3], rows[i][3]), (i, N, K)
            assert rel(tiles[i][3].cpu(), refs[i]) <= REL_F32, (i, N, K)
    first = [t[3].clone() for t in tiles]
    b.run()
    for t, f in zip(tiles, first):
        assert torch.equal(t[3], f)


def test_tile_skinny_forms(dev):
    """bf16 outputs are the rounded fp32 outputs; y_mode add adds; every
    row of the product is that row's M = 1 GEMV."""
    M, N, K = 8, 2560, 6912
    idx, p, cb = random_layer(N, K, 3, 8, 128, 4777)
    pt, ct = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
    tp, tc = ops.tile_layout(pt, ct, N, K)
    x = torch.randn(M, K, device=dev).to(torch.bfloat16)
    y32 = torch.empty(M, N, device=dev)
    ops.GemvBatch([(x, tp, tc, y32, N, K)], m=M, layout="tile").run()
    y16 = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    ops.GemvBatch([(x, tp, tc, y16, N, K)], m=M, layout="tile").run()
    assert torch.equal(y16, y32.to(torch.bfloat16))
    y0 = torch.randn(M, N, device=dev)
    ya = y0.clone()
    ops.GemvBatch([(x, tp, tc, ya, N, K, {"y": "add"})], m=M, layout="tile").run()
    assert rel((ya - y0).cpu(), y32.cpu()) <= 1e-5
    for m in range(M):
        assert rel(y32[m].cpu(), ops.gemv(x[m].contiguous(), pt, ct, N, K).cpu()) <= 1e-5


def test_tile_layout_rejects(dev):
    pt = torch.zeros(48 * 4, dtype=torch.uint8, device=dev)
    cb = torch.zeros(4, 8, device=dev)
    with pytest.raises(ValueError):
        ops.tile_layout(pt, cb, 4, 200)
    with pytest.raises(ValueError):
        ops.tile_layout(pt, torch.zeros(8, 8, device=dev), 8, 128)  # too few bytes
    x = torch.zeros(2, 128, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        ops.GemvBatch([(x, pt, cb, torch.empty(1, 4, device=dev), 4, 128)], m=1, layout="tile")
    # a reference-layout layer is not a tile-layout one
    with pytest.raises(ValueError):
        ops.GemvBatch([(x, pt, cb, torch.empty(2, 4, device=dev), 4, 128)], m=2, layout="tile")


@pytest.mark.parametrize("M", [3, 14])
def test_tile_skinny_task_runs_cross_items(dev, M):
    """Many small items on the tile layout: 256-row tasks whose second
    128-row half is partly or wholly past N (every item with N <= 256),
    workgroup runs that cross many item boundaries, partial last slices,
    y += items; every item gives the reference-layout kernel's bits and a
    spread sample is within the fp64 bar."""
    n = 160
    rows, tiles, refs = [], [], []
    for i in range(n):
        N, K = 1 + (i * 53) % 300, 128 * (1 + i % 7)
        idx, p, cb = random_layer(N, K, 3, 8, 128, 8100 + i)
        x = torch.randn(M, K, generator=torch.Generator().manual_seed(700 + i))
        x = x.to(torch.bfloat16).to(dev)
        pt, ct = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
        tp, tc = ops.tile_layout(pt, ct, N, K)
        add = i % 4 == 0
        y0 = torch.randn(M, N, generator=torch.Generator().manual_seed(3 + i)).to(dev)
        form = ({"y": "add"},) if add else ()
        rows.append((x, pt, ct, y0.clone() if add else torch.full((M, N), float("nan"),
                                                                 device=dev), N, K) + form)
        tiles.append((x, tp, tc, y0.clone() if add else torch.full((M, N), float("nan"),
                                                                  device=dev), N, K) + form)
        refs.append((idx, cb, x.cpu(), y0.cpu() if add else None))
    note(f"tile skinny M={M} with {n} small items")
    ops.GemvBatch(rows, m=M).run()
    ops.GemvBatch(tiles, m=M, layout="tile").run()
    torch.cuda.synchronize()
    for i in range(n):
        assert torch.equal(tiles[i][3], rows[i][3]), (i, tiles[i][4], tiles[i][5])
    for i in range(0, n, 5):
        idx, cb, x, y0 = refs[i]
        N, K = tiles[i][4], tiles[i][5]
        got = tiles[i][3].cpu()
        if y0 is not None:
            got = got - y0
        assert rel(got, ref_gemv(x, idx, cb, 128, N, K)) <= REL_F32, (i, N, K)
