"""GPU parity of the selector-ordered unit layout (nb_stream_layout) and the
batched GEMV on it (nb_gemv_batched_sel), run with -m gpu.

Bars: the layout's bytes equal the numpy construction from the unpacked
indices (tests/test_stream_layout.py, pinned there against the selectors the
reference layout yields), also when written in place; every product of
nb_gemv_batched_sel is bit-identical to nb_gemv_batched on the reference
layout (the same selectors feed the same MFMAs in the same order) for
multi-item batches (the batched kernel) and for one-item batches in every
activation and output form (the whole-row kernel), and within 1e-3 of the
fp64 brute force on the bf16-rounded weights."""
import numpy as np
import pytest
import torch

from nativebit_amd import ops
from oracle import oracle as O

from test_gpu_parity import REL_F32, note, random_layer, ref_gemv, rel
from test_stream_layout import sel_layout_np

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N,K", [(1, 128), (37, 384), (2560, 2560), (6912, 2560), (300, 6912)])
def test_stream_layout_bytes(dev, N, K):
    note(f"stream layout {N}x{K}")
    idx, p, cb = random_layer(N, K, 3, 8, 128, 700 + N)
    pt = torch.from_numpy(p).to(dev)
    want = sel_layout_np(idx[: N * K])
    got = ops.stream_layout(pt, N, K)
    assert np.array_equal(got.cpu().numpy(), want)
    inplace = pt.clone()
    ops.stream_layout(inplace, N, K, out=inplace)
    assert np.array_equal(inplace.cpu().numpy()[: want.size], want)


def test_batched_sel_equals_reference_layout(dev):
    """A multi-item batch (the 2.2B shapes, ragged N, K not a multiple of a
    64-block chunk): the same bits as nb_gemv_batched, twice in a row."""
    shapes = [(2560, 2560), (6912, 2560), (2560, 6912), (7680, 2560), (100, 384), (1, 128),
              (1001, 1280)]
    g = torch.Generator().manual_seed(9)
    ref_items, sel_items, refs = [], [], []
    for i, (N, K) in enumerate(shapes):
        note(f"batched sel item {i} {N}x{K}")
        idx, p, cb = random_layer(N, K, 3, 8, 128, 810 + i)
        pt, ct = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
        x = torch.randn(K, generator=g).to(torch.bfloat16)
        ref_items.append((x.to(dev), pt, ct, torch.full((N,), float("nan"), device=dev), N, K))
        sel_items.append((x.to(dev), ops.stream_layout(pt, N, K), ct,
                          torch.full((N,), float("nan"), device=dev), N, K))
        refs.append(ref_gemv(x, idx, cb, 128, N, K)[0])
    ops.GemvBatch(ref_items).run()
    b = ops.GemvBatch(sel_items, layout="sel")
    b.run()
    torch.cuda.synchronize()
    for i, (r, s, want) in enumerate(zip(ref_items, sel_items, refs)):
        assert torch.equal(s[3], r[3]), (i, shapes[i])
        assert rel(s[3].cpu(), want) <= REL_F32, (i, shapes[i])
    first = [s[3].clone() for s in sel_items]
    b.run()
    for s, f in zip(sel_items, first):
        assert torch.equal(s[3], f)


@pytest.mark.parametrize("N,K", [(2560, 2560), (13824, 2560), (2560, 6912), (71, 8192)])
@pytest.mark.parametrize("mode,yf", [("bf16", "store"), ("rmsnorm", "store"), ("bf16", "add"),
                                     ("silu_mul", "add"), ("rmsnorm", "add")])
def test_single_item_sel_equals_reference_layout(dev, N, K, mode, yf):
    """One-item batches run the whole-row kernel: every fused form gives the
    reference layout's bits."""
    note(f"single sel {mode} {yf} {N}x{K}")
    g = torch.Generator().manual_seed(N + K)
    idx, p, cb = random_layer(N, K, 3, 8, 128, 900 + N)
    pt, ct = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
    form = {"y": yf}
    if mode == "rmsnorm":
        x = (torch.randn(K, generator=g) * 3).to(dev)
        form["x"] = ("rmsnorm", (1 + 0.1 * torch.randn(K, generator=g)).to(dev), 1e-6)
    elif mode == "silu_mul":
        x = (torch.randn(2 * K, generator=g) * 2).to(dev)
        form["x"] = "silu_mul"
    else:
        x = torch.randn(K, generator=g).to(torch.bfloat16).to(dev)
    y0 = torch.randn(N, generator=g).to(dev)
    ys = [y0.clone() if yf == "add" else torch.full((N,), float("nan"), device=dev)
          for _ in range(2)]
    ops.GemvBatch([(x, pt, ct, ys[0], N, K, form)]).run()
    ops.GemvBatch([(x, ops.stream_layout(pt, N, K), ct, ys[1], N, K, form)], layout="sel").run()
    assert torch.equal(ys[1], ys[0])


def test_single_item_sel_silu_pairs_and_bf16_out(dev):
    """The SwiGLU-pair output (interleaved gate/up rows) and bf16 outputs."""
    F, K = 2 * 6912, 2560
    idx, p, cb = random_layer(F, K, 3, 8, 128, 1234)
    pt, ct = torch.from_numpy(p).to(dev), torch.from_numpy(cb).to(dev)
    ps = ops.stream_layout(pt, F, K)
    x = torch.randn(K, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(dev)
    a, b = (torch.empty(F // 2, dtype=torch.bfloat16, device=dev) for _ in range(2))
    ops.GemvBatch([(x, pt, ct, a, F, K, {"y": "silu_pairs"})]).run()
    ops.GemvBatch([(x, ps, ct, b, F, K, {"y": "silu_pairs"})], layout="sel").run()
    assert torch.equal(a, b)
    c, d = (torch.empty(F, dtype=torch.bfloat16, device=dev) for _ in range(2))
    ops.GemvBatch([(x, pt, ct, c, F, K), (x, pt, ct, c.clone(), F, K)]).run()
    ops.GemvBatch([(x, ps, ct, d, F, K), (x, ps, ct, d.clone(), F, K)], layout="sel").run()
    assert torch.equal(c, d)


def test_stream_layout_rejects(dev):
    pt = torch.zeros(48 * 4, dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError):
        ops.stream_layout(pt, 4, 200)
    with pytest.raises(ValueError):
        ops.stream_layout(pt, 8, 256)  # too few bytes
    x = torch.zeros(2, 128, dtype=torch.bfloat16, device=dev)
    cb = torch.zeros(4, 8, device=dev)
    with pytest.raises(ValueError):
        ops.GemvBatch([(x, pt, cb, torch.empty(2, 4, device=dev), 4, 128)], m=2, layout="sel")
