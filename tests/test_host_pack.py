"""Host-side format code (nativebit_amd.pack, .synth) against the oracle.

Mirrors the reference's own pack tests (tests/test_pack.py:25-151: round
trips, odd lengths, compression ratio, 4-bit and generic widths,
reconstruct_weight) and adds byte-exact agreement with the oracle stream and
the golden vectors.
"""
import numpy as np
import pytest
import torch

from nativebit_amd import pack as P
from nativebit_amd import synth
from oracle import oracle as O


def test_golden(golden):
    for v in golden["bitstream"]:
        got = P.pack_nbits(torch.tensor(v["indices"], dtype=torch.uint8), v["bits"])
        assert bytes(got.numpy()).hex() == v["hex"], v["name"]
        back = P.unpack_nbits(torch.from_numpy(np.frombuffer(bytes.fromhex(v["hex"]), np.uint8)),
                              len(v["indices"]), v["bits"])
        assert back.tolist() == v["indices"], v["name"]


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("n", [0, 1, 3, 7, 10, 13, 100, 1001, 100_000])
def test_matches_oracle(bits, n):
    rng = np.random.default_rng(1000 * bits + n)
    idx = rng.integers(0, 1 << bits, n, dtype=np.uint8)
    got = P.pack_nbits(torch.from_numpy(idx), bits).numpy()
    assert np.array_equal(got, O.pack(idx, bits))
    assert np.array_equal(P.unpack_nbits(torch.from_numpy(got), n, bits).numpy(), idx)


def test_reference_named_packers():
    idx = torch.randint(0, 8, (1001,), dtype=torch.uint8)
    assert torch.equal(P.unpack_3bit(P.pack_3bit(idx), 1001), idx)
    assert P.pack_3bit(torch.randint(0, 8, (8,), dtype=torch.uint8)).numel() == 3
    i4 = torch.randint(0, 16, (101,), dtype=torch.uint8)
    assert P.pack_4bit(i4[:100]).numel() == 50
    assert torch.equal(P.unpack_4bit(P.pack_4bit(i4), 101), i4)
    assert torch.equal(P.pack_nbits(idx[:24], 3), P.pack_3bit(idx[:24]))
    assert bytes(P.pack_indices_3bit(idx.numpy())) == bytes(P.pack_3bit(idx).numpy())


def test_reconstruct_weight_matches_oracle():
    rng = np.random.default_rng(11)
    nb, bs, ne = 7, 16, 8
    total = nb * bs - 9
    idx = rng.integers(0, ne, nb * bs, dtype=np.uint8)
    cb = rng.standard_normal((nb, ne)).astype(np.float32)
    w = P.reconstruct_weight(torch.from_numpy(idx), torch.from_numpy(cb), (total,), bs, total)
    assert np.array_equal(w.numpy(), O.dequant(idx, cb, bs, total))


def test_quantize_weight_matches_oracle():
    rng = np.random.default_rng(12)
    nb, bs, ne = 40, 128, 8
    w = (rng.standard_normal(nb * bs) * 0.02).astype(np.float32)
    cb = np.sort(rng.standard_normal((nb, ne)).astype(np.float32) * 0.02, axis=1)
    got = P.quantize_weight(w.reshape(40, 128), cb)
    assert np.array_equal(got.reshape(-1), O.quantize(w, cb, bs))


def test_synth_layer_is_consistent():
    lay = synth.make_layer(48, 256, n_entries=8, block_size=128, seed=3, keep_indices=True)
    assert lay.codebook.shape == (96, 8)
    # quantile codebooks are sorted and span each block's min..max
    assert torch.all(lay.codebook[:, 1:] >= lay.codebook[:, :-1])
    assert np.array_equal(lay.packed.numpy(), O.pack(lay.indices.numpy(), 3))
    gen = torch.Generator().manual_seed(3)
    w = torch.randn(48 * 256, generator=gen) * 0.02
    blocks = w.reshape(96, 128)
    assert torch.equal(lay.codebook[:, 0], blocks.min(dim=1).values)
    assert torch.equal(lay.codebook[:, -1], blocks.max(dim=1).values)
    assert np.array_equal(lay.indices.numpy(), O.quantize(w.numpy(), lay.codebook.numpy(), 128))


def test_layer_bytes_config0():
    # 6912x2560, NE 8, BS 128, x fp32, y fp32: the byte count the benchmark reports
    assert synth.layer_bytes(6912, 2560, 8, 128, x_bytes=4) == 11_097_088
    per_layer = sum(synth.layer_bytes(n, k, 8, 128) for _, n, k in synth.LAYER_SHAPES)
    assert per_layer == 49_712_640
