"""Pins the CPU oracle (oracle/) before anything is compared against it.

Each oracle function is checked against something that does not share its
code:

* pack / unpack / pack3_groups: hand-derived byte strings in
  tests/golden/known_answers.json (written from the format definition and
  cross-checked there against a big-integer closed form), the padding-length
  rules, round trips (the reference's own test cases, tests/test_pack.py:25-114),
  and agreement between the per-bit stream and the reference's bits24 form;
* dequant: the exact gather on golden cases and a hand example;
* matmul_f64 / matvec_3bit_k1: golden GEMVs whose exact rational answer is
  representable in fp32;
* quantize: brute force over entries on small inputs, with planted ties;
* round_bf16: hand-derived rounding cases and torch's own bf16 cast;
* torch_* restatements: equality with the C functions above.

A mutated oracle is shown to fail the golden vectors (planted on the CPU).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O


def hexbytes(h):
    return np.frombuffer(bytes.fromhex(h), dtype=np.uint8)


def test_golden_streams_pack(golden):
    for v in golden["bitstream"]:
        got = O.pack(v["indices"], v["bits"])
        assert got.tobytes().hex() == v["hex"], v["name"]


def test_golden_streams_unpack(golden):
    for v in golden["bitstream"]:
        got = O.unpack(hexbytes(v["hex"]), len(v["indices"]), v["bits"])
        assert got.tolist() == v["indices"], v["name"]


def test_golden_3bit_group_form(golden):
    for v in golden["bitstream"]:
        if v["bits"] == 3:
            assert O.pack3_groups(v["indices"]).tobytes().hex() == v["hex"], v["name"]


def test_lengths(golden):
    for e in golden["lengths"]:
        assert O.packed_nbytes(e["count"], e["bits"]) == e["nbytes"]


@pytest.mark.parametrize("n", [1, 3, 7, 10, 13, 100, 1001, 100_000])
@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 7, 8])
def test_roundtrip(n, bits):
    rng = np.random.default_rng(n * 31 + bits)
    idx = rng.integers(0, 1 << bits, n, dtype=np.uint8)
    p = O.pack(idx, bits)
    assert p.size == O.packed_nbytes(n, bits)
    assert np.array_equal(O.unpack(p, n, bits), idx)


@pytest.mark.parametrize("n", [8, 9, 24, 1001, 4096])
def test_stream_equals_group_form(n):
    rng = np.random.default_rng(n)
    idx = rng.integers(0, 8, n, dtype=np.uint8)
    assert np.array_equal(O.pack(idx, 3), O.pack3_groups(idx))


def test_all_zeros_and_sevens():
    for v in (0, 7):
        idx = np.full(16, v, dtype=np.uint8)
        p = O.pack(idx, 3)
        assert p.tobytes() == (b"\x00" * 6 if v == 0 else b"\xff" * 6)
        assert np.array_equal(O.unpack(p, 16, 3), idx)


def test_dequant_hand_example():
    cb = np.array([[0.5, -1.0, 2.0, 0.0], [3.0, 4.0, -5.0, 6.5]], dtype=np.float32)
    idx = np.array([2, 0, 1, 3, 3, 2, 1, 0], dtype=np.uint8)   # two blocks of 4
    w = O.dequant(idx, cb, 4, 7)                               # tail trimmed
    assert w.tolist() == [2.0, 0.5, -1.0, 0.0, 6.5, -5.0, 4.0]


def test_golden_gemv_dequant_and_f64(golden):
    for g in golden["gemv"]:
        N, K, bs = g["N"], g["K"], g["block_size"]
        cb = np.array(g["codebook"], dtype=np.float32)
        idx = O.unpack(hexbytes(g["packed_hex"]), len(g["indices"]), g["bits"])
        assert idx.tolist() == g["indices"], g["name"]
        w = O.dequant(idx, cb, bs, N * K).reshape(N, K)
        for i in (0, N * K // 2, N * K - 1):
            assert w.reshape(-1)[i] == cb[i // bs][g["indices"][i]]
        y = O.matmul_f64(np.array(g["x"], dtype=np.float32), w)[0]
        assert y.tolist() == g["y"], g["name"]


def test_k1_order_on_golden(golden):
    g = next(c for c in golden["gemv"] if c["name"] == "g3_n8_k256_bs128")
    y = O.matvec_3bit_k1(np.array(g["x"], np.float32), hexbytes(g["packed_hex"]),
                         np.array(g["codebook"], np.float32), g["N"], g["K"])
    assert y.tolist() == g["y"]


def test_k1_close_to_f64_random():
    rng = np.random.default_rng(5)
    N, K = 64, 512
    idx = rng.integers(0, 8, N * K, dtype=np.uint8)
    cb = rng.standard_normal((N * K // 128, 8)).astype(np.float32) * 0.02
    x = rng.standard_normal(K).astype(np.float32)
    p = O.pack(idx, 3)
    w = O.dequant(idx, cb, 128, N * K).reshape(N, K)
    ref = O.matmul_f64(x, w)[0]
    got = O.matvec_3bit_k1(x, p, cb, N, K)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-5


def test_quantize_brute_force_and_ties():
    rng = np.random.default_rng(7)
    nb, bs, ne = 6, 16, 8
    cb = np.sort(rng.standard_normal((nb, ne)).astype(np.float32), axis=1)
    w = rng.standard_normal(nb * bs - 5).astype(np.float32)
    # planted exact ties: the midpoint of two entries whose distances round equal
    cb[0] = np.array([-3, -2, -1, 0.25, 0.75, 2, 3, 4], dtype=np.float32)
    w[3] = 0.5
    idx = O.quantize(w, cb, bs)
    for i in range(nb * bs):
        v = w[i] if i < w.size else np.float32(0.0)
        c = cb[i // bs]
        d = [(v - c[e]) * (v - c[e]) for e in range(ne)]
        assert idx[i] == d.index(min(d)), i
    assert idx[3] == 3  # first of the tied entries 3 and 4


def test_round_bf16_cases():
    one = 1.0
    cases = {
        one: one,
        one + 2.0 ** -8: one,                       # tie -> even (mantissa 0)
        one + 3 * 2.0 ** -8: one + 2.0 ** -6,       # tie -> even (mantissa 2)
        one + 2.0 ** -8 + 2.0 ** -20: one + 2.0 ** -7,
        -2.5: -2.5,
    }
    for a, b in cases.items():
        assert float(O.round_bf16(np.float32(a))) == b, a
    rng = np.random.default_rng(3)
    v = (rng.standard_normal(2000) * 10.0 ** rng.integers(-30, 30, 2000)).astype(np.float32)
    ref = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    assert np.array_equal(O.round_bf16(v), ref)


@pytest.mark.parametrize("bits", [2, 3, 4, 5])
def test_torch_unpack_matches_c(bits):
    rng = np.random.default_rng(bits)
    nb, bs = 12, 64
    idx = rng.integers(0, 1 << bits, nb * bs, dtype=np.uint8)
    p = O.pack(idx, bits)
    t = O.torch_unpack_indices(torch.from_numpy(p), nb, bs, bits)
    assert np.array_equal(t.reshape(-1).numpy().astype(np.uint8), idx)


def test_torch_linear_matches_golden(golden):
    for g in golden["gemv"]:
        y = O.torch_packed_linear_f32(
            torch.tensor(g["x"], dtype=torch.float32), torch.from_numpy(hexbytes(g["packed_hex"])),
            torch.tensor(g["codebook"], dtype=torch.float32), g["N"], g["K"],
            g["block_size"], g["bits"])
        assert y.tolist() == g["y"], g["name"]
        yb = O.torch_packed_linear_bf16(
            torch.tensor(g["x"], dtype=torch.float32), torch.from_numpy(hexbytes(g["packed_hex"])),
            torch.tensor(g["codebook"], dtype=torch.float32), g["N"], g["K"],
            g["block_size"], g["bits"])
        # golden values are exact in bf16 inputs; the bf16 output rounds y
        assert torch.equal(yb.float(), torch.tensor(g["y"]).to(torch.bfloat16).float()), g["name"]


def test_planted_mistake_is_caught(golden):
    """An MSB-first packer (a plausible slip) disagrees with the golden set."""
    def msb_first(indices, bits):
        stream = []
        for v in indices:
            stream += [(v >> (bits - 1 - b)) & 1 for b in range(bits)]
        stream += [0] * (-len(stream) % 8)
        return bytes(np.packbits(np.array(stream, np.uint8), bitorder="little")).hex()

    wrong = sum(msb_first(v["indices"], v["bits"]) != v["hex"] for v in golden["bitstream"])
    assert wrong >= len(golden["bitstream"]) // 2
