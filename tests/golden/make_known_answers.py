"""Writes tests/golden/known_answers.json.

The fixture pins the packed-index format and the tiny-GEMV arithmetic without
running any reference code.  Two independent statements are recorded for
every bitstream vector:

* ``hex``: written down by hand from the format definition (index i occupies
  bits [i*b, (i+1)*b) of a little-endian, LSB-first stream;
  nativebit/pack.py:21-41, 75-82, 97-116; inference/pack.py:38-57).  For
  example [0..7] at 3 bits: bits24 = 0 + 1*8 + 2*64 + 3*512 + 4*4096 +
  5*32768 + 6*262144 + 7*2097152 = 0xFAC688, bytes 88 C6 FA.
* the closed form below (one big integer sum_i idx_i << (b*i), written out
  little endian), which this script checks against every hand-written hex.

The tiny GEMV cases use dyadic codebook values and small-integer activations,
so the exact result (computed here with Fractions) is representable in fp32
and any correct kernel must reproduce it bit for bit.

Run: python tests/golden/make_known_answers.py
"""
from __future__ import annotations

import json
import os
from fractions import Fraction

HERE = os.path.dirname(os.path.abspath(__file__))


def packed_len(n: int, bits: int) -> int:
    # 3-bit pads to whole 24-bit groups (nativebit/pack.py:29-32); others to
    # whole bytes (nativebit/pack.py:105-107, 79-80).
    if bits == 3:
        return 3 * ((n + 7) // 8)
    return (n * bits + 7) // 8


def closed_form(indices, bits: int) -> str:
    v = 0
    for i, x in enumerate(indices):
        assert 0 <= x < (1 << bits)
        v += x << (bits * i)
    return v.to_bytes(packed_len(len(indices), bits), "little").hex()


# (name, bits, indices, hand-written hex)
HAND = [
    ("3bit_ramp", 3, [0, 1, 2, 3, 4, 5, 6, 7], "88c6fa"),
    ("3bit_all7", 3, [7] * 8, "ffffff"),
    ("3bit_first1", 3, [1, 0, 0, 0, 0, 0, 0, 0], "010000"),
    ("3bit_i2_1", 3, [0, 0, 1, 0, 0, 0, 0, 0], "400000"),   # bit 6
    ("3bit_i2_4", 3, [0, 0, 4, 0, 0, 0, 0, 0], "000100"),   # bit 8
    ("3bit_i5_1", 3, [0, 0, 0, 0, 0, 1, 0, 0], "008000"),   # bit 15
    ("3bit_i5_2", 3, [0, 0, 0, 0, 0, 2, 0, 0], "000001"),   # bit 16
    ("3bit_single7", 3, [7], "070000"),                     # padded group
    ("3bit_len10", 3, [7] * 10, "ffffff3f0000"),            # 30 bits set
    ("3bit_two_groups", 3, [0, 0, 0, 0, 0, 0, 0, 0, 5, 0, 0, 0, 0, 0, 0, 1],
     "000000050020"),
    ("4bit_pair", 4, [1, 2], "21"),
    ("4bit_ramp", 4, list(range(16)), "1032547698badcfe"),
    ("4bit_odd", 4, [15, 1, 9], "1f09"),
    ("2bit_quad", 2, [1, 2, 3, 0], "39"),
    ("2bit_two", 2, [3, 2, 1, 0, 0, 1, 2, 3], "1be4"),
    ("2bit_len5", 2, [3, 3, 3, 3, 1], "ff01"),
    ("5bit_two", 5, [31, 1], "3f00"),                       # bits 0-4, bit 5
    ("1bit_byte", 1, [1, 0, 1, 1, 0, 0, 0, 1, 1], "8d01"),
    ("8bit_bytes", 8, [0, 255, 128], "00ff80"),
]

# Packed lengths from the padding rules (written independently from the
# rules quoted above).
LENGTHS = [
    (3, 1, 3), (3, 8, 3), (3, 10, 6), (3, 1001, 378), (3, 100000, 37500),
    (4, 100, 50), (4, 101, 51), (2, 100, 25), (2, 101, 26), (5, 50, 32),
    (1, 9, 2), (8, 7, 7), (3, 0, 0), (4, 0, 0),
]


def gemv_case(name, N, K, bs, bits, ne, seed):
    """A tiny GEMV whose exact answer is fp32-representable.

    cb[b][e] = (e - (ne-1)/2) * 2^-(b % 4) / 4, x[k] = ((3k + seed) % 7) - 3.
    Blocks tile the flat (N*K) weight array; the tail block is zero padded.
    """
    total = N * K
    nb = -(-total // bs)
    # a deterministic index pattern that exercises every entry
    idx = [((i * 5 + seed) * 7 + i // 3) % ne for i in range(nb * bs)]
    cb = [[Fraction(2 * e - (ne - 1), 2) / (4 * 2 ** (b % 4)) for e in range(ne)]
          for b in range(nb)]
    x = [((3 * k + seed) % 7) - 3 for k in range(K)]
    w = [cb[i // bs][idx[i]] for i in range(total)]
    y = [sum(Fraction(x[k]) * w[n * K + k] for k in range(K)) for n in range(N)]
    return {
        "name": name, "N": N, "K": K, "block_size": bs, "bits": bits,
        "n_entries": ne,
        "indices": idx,
        "packed_hex": closed_form(idx, bits),
        "codebook": [[float(v) for v in row] for row in cb],
        "x": x,
        "y": [float(v) for v in y],
        "y_exact": [str(v) for v in y],
    }


def main():
    vectors = []
    for name, bits, idx, hx in HAND:
        cf = closed_form(idx, bits)
        if cf != hx:
            raise SystemExit(f"{name}: hand {hx} != closed form {cf}")
        vectors.append({"name": name, "bits": bits, "indices": idx, "hex": hx})
    for bits, n, nbytes in LENGTHS:
        assert packed_len(n, bits) == nbytes, (bits, n)
    gemv = [
        gemv_case("g3_n4_k16_bs8", 4, 16, 8, 3, 8, 1),
        gemv_case("g3_ragged_n3_k10_bs8", 3, 10, 8, 3, 8, 2),
        gemv_case("g4_n5_k32_bs16", 5, 32, 16, 4, 16, 3),
        gemv_case("g2_n6_k64_bs32", 6, 64, 32, 2, 4, 4),
        gemv_case("g3_n8_k256_bs128", 8, 256, 128, 3, 8, 5),
        gemv_case("g3_ne5_n4_k24_bs8", 4, 24, 8, 3, 5, 6),
    ]
    for g in gemv:
        for v, e in zip(g["y"], g["y_exact"]):
            assert Fraction(v) == Fraction(e), (g["name"], v, e)  # fp64-exact
    out = {
        "about": "Known answers for NativeBit's packed-index stream and tiny "
                 "GEMVs; generated by make_known_answers.py.",
        "bitstream": vectors,
        "lengths": [{"bits": b, "count": n, "nbytes": m} for b, n, m in LENGTHS],
        "gemv": gemv,
    }
    path = os.path.join(HERE, "known_answers.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(f"wrote {path}: {len(vectors)} streams, {len(gemv)} gemv cases")


if __name__ == "__main__":
    main()
