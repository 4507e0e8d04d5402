/*
 * nb_oracle.c -- CPU restatement of NativeBit's packed-weight path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (nativebit_amd/) links,
 * loads or calls this file.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may use it, and only as the checker.
 *
 * Every function is written from the mathematics of the reference format, in
 * the plainest possible form (per-bit loops, fp64 sums), so that it can be
 * checked by hand and disagrees loudly with any vectorised or GPU version
 * that drops a term, swaps an index or mis-places a bit.
 *
 * Reference semantics followed (NorthernLightx/NativeBit):
 *   bitstream      nativebit/pack.py:21-41   (pack_3bit group formula)
 *                  nativebit/pack.py:75-82   (pack_4bit, low nibble first)
 *                  nativebit/pack.py:97-116  (pack_nbits, LSB-first per bit)
 *                  inference/pack.py:38-57   (pack_indices_3bit, bits24 LE)
 *                  inference/triton_kernel.py:199-220 (pack_indices_to_3bit)
 *   unpack         nativebit/pack.py:44-68, 85-90, 119-138
 *   dequant        nativebit/pack.py:145-169 (reconstruct_weight gather)
 *                  inference/triton_kernel.py:268-273, nativebit/inference.py:42-46
 *   quantize       inference/pack.py:21-35 (squared distance, first argmin)
 *                  nativebit/layers.py:78-94
 *   matvec order   inference/cuda_kernel.py:53-81 (fp32, per-row sequential)
 *
 * Pinning (see tests/test_oracle.py): hand-derived known answers in
 * tests/golden/, closed forms (round trips, lengths), exact rational
 * arithmetic on tiny GEMVs, and equality between the per-bit stream and the
 * 3-bit group formula.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

/* Packed byte count.  3-bit pads the index count to a multiple of 8 (one
 * 24-bit group = 3 bytes, nativebit/pack.py:29-32); every other width pads to
 * whole bytes (nativebit/pack.py:105-107; 4-bit: 79-80). */
size_t oracle_packed_nbytes(size_t count, int bits) {
    if (bits == 3) return ((count + 7) / 8) * 3;
    return (count * (size_t)bits + 7) / 8;
}

/* Index i occupies stream bits [i*bits, (i+1)*bits), least significant bit
 * first, bit k of the stream being bit (k % 8) of byte k / 8
 * (nativebit/pack.py:109-115).  Bytes past the last index are zero. */
void oracle_pack(const uint8_t* idx, size_t count, int bits, uint8_t* out) {
    size_t nbytes = oracle_packed_nbytes(count, bits);
    memset(out, 0, nbytes);
    size_t pos = 0;
    for (size_t i = 0; i < count; ++i) {
        unsigned v = idx[i];
        for (int b = 0; b < bits; ++b, ++pos) {
            if ((v >> b) & 1u) out[pos / 8] |= (uint8_t)(1u << (pos % 8));
        }
    }
}

/* Inverse of oracle_pack (nativebit/pack.py:126-138). */
void oracle_unpack(const uint8_t* packed, size_t count, int bits, uint8_t* out) {
    size_t pos = 0;
    for (size_t i = 0; i < count; ++i) {
        unsigned v = 0;
        for (int b = 0; b < bits; ++b, ++pos) {
            unsigned bit = (packed[pos / 8] >> (pos % 8)) & 1u;
            v |= bit << b;
        }
        out[i] = (uint8_t)v;
    }
}

/* The 3-bit packer as the reference writes it: eight indices form
 * bits24 = sum_j i_j << 3j, stored little endian (inference/pack.py:49-56,
 * nativebit/pack.py:37-41).  Kept separate from oracle_pack so the tests can
 * show the two statements agree. */
void oracle_pack3_groups(const uint8_t* idx, size_t count, uint8_t* out) {
    size_t groups = (count + 7) / 8;
    for (size_t g = 0; g < groups; ++g) {
        uint32_t bits24 = 0;
        for (int j = 0; j < 8; ++j) {
            size_t i = g * 8 + (size_t)j;
            uint32_t v = i < count ? (idx[i] & 7u) : 0u;
            bits24 |= v << (3 * j);
        }
        out[3 * g + 0] = (uint8_t)(bits24 & 0xFFu);
        out[3 * g + 1] = (uint8_t)((bits24 >> 8) & 0xFFu);
        out[3 * g + 2] = (uint8_t)((bits24 >> 16) & 0xFFu);
    }
}

/* reconstruct_weight (nativebit/pack.py:145-169): w[i] = cb[i / bs][idx[i]]
 * for i < total.  An exact copy of a codebook entry, no arithmetic. */
void oracle_dequant(const uint8_t* idx, const float* cb, size_t num_blocks,
                    int n_entries, int block_size, size_t total, float* w) {
    (void)num_blocks;
    for (size_t i = 0; i < total; ++i) {
        size_t blk = i / (size_t)block_size;
        w[i] = cb[blk * (size_t)n_entries + idx[i]];
    }
}

/* torch's float -> bfloat16 conversion (round to nearest, ties to even; NaN
 * stays NaN), as used by W.to(torch.bfloat16) in inference/eval_ppl.py:166.
 * Returns the bf16 value widened back to float. */
float oracle_round_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) {
        u = (u | 0x00400000u) & 0xFFFF0000u;  /* quiet NaN */
    } else {
        uint32_t lsb = (u >> 16) & 1u;
        u = (u + 0x7FFFu + lsb) & 0xFFFF0000u;
    }
    float r;
    memcpy(&r, &u, 4);
    return r;
}

/* y[m][n] = sum_k x[m][k] * w[n][k] with every product and sum in fp64:
 * the brute-force reference the GEMV kernels are held to (the reference's
 * own matmul is torch/BLAS and pins nothing). */
void oracle_matmul_f64(const float* x, int M, int K, const float* w, int N,
                       double* y) {
    for (int m = 0; m < M; ++m) {
        const float* xr = x + (size_t)m * K;
        for (int n = 0; n < N; ++n) {
            const float* wr = w + (size_t)n * K;
            double acc = 0.0;
            for (int k = 0; k < K; ++k) acc += (double)xr[k] * (double)wr[k];
            y[(size_t)m * N + n] = acc;
        }
    }
}

/* The reference device kernel's arithmetic, fp32 in its exact order
 * (inference/cuda_kernel.py:53-81): one output row at a time, blocks of 128
 * in order, groups of 8 in order, acc += cb[idx] * x.  Only defined for
 * 3-bit, 8 entries, block 128 and K % 128 == 0, as the reference kernel. */
void oracle_matvec_3bit_k1(const float* x, const uint8_t* packed,
                           const float* cb, int N, int K, float* y) {
    const int bpr = K / 128;
    for (int r = 0; r < N; ++r) {
        float acc = 0.0f;
        for (int kb = 0; kb < bpr; ++kb) {
            size_t block = (size_t)r * bpr + kb;
            const uint8_t* pb = packed + block * 48;
            const float* c = cb + block * 8;
            for (int g = 0; g < 16; ++g) {
                uint32_t bits24 = (uint32_t)pb[g * 3] |
                                  ((uint32_t)pb[g * 3 + 1] << 8) |
                                  ((uint32_t)pb[g * 3 + 2] << 16);
                for (int j = 0; j < 8; ++j) {
                    int i = (bits24 >> (3 * j)) & 7;
                    acc = fmaf(c[i], x[kb * 128 + g * 8 + j], acc);
                }
            }
        }
        y[r] = acc;
    }
}

/* Nearest-entry assignment with squared distance and the first minimum on
 * ties (inference/pack.py:21-35, numpy argmin; nativebit/layers.py:88-90).
 * Weights past `total` count as 0.0, as the reference zero-pads the flat
 * tail.  The distance is computed in fp32 like the reference. */
void oracle_quantize(const float* w, size_t total, const float* cb,
                     size_t num_blocks, int n_entries, int block_size,
                     uint8_t* idx) {
    for (size_t b = 0; b < num_blocks; ++b) {
        const float* c = cb + b * (size_t)n_entries;
        for (int j = 0; j < block_size; ++j) {
            size_t i = b * (size_t)block_size + (size_t)j;
            float v = i < total ? w[i] : 0.0f;
            int best = 0;
            float bd = (v - c[0]) * (v - c[0]);
            for (int e = 1; e < n_entries; ++e) {
                float d = (v - c[e]) * (v - c[e]);
                if (d < bd) { bd = d; best = e; }
            }
            idx[i] = (uint8_t)best;
        }
    }
}
