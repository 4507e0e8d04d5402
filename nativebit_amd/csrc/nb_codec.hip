// Bit-exact format kernels: unpack, pack and dequantize NativeBit index
// streams on gfx950 (their outputs must equal the reference's byte for
// byte).  The bulk of a stream goes through chunk kernels: a chunk is 32
// indices = 4 groups of 8 = BITS whole dwords of the LSB-first stream, so a
// thread moves BITS dwords one way and 32 index bytes (or 32 weights) the
// other with wide loads and stores, its field offsets fixed at compile time.
// The last count % 32 indices, and pointers without the chunk kernels'
// alignment, go through per-element grid-stride kernels.
//
// Reference semantics: nativebit/pack.py:21-169 (pack_3bit, unpack_3bit,
// pack_4bit, unpack_4bit, pack_nbits, unpack_nbits, reconstruct_weight),
// inference/triton_kernel.py:199-220 (pack_indices_to_3bit),
// inference/pack.py:21-35 (quantize_weight, fused here with the pack).
#include <math.h>

#include <type_traits>

#include "nb_device.h"
#include "nb_internal.h"

namespace nb {
namespace {

constexpr int kThreads = 256;

// Grid for a grid-stride loop over `n` items: enough workgroups to cover
// every CU several times, never more than needed.
inline int grid_for(int64_t n) {
    int64_t want = (n + kThreads - 1) / kThreads;
    int64_t cap = (int64_t)device_cu_count() * 16;
    if (want < 1) want = 1;
    return (int)(want < cap ? want : cap);
}

__global__ __launch_bounds__(kThreads) void unpack_kernel(
    const uint8_t* __restrict__ packed, int64_t nbytes,
    uint8_t* __restrict__ out, int64_t first, int64_t count, int bits) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = first + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < count;
         i += stride) {
        out[i] = (uint8_t)read_field(packed, nbytes, i, bits);
    }
}

// One output byte per iteration: byte b holds stream bits [8b, 8b+8), i.e.
// the fields of indices floor(8b/bits) .. floor((8b+7)/bits).
__global__ __launch_bounds__(kThreads) void pack_kernel(
    const uint8_t* __restrict__ idx, int64_t count, int bits,
    uint8_t* __restrict__ out, int64_t first_byte, int64_t nbytes) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    const uint32_t mask = (1u << bits) - 1u;
    for (int64_t b = first_byte + (int64_t)blockIdx.x * kThreads + threadIdx.x; b < nbytes;
         b += stride) {
        const int64_t first_bit = b * 8;
        const int64_t i0 = first_bit / bits;
        const int64_t i1 = (first_bit + 7) / bits;
        uint32_t v = 0;
        for (int64_t i = i0; i <= i1 && i < count; ++i) {
            const int64_t shift = i * bits - first_bit;  // in (-bits, 8)
            const uint32_t f = idx[i] & mask;
            v |= shift >= 0 ? (f << shift) : (f >> (-shift));
        }
        out[b] = (uint8_t)(v & 0xFFu);
    }
}

// Nearest codebook entry of flat weight i: squared distance (w - c)^2 to
// each entry of its block's codebook in fp32, the first index on ties
// (strict <, as numpy's and torch's argmin); weights at or past `total`
// (the padded tail of the last block) are 0.0.  Inputs are finite.
__device__ __forceinline__ uint32_t nearest_entry(const float* __restrict__ w, int64_t total,
                                                  const float* __restrict__ cb, int n_entries,
                                                  int64_t blk, int64_t i) {
    const float v = i < total ? w[i] : 0.f;
    const float* c = cb + blk * n_entries;
    float d = v - c[0];
    float best_d = d * d;
    uint32_t best = 0;
    for (int e = 1; e < n_entries; ++e) {
        d = v - c[e];
        const float dd = d * d;
        if (dd < best_d) {
            best_d = dd;
            best = (uint32_t)e;
        }
    }
    return best;
}

// Quantize-at-pack: one thread per group of 8 indices, i.e. `bits` whole
// bytes of the LSB-first stream (8 fields of `bits` bits), each field the
// weight's nearest entry, so the (blocks x block_size x entries) distance
// tensor of the reference's quantize_weight never exists
// (inference/pack.py:21-35).  Up to 16 entries the block's codebook stays in
// registers while consecutive indices share a block; NE (4, 8 or 16, else
// 0 = any count up to 16) fixes the compare loop's length.
template <bool kSmallNE, int NE>
__global__ __launch_bounds__(kThreads) void quantize_pack_kernel(
    const float* __restrict__ w, int64_t total, const float* __restrict__ cb, int n_entries,
    int block_size, int64_t count, int bits, uint8_t* __restrict__ out, int64_t nbytes,
    int64_t first_group) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    const int64_t groups = (count + 7) / 8;
    for (int64_t t = first_group + (int64_t)blockIdx.x * kThreads + threadIdx.x; t < groups;
         t += stride) {
        float c[16];
        int64_t cur_block = -1;
        uint64_t acc = 0;  // 8 fields, LSB first (8 * bits <= 64)
        // block of index 8t + j, advanced one index at a time (one division
        // per group, not per weight)
        int64_t blk = (8 * t) / block_size;
        int in_blk = (int)(8 * t - blk * block_size);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int64_t i = 8 * t + j;
            if (j > 0 && ++in_blk == block_size) {
                in_blk = 0;
                ++blk;
            }
            uint32_t f = 0;
            if (i < count) {
                if (kSmallNE) {
                    const float v = i < total ? w[i] : 0.f;
                    constexpr int kE = NE ? NE : 16;
                    if (blk != cur_block) {
                        cur_block = blk;
#pragma unroll
                        for (int e = 0; e < kE; ++e) c[e] = e < n_entries ? cb[blk * n_entries + e] : 0.f;
                    }
                    float d = v - c[0];
                    float best_d = d * d;
#pragma unroll
                    for (int e = 1; e < kE; ++e) {
                        d = v - c[e];
                        const float dd = d * d;
                        if ((NE || e < n_entries) && dd < best_d) {
                            best_d = dd;
                            f = (uint32_t)e;
                        }
                    }
                } else {
                    f = nearest_entry(w, total, cb, n_entries, blk, i);
                }
            }
            acc |= (uint64_t)f << (j * bits);
        }
        // bytes bits * t .. bits * t + bits - 1 of the stream
        for (int k = 0; k < bits; ++k) {
            const int64_t ob = (int64_t)bits * t + k;
            if (ob < nbytes) out[ob] = (uint8_t)(acc >> (8 * k));
        }
    }
}

// Quantize-at-pack for the standard formats (NE = 2^BITS entries, blocks a
// multiple of 32 weights): one thread per chunk of 32 real weights, which
// lies in one block -- the block's NE entries and the 32 weights come in
// with vector loads, the nearest-entry search is the same squared-distance
// compare (first index on ties), and the 32 fields leave as BITS dwords.
template <int BITS>
__global__ __launch_bounds__(kThreads) void quantize_chunks_kernel(
    const float4* __restrict__ w, const float4* __restrict__ cb, int block_size,
    uint32_t* __restrict__ out, int64_t chunks) {
    constexpr int NE = 1 << BITS;
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x; c < chunks; c += stride) {
        const float4* tp = cb + (c * 32 / block_size) * (NE / 4);
        float t[NE];
#pragma unroll
        for (int q = 0; q < NE / 4; ++q) {
            const float4 u = tp[q];
            t[4 * q] = u.x;
            t[4 * q + 1] = u.y;
            t[4 * q + 2] = u.z;
            t[4 * q + 3] = u.w;
        }
        float v[32];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float4 u = w[8 * c + q];
            v[4 * q] = u.x;
            v[4 * q + 1] = u.y;
            v[4 * q + 2] = u.z;
            v[4 * q + 3] = u.w;
        }
        uint32_t o[BITS];
#pragma unroll
        for (int k = 0; k < BITS; ++k) o[k] = 0;
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            float d = v[j] - t[0];
            float best_d = d * d;
            uint32_t f = 0;
#pragma unroll
            for (int e = 1; e < NE; ++e) {
                d = v[j] - t[e];
                const float dd = d * d;
                if (dd < best_d) {
                    best_d = dd;
                    f = (uint32_t)e;
                }
            }
            const int bit = j * BITS;
            o[bit >> 5] |= f << (bit & 31);
            if ((bit & 31) + BITS > 32) o[(bit >> 5) + 1] |= f >> (32 - (bit & 31));
        }
#pragma unroll
        for (int k = 0; k < BITS; ++k) out[c * BITS + k] = o[k];
    }
}

// Per-block quantile codebooks: cb[b][e] = quantile(w_block, q_e) with
// linear interpolation, as torch.quantile(w_block, linspace(0, 1, NE))
// (nativebit/codebook_utils.py:6-22, called per block by
// nativebit/layers.py:76): sort the block, rank = q_e * (n - 1) in fp32,
// lower = (int) rank, upper = ceil(rank), weight = rank - lower, and
// torch's lerp, which rounds once: fma(weight, hi - lo, lo) for weight < 0.5,
// else fma(weight - 1, hi - lo, hi).  The last block takes only the weights
// that exist (n = total - first).  One 64-lane workgroup per block: the
// block is sorted in LDS by a bitonic network over the next power of two
// (+inf padding), every compare-exchange of a pass on its own lane, a
// barrier between passes.  Inputs are finite.
constexpr int kCbMaxBlock = 1024;
constexpr int kCbMaxEntries = 256;
struct QuantileFractions {
    float q[kCbMaxEntries];
};

__global__ __launch_bounds__(64) void block_codebooks_kernel(
    const float* __restrict__ w, int64_t total, int64_t num_blocks, int block_size, int n_entries,
    QuantileFractions qf, float* __restrict__ cb) {
    __shared__ float v[kCbMaxBlock];
    const int lane = threadIdx.x;
    for (int64_t b = blockIdx.x; b < num_blocks; b += gridDim.x) {
        const int64_t first = b * block_size;
        const int n = (int)min((int64_t)block_size, total - first);
        int P = 1;
        while (P < n) P <<= 1;
        for (int i = lane; i < P; i += 64) v[i] = i < n ? w[first + i] : INFINITY;
        __syncthreads();
        for (int k = 2; k <= P; k <<= 1) {
            for (int j = k >> 1; j > 0; j >>= 1) {
                for (int t = lane; t < P / 2; t += 64) {
                    // pair (i, i + j) of pass (k, j)
                    const int i = ((t / j) * 2 * j) + (t % j);
                    const float a = v[i], c = v[i + j];
                    const bool up = (i & k) == 0;
                    if ((a > c) == up) {
                        v[i] = c;
                        v[i + j] = a;
                    }
                }
                __syncthreads();
            }
        }
        const float last_index = (float)(n - 1);
        for (int e = lane; e < n_entries; e += 64) {
            // each product and difference rounded on its own, as torch's
            // CPU quantile computes them: no contraction into fma here
#pragma clang fp contract(off)
            const float rank = qf.q[e] * last_index;
            const int lo = (int)rank;
            const int hi = (int)ceilf(rank);
            const float wt = rank - (float)lo;
            const float a = v[lo], c = v[hi];
            const float r = fabsf(wt) < 0.5f ? __builtin_fmaf(wt, c - a, a)
                                             : __builtin_fmaf(wt - 1.0f, c - a, c);
            cb[b * n_entries + e] = r;
        }
        __syncthreads();
    }
}

// The same codebooks for blocks of at most 64 * H weights, sorted in one
// wave's registers: value i of the (+inf padded) block sits in lane i % 64,
// slot i / 64; each bitonic pass pairs i with i ^ j (a cross-lane shuffle for
// j < 64, another slot of the same lane otherwise) and keeps the min or the
// max, so no LDS and no barrier is involved.  Entries are then formed as in
// block_codebooks_kernel from values fetched by shuffles.
template <int H>
__device__ __forceinline__ float sorted_at(const float (&v)[H], int idx) {
    float r = __shfl(v[0], idx & 63, 64);
#pragma unroll
    for (int h = 1; h < H; ++h) {
        const float u = __shfl(v[h], idx & 63, 64);
        r = (idx >> 6) == h ? u : r;
    }
    return r;
}

template <int H>
__global__ __launch_bounds__(kThreads) void block_codebooks_wave_kernel(
    const float* __restrict__ w, int64_t total, int64_t num_blocks, int block_size, int n_entries,
    QuantileFractions qf, float* __restrict__ cb) {
    constexpr int P = 64 * H;
    const int lane = threadIdx.x & 63;
    const int64_t nwaves = ((int64_t)gridDim.x * kThreads) >> 6;
    for (int64_t b = ((int64_t)blockIdx.x * kThreads + threadIdx.x) >> 6; b < num_blocks;
         b += nwaves) {
        const int64_t first = b * block_size;
        const int n = (int)min((int64_t)block_size, total - first);
        float v[H];
#pragma unroll
        for (int h = 0; h < H; ++h) {
            const int i = lane + 64 * h;
            v[h] = i < n ? w[first + i] : INFINITY;
        }
#pragma unroll
        for (int k = 2; k <= P; k <<= 1) {
#pragma unroll
            for (int j = k >> 1; j > 0; j >>= 1) {
                float o[H];
#pragma unroll
                for (int h = 0; h < H; ++h) {
                    o[h] = j < 64 ? __shfl_xor(v[h], j, 64) : v[h ^ (j >> 6)];
                }
#pragma unroll
                for (int h = 0; h < H; ++h) {
                    const int i = lane + 64 * h;
                    const bool keep_min = ((i & j) == 0) == ((i & k) == 0);
                    v[h] = keep_min ? fminf(v[h], o[h]) : fmaxf(v[h], o[h]);
                }
            }
        }
        const float last_index = (float)(n - 1);
        for (int e0 = 0; e0 < n_entries; e0 += 64) {  // uniform: every lane shuffles
            const int e = e0 + lane;
            float rank, wt;
            int lo, hi;
            {
                // each product and difference rounded on its own, as torch's
                // CPU quantile computes them: no contraction into fma here
#pragma clang fp contract(off)
                rank = qf.q[e < n_entries ? e : 0] * last_index;
                lo = (int)rank;
                hi = (int)ceilf(rank);
                wt = rank - (float)lo;
            }
            const float a = sorted_at<H>(v, lo), c = sorted_at<H>(v, hi);
            const float r = fabsf(wt) < 0.5f ? __builtin_fmaf(wt, c - a, a)
                                             : __builtin_fmaf(wt - 1.0f, c - a, c);
            if (e < n_entries) cb[b * n_entries + e] = r;
        }
    }
}

template <bool kBF16>
__global__ __launch_bounds__(kThreads) void dequant_kernel(
    const uint8_t* __restrict__ packed, int64_t nbytes,
    const float* __restrict__ cb, void* __restrict__ w, int64_t first, int64_t total,
    int bits, int n_entries, int block_size) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    const uint32_t last = (uint32_t)(n_entries - 1);
    for (int64_t i = first + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
         i += stride) {
        uint32_t e = read_field(packed, nbytes, i, bits);
        e = e < last ? e : last;
        const float v = cb[(i / block_size) * n_entries + e];
        if (kBF16) {
            static_cast<bf16_bits*>(w)[i] = f32_to_bf16_rne(v);
        } else {
            static_cast<float*>(w)[i] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// chunk kernels (32 indices <-> BITS dwords)
// ---------------------------------------------------------------------------
// Field j (0..31) of a chunk: bits [j*BITS, (j+1)*BITS) of the little-endian
// dwords d; j is a constant once the callers' loops are unrolled.
template <int BITS>
__device__ __forceinline__ uint32_t chunk_field(const uint32_t (&d)[BITS], int j) {
    const int bit = j * BITS;
    const int w = bit >> 5;
    const int off = bit & 31;
    const uint32_t mask = (1u << BITS) - 1u;
    if (off + BITS > 32) return __builtin_amdgcn_alignbit(d[w + 1], d[w], off) & mask;
    return (d[w] >> off) & mask;
}

template <int BITS>
__device__ __forceinline__ void load_chunk(const uint32_t* __restrict__ packed, int64_t c,
                                           uint32_t (&d)[BITS]) {
    const uint32_t* p = packed + c * BITS;
#pragma unroll
    for (int w = 0; w < BITS; ++w) d[w] = __builtin_nontemporal_load(p + w);
}

// Stores the Q 16-byte pieces of each lane's chunk so that every store
// instruction of the wave writes 64 consecutive pieces (1 KiB): the pieces go
// through the wave's LDS area (lane pitch Q + 1 pieces) and come back in
// output order.  Lane l holds chunk c0 + l; pieces at or past `limit` (the
// end of the output, counted from dst) are not stored.  Every lane of the
// wave calls this.  A wave's LDS operations complete in issue order, so the
// fences only keep the compiler from moving the accesses.
template <int Q>
__device__ __forceinline__ void wave_store_pieces(uint4* __restrict__ lds, const uint4 (&v)[Q],
                                                  uint4* __restrict__ dst, int64_t c0,
                                                  int64_t limit, int lane) {
#pragma unroll
    for (int q = 0; q < Q; ++q) lds[lane * (Q + 1) + q] = v[q];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int k = 0; k < Q; ++k) {
        const int i = k * 64 + lane;  // piece of the wave's output
        const uint4 u = lds[(i / Q) * (Q + 1) + (i % Q)];
        const int64_t o = c0 * Q + i;
        if (o < limit) dst[o] = u;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Grid-stride over chunks in whole waves: the loop condition is the wave's
// first chunk, so every lane of a wave runs the same iterations (the wave
// store needs all of them); lanes past the last chunk compute on chunk 0
// and store nothing.
#define NB_CHUNK_LOOP(chunks)                                                        \
    const int lane = threadIdx.x & 63;                                               \
    const int64_t stride = (int64_t)gridDim.x * kThreads;                            \
    for (int64_t c0 = (int64_t)blockIdx.x * kThreads + (threadIdx.x & ~63); c0 < (chunks); \
         c0 += stride)

template <int BITS>
__global__ __launch_bounds__(kThreads) void unpack_chunks_kernel(
    const uint32_t* __restrict__ packed, uint4* __restrict__ out, int64_t chunks) {
    __shared__ uint4 lds[kThreads / 64][64 * 3];
    NB_CHUNK_LOOP(chunks) {
        const int64_t c = c0 + lane < chunks ? c0 + lane : 0;
        uint32_t d[BITS];
        load_chunk<BITS>(packed, c, d);
        uint32_t o[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            o[k] = chunk_field<BITS>(d, 4 * k) | (chunk_field<BITS>(d, 4 * k + 1) << 8) |
                   (chunk_field<BITS>(d, 4 * k + 2) << 16) | (chunk_field<BITS>(d, 4 * k + 3) << 24);
        }
        const uint4 v[2] = {make_uint4(o[0], o[1], o[2], o[3]), make_uint4(o[4], o[5], o[6], o[7])};
        wave_store_pieces<2>(lds[threadIdx.x >> 6], v, out, c0, 2 * chunks, lane);
    }
}

template <int BITS>
__global__ __launch_bounds__(kThreads) void pack_chunks_kernel(
    const uint4* __restrict__ idx, uint32_t* __restrict__ out, int64_t chunks) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    const uint32_t mask = (1u << BITS) - 1u;
    for (int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x; c < chunks; c += stride) {
        const uint4 a = idx[2 * c], b = idx[2 * c + 1];
        const uint32_t in[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint32_t o[BITS];
#pragma unroll
        for (int w = 0; w < BITS; ++w) o[w] = 0;
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const uint32_t f = (in[j >> 2] >> (8 * (j & 3))) & mask;
            const int bit = j * BITS;
            const int w = bit >> 5;
            const int off = bit & 31;
            o[w] |= f << off;
            if (off + BITS > 32) o[w + 1] |= f >> (32 - off);
        }
        uint32_t* p = out + c * BITS;
#pragma unroll
        for (int w = 0; w < BITS; ++w) p[w] = o[w];
    }
}

// Two finite fp32 values rounded to bf16 (nearest, ties to even), packed low
// | high: gfx950 converts a pair in one instruction (v_cvt_pk_bf16_f32).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2_rne(float lo, float hi) {
    const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

// block_size % 32 == 0, so a chunk lies inside one block.
template <int BITS, bool kBF16>
__global__ __launch_bounds__(kThreads) void dequant_chunks_kernel(
    const uint32_t* __restrict__ packed, const float* __restrict__ cb, void* __restrict__ w,
    int64_t chunks, int n_entries, int block_size) {
    constexpr int Q = kBF16 ? 4 : 8;  // 16-byte pieces per chunk
    __shared__ uint4 lds[kThreads / 64][64 * (Q + 1)];
    const uint32_t last = (uint32_t)(n_entries - 1);
    NB_CHUNK_LOOP(chunks) {
        const int64_t c = c0 + lane < chunks ? c0 + lane : 0;
        uint32_t d[BITS];
        load_chunk<BITS>(packed, c, d);
        const float* tab = cb + (c * 32 / block_size) * n_entries;
        float v[32];
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const uint32_t e = chunk_field<BITS>(d, j);
            v[j] = tab[e < last ? e : last];
        }
        uint4 pc[Q];
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            if (kBF16) {
                uint32_t h[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) h[k] = pack_bf16x2_rne(v[8 * q + 2 * k], v[8 * q + 2 * k + 1]);
                pc[q] = make_uint4(h[0], h[1], h[2], h[3]);
            } else {
                pc[q] = make_uint4(__float_as_uint(v[4 * q]), __float_as_uint(v[4 * q + 1]),
                                   __float_as_uint(v[4 * q + 2]), __float_as_uint(v[4 * q + 3]));
            }
        }
        wave_store_pieces<Q>(lds[threadIdx.x >> 6], pc, static_cast<uint4*>(w), c0, Q * chunks,
                             lane);
    }
}

// f(std::integral_constant<int, bits>) for bits 1..8.
template <typename F>
void with_bits(int bits, F&& f) {
    switch (bits) {
        case 1: f(std::integral_constant<int, 1>{}); break;
        case 2: f(std::integral_constant<int, 2>{}); break;
        case 3: f(std::integral_constant<int, 3>{}); break;
        case 4: f(std::integral_constant<int, 4>{}); break;
        case 5: f(std::integral_constant<int, 5>{}); break;
        case 6: f(std::integral_constant<int, 6>{}); break;
        case 7: f(std::integral_constant<int, 7>{}); break;
        case 8: f(std::integral_constant<int, 8>{}); break;
    }
}

inline bool is_aligned(const void* p, uintptr_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

}  // namespace

int launch_unpack(const uint8_t* packed, uint8_t* out, int64_t count, int bits,
                  hipStream_t stream) {
    if (count == 0) return NB_OK;
    const int64_t nbytes = packed_nbytes(count, bits);
    int64_t first = 0;
    if (is_aligned(packed, 4) && is_aligned(out, 16)) {
        const int64_t chunks = count / 32;
        if (chunks > 0) {
            with_bits(bits, [&](auto B) {
                hipLaunchKernelGGL(unpack_chunks_kernel<decltype(B)::value>, dim3(grid_for(chunks)),
                                   dim3(kThreads), 0, stream,
                                   reinterpret_cast<const uint32_t*>(packed),
                                   reinterpret_cast<uint4*>(out), chunks);
            });
            first = chunks * 32;
        }
    }
    if (first < count) {
        hipLaunchKernelGGL(unpack_kernel, dim3(grid_for(count - first)), dim3(kThreads), 0,
                           stream, packed, nbytes, out, first, count, bits);
    }
    return check_launch("nb_unpack");
}

int launch_pack(const uint8_t* idx, uint8_t* out, int64_t count, int bits,
                hipStream_t stream) {
    const int64_t nbytes = packed_nbytes(count, bits);
    if (nbytes == 0) return NB_OK;
    // chunk c writes stream bytes [4 * bits * c, 4 * bits * (c + 1)) from
    // indices [32c, 32c + 32); the per-byte kernel writes the rest, padding
    // included
    int64_t first_byte = 0;
    if (is_aligned(idx, 16) && is_aligned(out, 4)) {
        const int64_t chunks = count / 32;
        if (chunks > 0) {
            with_bits(bits, [&](auto B) {
                hipLaunchKernelGGL(pack_chunks_kernel<decltype(B)::value>, dim3(grid_for(chunks)),
                                   dim3(kThreads), 0, stream,
                                   reinterpret_cast<const uint4*>(idx),
                                   reinterpret_cast<uint32_t*>(out), chunks);
            });
            first_byte = chunks * 4 * bits;
        }
    }
    if (first_byte < nbytes) {
        hipLaunchKernelGGL(pack_kernel, dim3(grid_for(nbytes - first_byte)), dim3(kThreads), 0,
                           stream, idx, count, bits, out, first_byte, nbytes);
    }
    return check_launch("nb_pack");
}

int launch_quantize_pack(const float* w, int64_t total, const float* codebook,
                         int64_t num_blocks, int n_entries, int block_size, int bits,
                         uint8_t* out, hipStream_t stream) {
    const int64_t count = num_blocks * block_size;
    const int64_t nbytes = packed_nbytes(count, bits);
    if (nbytes == 0) return NB_OK;
    // chunks of 32 real weights in the standard formats; the general kernel
    // takes the remaining groups (the tail and the zero-padded weights)
    int64_t first_group = 0;
    if ((n_entries == 4 || n_entries == 8 || n_entries == 16) && n_entries == (1 << bits) &&
        block_size % 32 == 0 && is_aligned(w, 16) && is_aligned(codebook, 16) &&
        is_aligned(out, 4)) {
        const int64_t chunks = total / 32;
        if (chunks > 0) {
            auto chunk = [&](auto kernel) {
                hipLaunchKernelGGL(kernel, dim3(grid_for(chunks)), dim3(kThreads), 0, stream,
                                   reinterpret_cast<const float4*>(w),
                                   reinterpret_cast<const float4*>(codebook), block_size,
                                   reinterpret_cast<uint32_t*>(out), chunks);
            };
            if (bits == 2) chunk(quantize_chunks_kernel<2>);
            if (bits == 3) chunk(quantize_chunks_kernel<3>);
            if (bits == 4) chunk(quantize_chunks_kernel<4>);
            first_group = chunks * 4;
        }
    }
    const int64_t groups = (count + 7) / 8;
    if (first_group >= groups) return check_launch("nb_quantize_pack");
    const int grid = grid_for(groups - first_group);
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), 0, stream, w, total, codebook,
                           n_entries, block_size, count, bits, out, nbytes, first_group);
    };
    switch (n_entries) {
        case 4: go(quantize_pack_kernel<true, 4>); break;
        case 8: go(quantize_pack_kernel<true, 8>); break;
        case 16: go(quantize_pack_kernel<true, 16>); break;
        default:
            if (n_entries < 16) {
                go(quantize_pack_kernel<true, 0>);
            } else {
                go(quantize_pack_kernel<false, 0>);
            }
    }
    return check_launch("nb_quantize_pack");
}

int launch_block_codebooks(const float* w, int64_t total, int64_t num_blocks, int block_size,
                           int n_entries, const float* q, float* cb, hipStream_t stream) {
    if (num_blocks == 0) return NB_OK;
    QuantileFractions qf;
    for (int e = 0; e < kCbMaxEntries; ++e) qf.q[e] = e < n_entries ? q[e] : 0.f;
    if (block_size <= 256) {
        const int64_t want = (num_blocks + kThreads / 64 - 1) / (kThreads / 64);
        const int64_t cap = (int64_t)device_cu_count() * 16;
        const int grid = (int)(want < cap ? want : cap);
        auto go = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), 0, stream, w, total,
                               num_blocks, block_size, n_entries, qf, cb);
        };
        if (block_size <= 64) {
            go(block_codebooks_wave_kernel<1>);
        } else if (block_size <= 128) {
            go(block_codebooks_wave_kernel<2>);
        } else {
            go(block_codebooks_wave_kernel<4>);
        }
        return check_launch("nb_block_codebooks");
    }
    int64_t grid = num_blocks;
    const int64_t cap = (int64_t)device_cu_count() * 32;
    if (grid > cap) grid = cap;
    hipLaunchKernelGGL(block_codebooks_kernel, dim3((int)grid), dim3(64), 0, stream, w, total,
                       num_blocks, block_size, n_entries, qf, cb);
    return check_launch("nb_block_codebooks");
}

int launch_dequant(const uint8_t* packed, const float* codebook, void* w,
                   int w_dtype, int64_t total, int64_t num_blocks, int bits,
                   int n_entries, int block_size, hipStream_t stream) {
    if (total == 0) return NB_OK;
    (void)num_blocks;  // validated by the caller: num_blocks * block_size >= total
    // Fields of indices < total lie inside the first packed_nbytes(total)
    // bytes, so that is all the kernels may touch.
    const int64_t nbytes = packed_nbytes(total, bits);
    const bool bf16 = w_dtype == NB_BF16;
    int64_t first = 0;
    if (block_size % 32 == 0 && is_aligned(packed, 4) && is_aligned(w, 16)) {
        const int64_t chunks = total / 32;
        if (chunks > 0) {
            with_bits(bits, [&](auto B) {
                constexpr int kB = decltype(B)::value;
                auto kernel = bf16 ? dequant_chunks_kernel<kB, true> : dequant_chunks_kernel<kB, false>;
                hipLaunchKernelGGL(kernel, dim3(grid_for(chunks)), dim3(kThreads), 0, stream,
                                   reinterpret_cast<const uint32_t*>(packed), codebook, w, chunks,
                                   n_entries, block_size);
            });
            first = chunks * 32;
        }
    }
    if (first < total) {
        auto kernel = bf16 ? dequant_kernel<true> : dequant_kernel<false>;
        hipLaunchKernelGGL(kernel, dim3(grid_for(total - first)), dim3(kThreads), 0, stream,
                           packed, nbytes, codebook, w, first, total, bits, n_entries,
                           block_size);
    }
    return check_launch("nb_dequant");
}

}  // namespace nb
