// Bit-exact format kernels: unpack, pack and dequantize NativeBit index
// streams on gfx950.  These are the parity kernels of the path (their
// outputs must equal the reference's byte for byte), not the hot loop, so
// they favour simple, obviously-correct indexing over peak bandwidth; all of
// them are coalesced grid-stride loops.
//
// Reference semantics: nativebit/pack.py:21-169 (pack_3bit, unpack_3bit,
// pack_4bit, unpack_4bit, pack_nbits, unpack_nbits, reconstruct_weight),
// inference/triton_kernel.py:199-220 (pack_indices_to_3bit),
// inference/pack.py:21-35 (quantize_weight, fused here with the pack).
#include <math.h>

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
    uint8_t* __restrict__ out, int64_t count, int bits) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < count;
         i += stride) {
        out[i] = (uint8_t)read_field(packed, nbytes, i, bits);
    }
}

// One output byte per iteration: byte b holds stream bits [8b, 8b+8), i.e.
// the fields of indices floor(8b/bits) .. floor((8b+7)/bits).
__global__ __launch_bounds__(kThreads) void pack_kernel(
    const uint8_t* __restrict__ idx, int64_t count, int bits,
    uint8_t* __restrict__ out, int64_t nbytes) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    const uint32_t mask = (1u << bits) - 1u;
    for (int64_t b = (int64_t)blockIdx.x * kThreads + threadIdx.x; b < nbytes;
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
                                                  int block_size, int64_t i) {
    const float v = i < total ? w[i] : 0.f;
    const float* c = cb + (i / block_size) * n_entries;
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
    int block_size, int64_t count, int bits, uint8_t* __restrict__ out, int64_t nbytes) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    const int64_t groups = (count + 7) / 8;
    for (int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x; t < groups; t += stride) {
        float c[16];
        int64_t cur_block = -1;
        uint64_t acc = 0;  // 8 fields, LSB first (8 * bits <= 64)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int64_t i = 8 * t + j;
            uint32_t f = 0;
            if (i < count) {
                if (kSmallNE) {
                    const float v = i < total ? w[i] : 0.f;
                    const int64_t blk = i / block_size;
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
                    f = nearest_entry(w, total, cb, n_entries, block_size, i);
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

template <bool kBF16>
__global__ __launch_bounds__(kThreads) void dequant_kernel(
    const uint8_t* __restrict__ packed, int64_t nbytes,
    const float* __restrict__ cb, void* __restrict__ w, int64_t total,
    int bits, int n_entries, int block_size) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    const uint32_t last = (uint32_t)(n_entries - 1);
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
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

}  // namespace

int launch_unpack(const uint8_t* packed, uint8_t* out, int64_t count, int bits,
                  hipStream_t stream) {
    if (count == 0) return NB_OK;
    hipLaunchKernelGGL(unpack_kernel, dim3(grid_for(count)), dim3(kThreads), 0,
                       stream, packed, packed_nbytes(count, bits), out, count,
                       bits);
    return check_launch("nb_unpack");
}

int launch_pack(const uint8_t* idx, uint8_t* out, int64_t count, int bits,
                hipStream_t stream) {
    const int64_t nbytes = packed_nbytes(count, bits);
    if (nbytes == 0) return NB_OK;
    hipLaunchKernelGGL(pack_kernel, dim3(grid_for(nbytes)), dim3(kThreads), 0,
                       stream, idx, count, bits, out, nbytes);
    return check_launch("nb_pack");
}

int launch_quantize_pack(const float* w, int64_t total, const float* codebook,
                         int64_t num_blocks, int n_entries, int block_size, int bits,
                         uint8_t* out, hipStream_t stream) {
    const int64_t count = num_blocks * block_size;
    const int64_t nbytes = packed_nbytes(count, bits);
    if (nbytes == 0) return NB_OK;
    const int grid = grid_for((count + 7) / 8);
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), 0, stream, w, total, codebook,
                           n_entries, block_size, count, bits, out, nbytes);
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
    // bytes, so that is all the kernel may touch.
    const int64_t nbytes = packed_nbytes(total, bits);
    if (w_dtype == NB_BF16) {
        hipLaunchKernelGGL(dequant_kernel<true>, dim3(grid_for(total)),
                           dim3(kThreads), 0, stream, packed, nbytes, codebook,
                           w, total, bits, n_entries, block_size);
    } else {
        hipLaunchKernelGGL(dequant_kernel<false>, dim3(grid_for(total)),
                           dim3(kThreads), 0, stream, packed, nbytes, codebook,
                           w, total, bits, n_entries, block_size);
    }
    return check_launch("nb_dequant");
}

}  // namespace nb
