// Bit-exact format kernels: unpack, pack and dequantize NativeBit index
// streams on gfx950.  These are the parity kernels of the path (their
// outputs must equal the reference's byte for byte), not the hot loop, so
// they favour simple, obviously-correct indexing over peak bandwidth; all of
// them are coalesced grid-stride loops.
//
// Reference semantics: nativebit/pack.py:21-169 (pack_3bit, unpack_3bit,
// pack_4bit, unpack_4bit, pack_nbits, unpack_nbits, reconstruct_weight),
// inference/triton_kernel.py:199-220 (pack_indices_to_3bit).
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
