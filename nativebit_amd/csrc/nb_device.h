// Device helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nb {

typedef uint16_t bf16_bits;

// float -> bfloat16 bits, round to nearest even; NaN stays a quiet NaN.
// Same result as torch's float->bfloat16 cast.
__device__ __forceinline__ bf16_bits f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) {
        return (bf16_bits)((u | 0x00400000u) >> 16);
    }
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (bf16_bits)(u >> 16);
}

__device__ __forceinline__ float bf16_to_f32(bf16_bits h) {
    return __uint_as_float((uint32_t)h << 16);
}

// Loads of the packed weight stream and codebooks.  Marking them
// non-temporal (NB_STREAM_NT=1) measured slower on MI355X than plain loads.
#ifndef NB_STREAM_NT
#define NB_STREAM_NT 0
#endif
// Pointers into device memory seen as global-address-space pointers, so the
// loads are global_load_* (counted on vmcnt only).  A generic pointer -- one
// read from a table, say -- would become flat_load_*, which also counts on
// lgkmcnt: every LDS or scalar wait would then drain the weight prefetch.
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* as_global(const T* p) {
    return (const __attribute__((address_space(1))) T*)p;
}
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T* as_global_mut(T* p) {
    return (__attribute__((address_space(1))) T*)p;
}

template <typename T>
__device__ __forceinline__ T stream_load(const T* p) {
#if NB_STREAM_NT
    return __builtin_nontemporal_load(as_global(p));
#else
    return *as_global(p);
#endif
}

// f rounded to the nearest bfloat16 (ties to even), kept as a float.
__device__ __forceinline__ float round_bf16(float f) {
    return bf16_to_f32(f32_to_bf16_rne(f));
}

// Index i of an LSB-first stream of `bits`-bit fields (bits <= 8).  The
// second byte is read only when it lies inside the stream.
__device__ __forceinline__ uint32_t read_field(const uint8_t* __restrict__ p,
                                               int64_t nbytes, int64_t i,
                                               int bits) {
    const int64_t bit = i * bits;
    const int64_t byte = bit >> 3;
    uint32_t v = p[byte];
    if (byte + 1 < nbytes) v |= (uint32_t)p[byte + 1] << 8;
    return (v >> (bit & 7)) & ((1u << bits) - 1u);
}

}  // namespace nb
