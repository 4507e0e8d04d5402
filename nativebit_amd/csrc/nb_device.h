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

// Cross-lane reductions by DPP.  A ds_bpermute-based butterfly (what
// __shfl_xor compiles to) is six dependent LDS round trips per reduction;
// these are register moves within each row of 16 lanes plus four lane
// reads.  Every lane gets the same value; all lanes taking part must be
// active.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float lane_value(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
// Sum / max over each row of 16 lanes (pairs, quads, half-rows, rows).
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_mov<0xB1>(v);   // quad_perm(1, 0, 3, 2)
    v += dpp_mov<0x4E>(v);   // quad_perm(2, 3, 0, 1)
    v += dpp_mov<0x141>(v);  // row_half_mirror
    v += dpp_mov<0x140>(v);  // row_mirror
    return v;
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_mov<0xB1>(v));
    v = fmaxf(v, dpp_mov<0x4E>(v));
    v = fmaxf(v, dpp_mov<0x141>(v));
    v = fmaxf(v, dpp_mov<0x140>(v));
    return v;
}
// Sum / max over the 64 lanes of a wave (row totals added in row order).
__device__ __forceinline__ float wave64_sum(float v) {
    v = row16_sum(v);
    return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}
__device__ __forceinline__ float wave64_max(float v) {
    v = row16_max(v);
    return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)),
                 fmaxf(lane_value(v, 32), lane_value(v, 48)));
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
