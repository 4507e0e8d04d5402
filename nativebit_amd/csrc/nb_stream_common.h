// Device building blocks of the streaming 3-bit GEMV shared by the batched
// GEMV kernel (nb_gemv_stream.hip) and the persistent decode kernel
// (nb_decode_persistent.hip).
//
// Layout a wave computes on.  A block is 128 weights: 48 bytes of 3-bit
// indices and 8 fp32 codebook entries (32 bytes).  Lane l of a wave takes one
// block.  Its 48 index bytes are four 12-byte units of 32 indices.  Index j
// of a unit starts at bit 3j, so bytes 0,3,6,9 of a unit hold indices
// starting at bit offsets 0 and 3 of the byte (and the low bits of one
// more), bytes 1,4,7,10 at offsets 1 and 4, bytes 2,5,8,11 at 2 and 5.
// v_perm_b32 gathers each class into one dword, and a shift and a mask then
// yield four indices, one per byte: the selector bytes of a v_perm_b32
// lookup into the block's codebook, kept as byte planes of its bf16-rounded
// entries (low bytes of entries 0-7, high bytes of entries 0-7).  Eight
// selectors per unit (25 VALU ops for 32 indices), four v_perm_b32 per
// selector (two lookups, two interleaves), give 4 bf16 weights -- indices
// o, o+8, o+16, o+24 of the unit -- for one v_mfma_f32_4x4x4_16b_bf16.  The
// activations are staged in LDS in the same order (16-byte unit j = 4u + m
// of a column block holds the activations of selectors 2m and 2m+1 of unit
// u).  In that instruction lane 4b+i supplies row i of block b's A and
// column i of its B, and the diagonal D[b][i][i] -- lane 4b+i, accumulator
// i -- is the lane's own 4-term dot product: every lane accumulates a
// private dot product, so a lane can hold any block of any row.
//
// Weights are rounded to bf16 (RNE) as in the reference's bf16 path
// (inference/eval_ppl.py:149-174); accumulation is fp32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nb {
namespace stream {

typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;

// LDS bytes of one column block's staged activations: 16 units of 16 bytes,
// padded by one unit so that 16 consecutive blocks start in 16 different
// bank groups (272 bytes = 68 banks apart)
#ifndef NB_XCOL_UNITS
#define NB_XCOL_UNITS 17
#endif
constexpr int kXColBytes = NB_XCOL_UNITS * 16;

// Index offset o of selector s inside a 32-index unit: selector s yields
// indices o, o+8, o+16, o+24.
__host__ __device__ constexpr int sel_offset(int s) {
    return s == 0 ? 0 : s == 1 ? 1 : s == 2 ? 3 : s == 3 ? 4 : s == 4 ? 6 : s == 5 ? 7 : s == 6 ? 2 : 5;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
    bf16x2_t v;
    v.x = (__bf16)lo;
    v.y = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
}

// The eight selectors of one 12-byte unit (d0, d1, d2): selector s holds
// indices sel_offset(s) + 8k (k = 0..3), one per byte.
__device__ __forceinline__ void unit_selectors(uint32_t d0, uint32_t d1, uint32_t d2,
                                               uint32_t (&sel)[8]) {
    const uint32_t M = 0x07070707u;
    // T = bytes 0,3,6,9; U = bytes 1,4,7,10; E = bytes 2,5,8,11
    const uint32_t t = __builtin_amdgcn_perm(d2, __builtin_amdgcn_perm(d1, d0, 0x00060300u),
                                             0x05020100u);
    const uint32_t u = __builtin_amdgcn_perm(d2, __builtin_amdgcn_perm(d1, d0, 0x00070401u),
                                             0x06020100u);
    const uint32_t e = __builtin_amdgcn_perm(d2, __builtin_amdgcn_perm(d1, d0, 0x00000502u),
                                             0x07040100u);
    sel[0] = t & M;                 // bit offset 0 of T bytes
    sel[1] = (t >> 3) & M;          // offset 3
    sel[2] = (u >> 1) & M;          // offset 1 of U bytes
    sel[3] = (u >> 4) & M;          // offset 4
    sel[4] = (e >> 2) & M;          // offset 2 of E bytes
    sel[5] = (e >> 5) & M;          // offset 5
    // bits 6-7 of a T byte + bit 0 of the next (U) byte
    sel[6] = ((t >> 6) & 0x03030303u) | ((u << 2) & 0x04040404u);
    // bit 7 of a U byte + bits 0-1 of the next (E) byte
    sel[7] = ((u >> 7) & 0x01010101u) | ((e << 1) & 0x06060606u);
}

// The selector-ordered unit (nb_stream_layout, made once at load): the same
// 32 indices and 96 bits, placed so that selector s holds the same four
// indices as above.  Byte k of dword 0 holds index o(0)+8k in bits 0-2,
// o(1)+8k in bits 3-5 and the low two bits of o(6)+8k in bits 6-7; dword 1
// likewise o(2)+8k, o(3)+8k and the low bits of o(7)+8k; dword 2 o(4)+8k,
// o(5)+8k and the high bits of o(6)+8k (bit 6) and o(7)+8k (bit 7).  Six
// selectors are then one shift and one mask each, the last two two
// shifts, two masks and an or: 17 VALU ops for 32 indices.
__device__ __forceinline__ void unit_selectors_sel(uint32_t d0, uint32_t d1, uint32_t d2,
                                                   uint32_t (&sel)[8]) {
    const uint32_t M = 0x07070707u;
    sel[0] = d0 & M;
    sel[1] = (d0 >> 3) & M;
    sel[2] = d1 & M;
    sel[3] = (d1 >> 3) & M;
    sel[4] = d2 & M;
    sel[5] = (d2 >> 3) & M;
    sel[6] = ((d0 >> 6) & 0x03030303u) | ((d2 >> 4) & 0x04040404u);
    sel[7] = ((d1 >> 6) & 0x03030303u) | ((d2 >> 5) & 0x04040404u);
}

// The selector-ordered unit of the eight selectors of a unit (the inverse of
// unit_selectors_sel for selectors whose bytes are 0..7).
__host__ __device__ __forceinline__ void sel_unit_pack(const uint32_t (&sel)[8], uint32_t& d0,
                                                      uint32_t& d1, uint32_t& d2) {
    d0 = sel[0] | (sel[1] << 3) | ((sel[6] & 0x03030303u) << 6);
    d1 = sel[2] | (sel[3] << 3) | ((sel[7] & 0x03030303u) << 6);
    d2 = sel[4] | (sel[5] << 3) | (((sel[6] >> 2) & 0x01010101u) << 6) |
         (((sel[7] >> 2) & 0x01010101u) << 7);
}

__device__ __forceinline__ f32x4_t mfma44(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1,
                                          f32x4_t c) {
    u32x2_t a = {a0, a1}, b = {b0, b1};
    return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(bf16x4_t, a),
                                                 __builtin_bit_cast(bf16x4_t, b), c, 0, 0, 0);
}

template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

// One direct-to-LDS load: every lane reads 16 bytes at src + OFF, and lane
// i's bytes land at LDS byte address lds + OFF + 16 i (the instruction
// offset applies to both addresses).  Issued as inline asm so the compiler
// does not track it: it would otherwise make every later LDS access wait
// for all ring loads, draining the prefetch at each chunk.  Reads of the
// destination are ordered after the load by wait_vm.
template <int OFF>
__device__ __forceinline__ void dma16(uint32_t lds, const void* src) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off offset:%2 nt"
                 :
                 : "s"(lds), "v"(src), "n"(OFF)
                 : "memory", "m0");
}

// Waits until at most N vector-memory operations of this wave are
// outstanding.
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// Waits for every LDS operation of this wave (a slot's reads must be done
// before the slot is refilled).
__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory"); }

template <typename T>
__device__ __forceinline__ uint32_t lds_addr(T* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) T*)p;
}

// float DPP move within a quad (quad_perm control)
template <int CTRL>
__device__ __forceinline__ float quad_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ int quad_mov_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, false);
}
constexpr int quad_perm(int a, int b, int c, int d) { return a | (b << 2) | (c << 4) | (d << 6); }

// One lane's bytes of one block: 48 index bytes and 8 fp32 codebook entries.
struct SlotRegs {
    u32x4_t d0, d1, d2, c0, c1;
};

// The 32 bf16 activations w[0..15] (natural order, two per dword) of unit u
// of a column block, written to the staged layout at `col` (the column
// block's kXColBytes bytes).
__device__ __forceinline__ void stage_unit(unsigned char* col, int u, const uint32_t (&w)[16]) {
    auto xs = [&](int k) -> uint32_t { return (w[k >> 1] >> (16 * (k & 1))) & 0xffffu; };
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int oa = sel_offset(2 * m), ob = sel_offset(2 * m + 1);
        u32x4_t o;
        o.x = xs(oa) | (xs(oa + 8) << 16);
        o.y = xs(oa + 16) | (xs(oa + 24) << 16);
        o.z = xs(ob) | (xs(ob + 8) << 16);
        o.w = xs(ob + 16) | (xs(ob + 24) << 16);
        *reinterpret_cast<u32x4_t*>(col + (4 * u + m) * 16) = o;
    }
}

// The lane's dot product of its block (index dwords rd0..rd2, codebook
// rc0..rc1) with the staged activations of its column (xv = the column
// block's 16 units), as the four accumulators whose element (lane & 3)
// holds it (see diag_of).  kSel: the index bytes are in the
// selector-ordered unit layout (same selectors, same products).  The
// block's registers are taken by value: a reference to a caller's struct
// made the register allocator spill them.
template <bool kSel = false>
__device__ __forceinline__ f32x4_t block_dot(u32x4_t rd0, u32x4_t rd1, u32x4_t rd2, u32x4_t rc0,
                                             u32x4_t rc1, const u32x4_t (&xv)[16]) {
    const SlotRegs r = {rd0, rd1, rd2, rc0, rc1};
    // codebook byte planes (bf16-rounded entries)
    const uint32_t q0 = pack_bf16x2(__uint_as_float(r.c0.x), __uint_as_float(r.c0.y));
    const uint32_t q1 = pack_bf16x2(__uint_as_float(r.c0.z), __uint_as_float(r.c0.w));
    const uint32_t q2 = pack_bf16x2(__uint_as_float(r.c1.x), __uint_as_float(r.c1.y));
    const uint32_t q3 = pack_bf16x2(__uint_as_float(r.c1.z), __uint_as_float(r.c1.w));
    const uint32_t lo0 = __builtin_amdgcn_perm(q1, q0, 0x06040200u);
    const uint32_t hi0 = __builtin_amdgcn_perm(q1, q0, 0x07050301u);
    const uint32_t lo1 = __builtin_amdgcn_perm(q3, q2, 0x06040200u);
    const uint32_t hi1 = __builtin_amdgcn_perm(q3, q2, 0x07050301u);
    const uint32_t d[12] = {r.d0.x, r.d0.y, r.d0.z, r.d0.w, r.d1.x, r.d1.y,
                            r.d1.z, r.d1.w, r.d2.x, r.d2.y, r.d2.z, r.d2.w};
    f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        uint32_t sel[8];
        if constexpr (kSel) {
            unit_selectors_sel(d[3 * u], d[3 * u + 1], d[3 * u + 2], sel);
        } else {
            unit_selectors(d[3 * u], d[3 * u + 1], d[3 * u + 2], sel);
        }
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const uint32_t la = __builtin_amdgcn_perm(lo1, lo0, sel[s]);
            const uint32_t ha = __builtin_amdgcn_perm(hi1, hi0, sel[s]);
            const uint32_t w0 = __builtin_amdgcn_perm(ha, la, 0x05010400u);
            const uint32_t w1 = __builtin_amdgcn_perm(ha, la, 0x07030602u);
            const u32x4_t& x = xv[4 * u + (s >> 1)];
            // two accumulators halve the dependent-MFMA chain
            if (s & 1) {
                acc1 = mfma44(w0, w1, x.z, x.w, acc1);
            } else {
                acc0 = mfma44(w0, w1, x.x, x.y, acc0);
            }
        }
    }
    return acc0 + acc1;
}

// The lane's own dot product: diagonal element (lane & 3) of block_dot.
__device__ __forceinline__ float diag_of(const f32x4_t& a, int lane) {
    const int l3 = lane & 3;
    return l3 == 0 ? a.x : l3 == 1 ? a.y : l3 == 2 ? a.z : a.w;
}

}  // namespace stream
}  // namespace nb
