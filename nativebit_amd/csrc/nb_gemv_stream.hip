// Persistent streaming GEMV over a batch of packed 3-bit layers (gfx950).
//
//   for every problem p:  y_p[n] = sum_k x_p[k] * bf16(W_p[n][k])   (M = 1)
//
// One launch streams the packed weights of all problems.  Each problem's
// blocks (128 weights: 48 bytes of 3-bit indices, 32 bytes of fp32
// codebook) are cut into chunks of 64 consecutive blocks -- 3 KiB of index
// stream and 2 KiB of codebook, both contiguous in HBM -- numbered
// consecutively across problems.
//
// Memory side.  A wave loads a chunk with five global_load_lds_dwordx4
// (direct-to-LDS) instructions, each covering one contiguous KiB, marked
// non-temporal: the access shape under which MI355X streams at about
// 7 TB/s (a 16-rows x 4-blocks tile pattern read into registers stays near
// 5.7 TB/s even with all arithmetic removed).  Each wave owns a ring of
// NB_STREAM_DEPTH chunk slots in LDS; a slot is refilled as soon as its
// bytes are in registers, so NB_STREAM_DEPTH chunks per wave are in flight
// while one is computed.
//
// Compute side.  Lane l takes block l of the chunk.  Its 48 index bytes are
// four 12-byte units of 32 indices.  Index j of a unit starts at bit 3j, so
// bytes 0,3,6,9 of a unit hold indices starting at bit offsets 0 and 3 of
// the byte (and the low bits of one more), bytes 1,4,7,10 at offsets 1 and
// 4, bytes 2,5,8,11 at 2 and 5.  v_perm_b32 gathers each class into one
// dword, and a shift and a mask then yield four indices, one per byte: the
// selector bytes of a v_perm_b32 lookup into the block's codebook, kept as
// byte planes of its bf16-rounded entries (low bytes of entries 0-7, high
// bytes of entries 0-7).  Eight selectors per unit (25 VALU ops for 32
// indices), four v_perm_b32 per selector (two lookups, two interleaves),
// give 4 bf16 weights -- indices o, o+8, o+16, o+24 of the unit -- for one
// v_mfma_f32_4x4x4_16b_bf16.  The activations are staged in LDS in the same
// order.  In that instruction lane 4b+i supplies row i of block b's A and
// column i of its B, and the diagonal D[b][i][i] -- lane 4b+i, accumulator
// i -- is the lane's own 4-term dot product: every lane accumulates a
// private dot product, so a lane can hold any block of any row.
//
// Row sums.  A row of bpr <= 64 blocks lies in at most two consecutive
// chunks.  Lanes of a quad that share a row add their dot products in a
// fixed order (DPP); the quad's sum, or each lane's own value where the
// quad spans a row boundary, goes by LDS atomic to sum[row] in the chunk
// where the row starts, or to carry[chunk] for the blocks of a row that
// began in the previous chunk.  Each slot receives the lanes of one
// instruction of one wave, and y[row] = sum[row] + carry[the row's last
// chunk] (when it differs from its first), so results do not depend on
// which wave took which chunk.
// Workgroup ranges start and end on row boundaries, so no row is shared
// between workgroups; inside a workgroup waves take chunks one at a time
// from a counter in LDS.
//
// Weights are rounded to bf16 (RNE) as in the reference's bf16 path
// (inference/eval_ppl.py:149-174); accumulation is fp32.
#include <algorithm>
#include <numeric>
#include <utility>
#include <vector>

#include "nb_device.h"
#include "nb_internal.h"

namespace nb {
namespace {

typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;

// waves per workgroup (three per SIMD: more waves hide the LDS and
// memory waits of each other better than a deeper ring) and chunks in
// flight per wave
#ifndef NB_STREAM_WAVES
#define NB_STREAM_WAVES 12
#endif
#ifndef NB_STREAM_DEPTH
#define NB_STREAM_DEPTH 2
#endif
#ifndef NB_STREAM_WG_PER_CU
#define NB_STREAM_WG_PER_CU 1
#endif
constexpr int kWaves = NB_STREAM_WAVES;
constexpr int kDepth = NB_STREAM_DEPTH;
static_assert(kDepth == 2 || kDepth == 3, "ring depth 2 or 3");

constexpr int kChunkBlocks = 64;
constexpr int kChunkIdxBytes = kChunkBlocks * 48;  // 3 KiB
constexpr int kChunkCbBytes = kChunkBlocks * 32;   // 2 KiB
constexpr int kSlotBytes = kChunkIdxBytes + kChunkCbBytes;
constexpr int kLoadsPerChunk = 5;
// LDS bytes of one column block's activations: 16 units of 16 bytes, padded
// by one unit so that 16 consecutive blocks start in 16 different bank
// groups (272 bytes = 68 banks apart)
#ifndef NB_XCOL_UNITS
#define NB_XCOL_UNITS 17
#endif
constexpr int kXColBytes = NB_XCOL_UNITS * 16;

// Index offset o of selector s inside a 32-index unit: selector s yields
// indices o, o+8, o+16, o+24 (see the file comment).
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

__device__ __forceinline__ f32x4_t mfma44(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1,
                                          f32x4_t c) {
    u32x2_t a = {a0, a1}, b = {b0, b1};
    return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(bf16x4_t, a),
                                                 __builtin_bit_cast(bf16x4_t, b), c, 0, 0, 0);
}

// One problem of the workgroup's range as the chunk loop reads it, copied
// into LDS at set-up (64 bytes).
struct ProbL {
    const uint8_t* packed;
    const float* codebook;
    void* y;
    int32_t nblocks, bpr, nchunks, chunk_begin;
    int32_t x_off;      // byte offset of this problem's x (permuted) in LDS
    int32_t y_off;      // float offset of its row sums (rows row_a..row_b-1)
    int32_t row_a;      // first row of this problem in the range
    int32_t row_b;      // one past the last row
    int32_t carry_off;  // float offset of its carries (chunks ca..)
    int32_t ca;         // first chunk of this problem in the range
};
static_assert(sizeof(ProbL) == 64, "ProbL is 64 bytes");

// The fields the loop needs, in scalar registers.
struct Prob {
    const uint8_t* packed;
    const float* codebook;
    int nblocks, bpr, chunk_begin, chunk_end, x_off, y_off, row_a, carry_off, ca;
    float inv_bpr;
};

template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ void read_prob(const ProbL* pl, int li, Prob& P) {
    const ProbL& s = pl[li];
    P.packed = uniform_ptr(s.packed);
    P.codebook = uniform_ptr(s.codebook);
    P.nblocks = __builtin_amdgcn_readfirstlane(s.nblocks);
    P.bpr = __builtin_amdgcn_readfirstlane(s.bpr);
    P.chunk_begin = __builtin_amdgcn_readfirstlane(s.chunk_begin);
    P.chunk_end = P.chunk_begin + __builtin_amdgcn_readfirstlane(s.nchunks);
    P.x_off = __builtin_amdgcn_readfirstlane(s.x_off);
    P.y_off = __builtin_amdgcn_readfirstlane(s.y_off);
    P.row_a = __builtin_amdgcn_readfirstlane(s.row_a);
    P.carry_off = __builtin_amdgcn_readfirstlane(s.carry_off);
    P.ca = __builtin_amdgcn_readfirstlane(s.ca);
    P.inv_bpr = 1.0f / (float)P.bpr;
}

// Where one ring slot's chunk belongs.  `valid` is false for loads issued
// after the wave ran out of chunks (they repeat the last address and are
// never consumed).
struct Meta {
    int li, lc;
    bool valid;
};

// One direct-to-LDS load: every lane reads 16 bytes at src + OFF, and lane
// i's bytes land at LDS byte address lds + OFF + 16 i (the instruction
// offset applies to both addresses).  Issued as inline asm so the compiler
// does not track it: it would otherwise make every later LDS atomic wait
// for all ring loads (the ring and the counters share one LDS array),
// draining the prefetch at each chunk.  Reads of a slot are ordered after
// its loads by wait_vm.
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

// One lane's bytes of one chunk.
struct SlotRegs {
    u32x4_t d0, d1, d2, c0, c1;
};

__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(kWaves / 4, kWaves / 4)))
void gemv_stream_kernel(
    const StreamProblem* __restrict__ probs, StreamRanges ranges, int y_dtype) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    // ---- set-up: the workgroup's chunks, problems, x vectors and counter --
    const int g = blockIdx.x;
    const int C0 = ranges.chunk0[g];
    const int C1 = ranges.chunk0[g + 1];
    const int p0 = ranges.prob0[g];
    const int np = ranges.prob1[g] - p0 + 1;
    ProbL* pl = reinterpret_cast<ProbL*>(smem);
    unsigned char* ring = smem + np * (int)sizeof(ProbL);
    unsigned char* xregion = ring + kWaves * kDepth * kSlotBytes;
    // every thread walks the range's problems (few) to lay out LDS
    int x_bytes = 0, y_floats = 0;
    for (int i = 0; i < np; ++i) {
        const StreamProblem& s = probs[p0 + i];
        const int ca = max(C0, s.chunk_begin) - s.chunk_begin;
        const int cb = min(C1, s.chunk_begin + s.nchunks) - s.chunk_begin;
        const int ra = (int)(((int64_t)ca * kChunkBlocks) / s.bpr);
        const int rb = min(s.N, (int)(((int64_t)cb * kChunkBlocks + s.bpr - 1) / s.bpr));
        if (tid == i) {
            ProbL d;
            d.packed = s.packed;
            d.codebook = s.codebook;
            d.y = s.y;
            d.nblocks = s.N * s.bpr;
            d.bpr = s.bpr;
            d.nchunks = s.nchunks;
            d.chunk_begin = s.chunk_begin;
            d.x_off = x_bytes;
            d.y_off = y_floats;
            d.row_a = ra;
            d.row_b = rb;
            d.carry_off = y_floats + (rb - ra);
            d.ca = ca;
            pl[i] = d;
        }
        x_bytes += s.bpr * kXColBytes;
        y_floats += (rb - ra) + (cb - ca);
    }
    float* ybuf = reinterpret_cast<float*>(xregion + x_bytes);
    int* next_chunk = reinterpret_cast<int*>(ybuf + y_floats);
    {
        // x of each problem in selector order: 16-byte unit j = 4u + m of
        // column block c, at c * kXColBytes + j * 16, holds the activations
        // of selectors 2m and 2m+1 of unit u (4 bf16 each, in lookup order).
        int off = 0;
        for (int i = 0; i < np; ++i) {
            const StreamProblem& s = probs[p0 + i];
            for (int q = tid; q < s.bpr * 4; q += 64 * kWaves) {
                const int c = q >> 2, u = q & 3;
                const u32x4_t* src = reinterpret_cast<const u32x4_t*>(s.x + c * 128 + u * 32);
                uint32_t w[16];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const u32x4_t t = *as_global(src + v);
                    w[4 * v] = t.x;
                    w[4 * v + 1] = t.y;
                    w[4 * v + 2] = t.z;
                    w[4 * v + 3] = t.w;
                }
                auto xs = [&](int k) -> uint32_t { return (w[k >> 1] >> (16 * (k & 1))) & 0xffffu; };
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const int oa = sel_offset(2 * m), ob = sel_offset(2 * m + 1);
                    u32x4_t o;
                    o.x = xs(oa) | (xs(oa + 8) << 16);
                    o.y = xs(oa + 16) | (xs(oa + 24) << 16);
                    o.z = xs(ob) | (xs(ob + 8) << 16);
                    o.w = xs(ob + 16) | (xs(ob + 24) << 16);
                    *reinterpret_cast<u32x4_t*>(xregion + off + c * kXColBytes + (4 * u + m) * 16) = o;
                }
            }
            off += s.bpr * kXColBytes;
        }
    }
    for (int e = tid; e < y_floats; e += 64 * kWaves) ybuf[e] = 0.f;
    if (tid == 0) *next_chunk = C0;
    __syncthreads();

    // ---- steady state: waves take chunks from the counter until none is left
    auto grab = [&]() -> int {
        int t = 0;
        if (lane == 0) t = atomicAdd(next_chunk, 1);
        return __builtin_amdgcn_readfirstlane(t);
    };
    unsigned char* my_ring = ring + wave * kDepth * kSlotBytes;
    const uint32_t my_ring_lds = lds_addr(my_ring);

    const int c_first = grab();
    if (c_first < C1) {
        // load cursor (runs kDepth chunks ahead of computation)
        int li = 0;
        Prob LP;
        read_prob(pl, 0, LP);
        while (c_first >= LP.chunk_end) read_prob(pl, ++li, LP);
        int lchunk = c_first;
        bool lvalid = true;

        // Loads the chunk at the load cursor into ring slot `slot`, records
        // where it belongs and moves the cursor to chunk `next` (taken from
        // the counter beforehand); past the wave's last chunk it marks the
        // slot invalid and loads nothing.  In a problem's partial last
        // chunk, lanes past the end of the stream re-read its last 16 bytes
        // (their blocks are not live).
        auto issue = [&](int slot, Meta& m, int next) {
            m.valid = lvalid;
            if (!lvalid) return;  // past the wave's last chunk: no load
            const int lc = lchunk - LP.chunk_begin;
            const uint32_t dst = __builtin_amdgcn_readfirstlane(my_ring_lds + slot * kSlotBytes);
            const uint8_t* ip = LP.packed + (int64_t)lc * kChunkIdxBytes + 16 * lane;
            const uint8_t* cp = reinterpret_cast<const uint8_t*>(LP.codebook) +
                                (int64_t)lc * kChunkCbBytes + 16 * lane;
            if ((lc + 1) * kChunkBlocks <= LP.nblocks) {
                dma16<0>(dst, ip);
                dma16<1024>(dst, ip);
                dma16<2048>(dst, ip);
                dma16<0>(dst + kChunkIdxBytes, cp);
                dma16<1024>(dst + kChunkIdxBytes, cp);
            } else {
                const uint8_t* ilast = LP.packed + (int64_t)LP.nblocks * 48 - 16;
                const uint8_t* clast =
                    reinterpret_cast<const uint8_t*>(LP.codebook) + (int64_t)LP.nblocks * 32 - 16;
                dma16<0>(dst, min(ip, ilast));
                dma16<0>(dst + 1024, min(ip + 1024, ilast));
                dma16<0>(dst + 2048, min(ip + 2048, ilast));
                dma16<0>(dst + kChunkIdxBytes, min(cp, clast));
                dma16<0>(dst + kChunkIdxBytes + 1024, min(cp + 1024, clast));
            }
            m.li = li;
            m.lc = lc;
            if (next >= C1) {
                lvalid = false;  // the wave's last chunk
            } else {
                lchunk = next;
                while (lchunk >= LP.chunk_end) read_prob(pl, ++li, LP);
            }
        };

        int ci = -1;  // problem whose fields are in CP
        Prob CP = {};

        // Per-chunk lane state computed before the chunk's bytes arrive.
        struct Lane {
            int row;
            bool live;
        };
        // The lane's block, row and column; requests its 16 activation
        // units from LDS.
        auto prepare = [&](const Meta& m, u32x4_t (&xv)[16]) -> Lane {
            if (m.li != ci) {
                read_prob(pl, m.li, CP);
                ci = m.li;
            }
            const int beta = m.lc * kChunkBlocks + lane;  // block of this lane
            Lane L;
            L.live = beta < CP.nblocks;
            // row = beta / bpr (beta < 2^24): float estimate, off by at most
            // one, then corrected
            int row = (int)__builtin_fmaf((float)beta, CP.inv_bpr, 0.5f * CP.inv_bpr);
            int rem = beta - (int)__umul24((unsigned)row, (unsigned)CP.bpr);
            row += rem >= CP.bpr ? 1 : (rem < 0 ? -1 : 0);
            rem = beta - (int)__umul24((unsigned)row, (unsigned)CP.bpr);
            L.row = row;
            const int col = L.live ? rem : 0;
            const unsigned char* xb = xregion + CP.x_off + col * kXColBytes;
#pragma unroll
            for (int j = 0; j < 16; ++j) xv[j] = *reinterpret_cast<const u32x4_t*>(xb + 16 * j);
            return L;
        };

        // This lane's 48 index bytes and 32 codebook bytes of a slot, in
        // registers once wait_lds() has returned.
        auto read_slot = [&](int slot) -> SlotRegs {
            const unsigned char* src = my_ring + slot * kSlotBytes;
            const u32x4_t* pi = reinterpret_cast<const u32x4_t*>(src + 48 * lane);
            const u32x4_t* pc = reinterpret_cast<const u32x4_t*>(src + kChunkIdxBytes + 32 * lane);
            SlotRegs r;
            r.d0 = pi[0];
            r.d1 = pi[1];
            r.d2 = pi[2];
            r.c0 = pc[0];
            r.c1 = pc[1];
            return r;
        };

        auto compute = [&](const SlotRegs& r, const Meta& m, const Lane& L,
                           const u32x4_t (&xv)[16]) {
            // codebook byte planes (bf16-rounded entries); a block that is
            // not live computes garbage on its own diagonal only
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
                unit_selectors(d[3 * u], d[3 * u + 1], d[3 * u + 2], sel);
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
            // the lane's own dot product is diagonal element (lane & 3)
            const f32x4_t a = acc0 + acc1;
            const int l3 = lane & 3;
            const float dot = l3 == 0 ? a.x : l3 == 1 ? a.y : l3 == 2 ? a.z : a.w;
            // quad pre-sum where the quad's four blocks share a row
            const int rowx = L.live ? L.row : -1 - lane;
            const bool quad_row = quad_mov_i<quad_perm(0, 0, 0, 0)>(rowx) ==
                                  quad_mov_i<quad_perm(3, 3, 3, 3)>(rowx);
            const float s2 = dot + quad_mov<quad_perm(1, 0, 3, 2)>(dot);
            const float s4 = s2 + quad_mov<quad_perm(2, 3, 0, 1)>(s2);
            if (L.live && (!quad_row || l3 == 0)) {
                // a row that began in the previous chunk goes to this
                // chunk's carry slot
                const bool carry = L.row * CP.bpr < m.lc * kChunkBlocks;
                const int slot = carry ? CP.carry_off + m.lc - CP.ca : CP.y_off + L.row - CP.row_a;
                atomicAdd(ybuf + slot, quad_row ? s4 : dot);
            }
        };

        // Ring of kDepth slots, unrolled so each slot index is a constant.
        // One step: take the next chunk number from the counter and request
        // this chunk's activations (both LDS, in flight while the wave waits
        // for the chunk), read the slot into registers, refill it with the
        // chunk kDepth ahead, and compute -- kDepth chunks are in flight
        // during the arithmetic.  Validity is monotonic: the first invalid
        // slot ends the wave's work.  The loop issues no other vector-memory
        // instruction, so the vmcnt waits count ring loads exactly (each
        // valid slot holds kLoadsPerChunk loads).
        Meta ma = {0, 0, false}, mb = {0, 0, false}, mc = {0, 0, false};
        // `after` = valid slots loaded after this one (their loads may stay
        // in flight).
        auto step = [&](int slot, Meta& m, int after) {
            const int next = lvalid ? grab() : C1;
            u32x4_t xv[16];
            const Lane L = prepare(m, xv);
            if (after == 2) {
                wait_vm<2 * kLoadsPerChunk>();
            } else if (after == 1) {
                wait_vm<kLoadsPerChunk>();
            } else {
                wait_vm<0>();
            }
            const SlotRegs r = read_slot(slot);
            wait_lds();
            const Meta cur = m;
            issue(slot, m, next);
            compute(r, cur, L, xv);
        };
        issue(0, ma, grab());
        if constexpr (kDepth == 2) {
            issue(1, mb, lvalid ? grab() : C1);
            while (true) {
                if (!ma.valid) break;
                step(0, ma, mb.valid ? 1 : 0);
                if (!mb.valid) break;
                step(1, mb, ma.valid ? 1 : 0);
            }
        } else {
            issue(1, mb, lvalid ? grab() : C1);
            issue(2, mc, lvalid ? grab() : C1);
            while (true) {
                if (!ma.valid) break;
                step(0, ma, (int)mb.valid + (int)mc.valid);
                if (!mb.valid) break;
                step(1, mb, (int)mc.valid + (int)ma.valid);
                if (!mc.valid) break;
                step(2, mc, (int)ma.valid + (int)mb.valid);
            }
        }
        wait_vm<0>();  // (nothing is in flight here; kept as a guard)
    }

    // ---- write the range's outputs (coalesced, after every wave is done) --
    __syncthreads();
    for (int i = 0; i < np; ++i) {
        const ProbL& P = pl[i];
        for (int e = tid; e < P.row_b - P.row_a; e += 64 * kWaves) {
            const int row = P.row_a + e;
            float val = ybuf[P.y_off + e];
            // the row's tail, if its last block lies in a later chunk
            const int c_first = (row * P.bpr) / kChunkBlocks;
            const int c_last = (row * P.bpr + P.bpr - 1) / kChunkBlocks;
            if (c_last != c_first) val += ybuf[P.carry_off + c_last - P.ca];
            if (y_dtype == NB_BF16) {
                *as_global_mut(static_cast<bf16_bits*>(P.y) + row) = f32_to_bf16_rne(val);
            } else {
                *as_global_mut(static_cast<float*>(P.y) + row) = val;
            }
        }
    }
}

// Chunks of one row-aligned tile of a problem: the smallest run of chunks
// that starts and ends on row boundaries.
int tile_chunks(int bpr) { return bpr / std::gcd(bpr, kChunkBlocks); }

}  // namespace

// LDS bytes the kernel uses for the chunk range [a, b) over problems
// [pa, pb] (same layout as the kernel's set-up).
static int64_t range_lds(const StreamProblem* hp, int pa, int pb, int a, int b) {
    int64_t n = (int64_t)(pb - pa + 1) * (int64_t)sizeof(ProbL) +
                (int64_t)kWaves * kDepth * kSlotBytes;
    for (int p = pa; p <= pb; ++p) {
        const StreamProblem& s = hp[p];
        const int ca = std::max(a, s.chunk_begin) - s.chunk_begin;
        const int cb = std::min(b, s.chunk_begin + s.nchunks) - s.chunk_begin;
        const int64_t ra = ((int64_t)ca * kChunkBlocks) / s.bpr;
        const int64_t rb = std::min<int64_t>(s.N, ((int64_t)cb * kChunkBlocks + s.bpr - 1) / s.bpr);
        n += (int64_t)s.bpr * kXColBytes + ((rb - ra) + (cb - ca)) * 4;
    }
    return n + 16;
}

// Problem holding chunk c (host copy of the table; binary search).
static int prob_of_chunk(const StreamProblem* hp, int nprob, int c) {
    int lo = 0, hi = nprob - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (hp[mid].chunk_begin <= c) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// The first row-aligned chunk boundary at or after global chunk c (a
// problem's first and last chunk boundaries are row-aligned).
static int aligned_at(const StreamProblem* hp, int nprob, int64_t c) {
    const int p = prob_of_chunk(hp, nprob, (int)c);
    const StreamProblem& P = hp[p];
    const int64_t lc = c - P.chunk_begin;
    const int64_t t = tile_chunks(P.bpr);
    const int64_t up = std::min<int64_t>((lc + t - 1) / t * t, P.nchunks);
    return P.chunk_begin + (int)up;
}

int launch_gemv_stream(const StreamProblem* dev_probs, const StreamProblem* host_probs,
                       int nprob, int y_dtype, hipStream_t stream) {
    if (nprob == 0) return NB_OK;
    const StreamProblem& last = host_probs[nprob - 1];
    const int total = last.chunk_begin + last.nchunks;
    if (total == 0) return NB_OK;
    const int64_t lds_max = device_lds_bytes();

    // Ranges balanced by chunks, one per workgroup: each takes an equal
    // share of the chunks still unassigned, snapped forward to a row
    // boundary.  A range whose problems, x vectors and outputs do not fit in
    // LDS first ends early, at the start of its last problem (the later
    // ranges share the piece); failing that it is halved (at a row
    // boundary) until it fits.
    const int64_t G = std::min<int64_t>((int64_t)device_cu_count() * NB_STREAM_WG_PER_CU, total);
    auto fits = [&](int a, int b) {
        return range_lds(host_probs, prob_of_chunk(host_probs, nprob, a),
                         prob_of_chunk(host_probs, nprob, b - 1), a, b) <= lds_max;
    };
    std::vector<int> out;
    out.reserve((size_t)G + 8);
    out.push_back(0);
    for (int64_t g = 1; g <= G; ++g) {
        const int a = out.back();
        int b = g == G ? total : aligned_at(host_probs, nprob, a + (total - a) / (G - g + 1));
        if (b <= a) continue;
        if (!fits(a, b)) {
            const int pl = host_probs[prob_of_chunk(host_probs, nprob, b - 1)].chunk_begin;
            if (pl > a && fits(a, pl)) b = pl;
        }
        std::vector<std::pair<int, int>> todo{{a, b}};
        while (!todo.empty()) {
            auto [x0, x1] = todo.back();
            todo.pop_back();
            if (x0 >= x1) continue;
            if (fits(x0, x1)) {
                out.push_back(x1);
                continue;
            }
            const int mid = aligned_at(host_probs, nprob, x0 + (x1 - x0) / 2);
            if (mid <= x0 || mid >= x1) {
                return fail(NB_EUNSUPPORTED,
                            "nb_gemv_batched: one row-aligned tile needs more LDS than %lld bytes",
                            (long long)lds_max);
            }
            todo.push_back({mid, x1});  // popped second
            todo.push_back({x0, mid});
        }
    }
    if (out.back() != total) out.push_back(total);  // (never: the last range ends at total)
    // launch in chunks of at most kStreamMaxGroups workgroups
    const int nranges = (int)out.size() - 1;
    for (int c0 = 0; c0 < nranges; c0 += kStreamMaxGroups) {
        const int n = std::min(kStreamMaxGroups, nranges - c0);
        StreamRanges R;
        int64_t lds = 0;
        for (int i = 0; i <= n; ++i) R.chunk0[i] = out[(size_t)(c0 + i)];
        for (int i = 0; i < n; ++i) {
            R.prob0[i] = prob_of_chunk(host_probs, nprob, R.chunk0[i]);
            R.prob1[i] = prob_of_chunk(host_probs, nprob, R.chunk0[i + 1] - 1);
            lds = std::max(lds, range_lds(host_probs, R.prob0[i], R.prob1[i], R.chunk0[i],
                                          R.chunk0[i + 1]));
        }
        hipLaunchKernelGGL(gemv_stream_kernel, dim3(n), dim3(64 * kWaves), (size_t)lds, stream,
                           dev_probs, R, y_dtype);
        const int st = check_launch("nb_gemv_batched");
        if (st) return st;
    }
    return NB_OK;
}

}  // namespace nb
