// Batched packed skinny GEMM on gfx950: many 3-bit layers, M <= 16
// activation rows, one launch.
//
//   for every problem p:  y_p[m][n] = sum_k x_p[m][k] * bf16(W_p[n][k]),  m < M
//
// The batched branch of PackedLinear.forward (inference/triton_kernel.py:
// 258-275) in its bf16 form (inference/eval_ppl.py:149-174) for the few
// token rows of a small-batch decode step, over all layers of the step.
//
// Work split.  A task is 128 R rows of one problem over all of K (R = 2 on
// the tile layout, 1 on the reference layout: skinny_r), taken in slices
// of 512 (4 blocks of 128); an item is one 128-row part (h = 0 .. R - 1) of
// one slice, items in (slice, h) order, and wave w of a workgroup owns rows
// 128 h + 16w .. + 15 of the task in item (s, h).  The R items of a slice
// share one x slice, so the workgroup loads x once per R x 40 KiB of
// weights (with the MFMAs removed, the kernel's time follows the bytes it
// brings into LDS, x included: 221 / 274 us at M = 5 / 16 for 45 / 56 KiB
// per item).  The grid is one workgroup per CU, each walking a
// contiguous range of tasks balanced by item count, so a workgroup's loads
// run on from one task into the next without a ramp.
//
// Memory side.  Each wave keeps a ring of three LDS slots, one slice each
// (16 rows x 4 blocks: 3 KiB of indices, 2 KiB of codebook), filled by
// global_load_lds_dwordx4: five instructions of 1 KiB, in which the lanes of
// one row read that row's contiguous 192 (128) bytes, so every instruction
// touches a few whole cache lines.  Within a row the 16-byte pieces land
// rotated -- index blocks by idx_rot(r) blocks, codebook pieces by
// cb_rot(r) pieces -- which makes the compute side's LDS reads
// conflict-free.  Slices i + 1 and i + 2 are in flight while slice i is
// computed.  The x slice
// (M rows x 512 bf16) arrives the same way into workgroup buffers of M
// rows, its 16-byte pieces placed by an XOR of the row so that the 16
// columns of one B-operand read fall in different banks: three buffers (x
// two slices ahead) where they fit beside the rings (M <= 13), else two.
//
// Compute side (unchanged arithmetic): lane l = q*16 + r takes row r of the
// wave's group and block q of the slice, reads its 48 index bytes and 8
// codebook entries from the slot, and turns them into 16 A-operands of
// v_mfma_f32_16x16x32_bf16 by register codebook lookups (v_perm_b32 on byte
// planes of the bf16-rounded entries, 17 VALU ops per 8 weights).  B is the
// x slice: MFMA column c = activation row min(c, M - 1).  The accumulator
// (16 rows x 16 columns per wave) stays in registers over all of K and is
// stored when the task's last slice is done: no cross-wave reduction.
//
// Tile layout (nb_tile_layout).  A one-time re-ordering of a layer for
// this kernel: the blocks of 16 rows x 4 column blocks (one wave's slice)
// are stored as the LDS image of a slot -- 3 KiB of indices, 2 KiB of
// codebook in two arrays, rows rotated as above -- tile (g, s) at tile
// index g * ceil(bpr / 4) + s, rows past N and blocks past bpr zero.  A
// slice then arrives by five contiguous 1 KiB loads (the access shape
// under which MI355X streams fastest) instead of 16 row pieces of 192 and
// 128 bytes.  Within every 12-byte unit of 32 indices, index 4s + t
// (s = 0..7, t = 0..3) is stored at index position o(s) + 8t,
// o = (0, 1, 3, 4, 6, 7, 2, 5): the byte-class extraction of the M = 1
// kernel (nb_stream_common.h, unit_selectors: 25 VALU ops per 32 indices)
// then yields selector s = indices 4s .. 4s + 3 in natural order, and two
// selectors are the 8 consecutive weights of one A operand -- 14.25 VALU
// ops per 8 weights instead of 17 plus the per-group selector builds.
// The MFMAs, their order and the x pieces are those of the reference
// layout, so both layouts give the same bits.
//
// Weights are rounded to bf16 (RNE), as the reference's bf16 path;
// accumulation is fp32.
#include <algorithm>
#include <type_traits>
#include <vector>

#include "nb_device.h"
#include "nb_internal.h"
#include "nb_stream_common.h"

namespace nb {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;

// waves per workgroup and slots per wave ring
#ifndef NB_SK_WAVES
#define NB_SK_WAVES 8
#endif
#ifndef NB_SK_DEPTH
#define NB_SK_DEPTH 3
#endif
constexpr int kSkWaves = NB_SK_WAVES;
constexpr int kSkThreads = 64 * kSkWaves;
constexpr int kSkRows = 16 * kSkWaves;         // rows of one item
// 128-row items per slice of a task: two on the tile layout; one on the
// reference layout, whose row bases are re-derived whenever the item's rows
// change (with two it measured slower: 312 -> 335 us at M = 16)
__host__ __device__ constexpr int skinny_r(bool tile) { return tile ? 2 : 1; }
constexpr int kSkSliceK = 512;                 // K of one slice (4 blocks)
constexpr int kSkMaxM = 16;
constexpr int kSkXRow = kSkSliceK * 2;         // LDS bytes of one staged x row
constexpr int kSkIdxBytes = 16 * 192;          // indices of one slot
constexpr int kSkSlot = kSkIdxBytes + 16 * 128;  // + codebooks
constexpr int kSkDepth = NB_SK_DEPTH;          // slots per wave
constexpr int kSkRing = kSkWaves * kSkDepth * kSkSlot;
constexpr int kSkLdsMax = 160 * 1024;
static_assert(kSkRing + 2 * kSkMaxM * kSkXRow <= kSkLdsMax, "LDS");
static_assert(kSkSlot == 5 * 1024, "five 1 KiB loads per slot");
// x buffers of a launch: three (x two slices ahead) when M rows of them fit
// beside the ring, else two (one slice ahead)
__host__ __device__ constexpr int skinny_xbufs(int M) {
    return kSkRing + 3 * M * kSkXRow <= kSkLdsMax ? 3 : 2;
}

// Rotations of row r (0..15) of a slot: its 48-byte index blocks b sit at
// block place (b + idx_rot(r)) & 3 of its 192 bytes, its 16-byte codebook
// pieces p at place (p + cb_rot(r)) & 7 of its 128 bytes.  A ds_read_b128
// of the compute side has the 16 lanes (q, r = 0..15) read one piece each
// of the same block q: with these rotations the 16 pieces fall in 16
// different 4-bank groups of the 64 banks, and each half of 8 lanes in 8
// different groups of 32 banks.
__host__ __device__ constexpr int idx_rot(int r) { return ((r >> 1) & 3) + (r >> 3); }
__host__ __device__ constexpr int cb_rot(int r) { return (r & 6) | ((r ^ (r >> 3)) & 1); }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
    bf16x2_t v;
    v.x = (__bf16)lo;
    v.y = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
}

// 8 bf16 weights (natural order) of one 24-bit index group `g` from the
// codebook byte planes lo0/lo1 (low bytes of entries 0-3 / 4-7) and
// hi0/hi1 (high bytes).
__device__ __forceinline__ u32x4_t lookup8(uint32_t g, uint32_t lo0, uint32_t lo1,
                                           uint32_t hi0, uint32_t hi1) {
    // lo16 = indices 0-3 at bits 0,3,6,9; hi16 = indices 4-7 likewise
    const uint32_t h = __builtin_amdgcn_ubfe(g, 0, 16) | ((g << 4) & 0xFFFF0000u);
    // selector bytes (i0, i1, i4, i5) and (i2, i3, i6, i7)
    const uint32_t sa = (h & 0x00070007u) | ((h << 5) & 0x07000700u);
    const uint32_t sb = ((h >> 6) & 0x00070007u) | ((h >> 1) & 0x07000700u);
    const uint32_t la = __builtin_amdgcn_perm(lo1, lo0, sa);
    const uint32_t ha = __builtin_amdgcn_perm(hi1, hi0, sa);
    const uint32_t lb = __builtin_amdgcn_perm(lo1, lo0, sb);
    const uint32_t hb = __builtin_amdgcn_perm(hi1, hi0, sb);
    u32x4_t w;
    w.x = __builtin_amdgcn_perm(ha, la, 0x05010400u);  // (w0, w1)
    w.y = __builtin_amdgcn_perm(hb, lb, 0x05010400u);  // (w2, w3)
    w.z = __builtin_amdgcn_perm(ha, la, 0x07030602u);  // (w4, w5)
    w.w = __builtin_amdgcn_perm(hb, lb, 0x07030602u);  // (w6, w7)
    return w;
}

// Group j (0..15) of eight 3-bit indices of a 128-index block in 12 dwords.
template <int J>
__device__ __forceinline__ uint32_t group24(const uint32_t (&d)[12]) {
    constexpr int bit = J * 24;
    constexpr int w = bit >> 5;
    constexpr int off = bit & 31;
    if constexpr (off == 0) {
        return d[w];
    } else if constexpr (off + 24 <= 32) {
        return d[w] >> off;
    } else {
        return __builtin_amdgcn_alignbit(d[w + 1], d[w], off);
    }
}

// The 16 MFMAs of a lane's block: group J of the block's indices times x
// piece q*16 + J of the lane's activation row, stored at place
// (q*16 + J) ^ swz of that row.
template <int J>
__device__ __forceinline__ void mfma_groups(const uint32_t (&d)[12], uint32_t lo0, uint32_t lo1,
                                            uint32_t hi0, uint32_t hi1,
                                            const unsigned char* xrow, int piece0, int swz,
                                            f32x4_t& acc) {
    if constexpr (J < 16) {
        const u32x4_t a = lookup8(group24<J>(d), lo0, lo1, hi0, hi1);
        const u32x4_t b =
            *reinterpret_cast<const u32x4_t*>(xrow + 16 * ((piece0 + J) ^ swz));
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                      __builtin_bit_cast(bf16x8_t, b), acc,
                                                      0, 0, 0);
        mfma_groups<J + 1>(d, lo0, lo1, hi0, hi1, xrow, piece0, swz, acc);
    }
}

// The same 16 MFMAs on the tile layout's index order: unit U (32 indices,
// dwords d[3U .. 3U + 2], a selector-ordered unit) gives groups 4U .. 4U +
// 3, selectors 2p and 2p + 1 being the eight weights of group 4U + p in
// natural order (17 VALU ops a unit to take the selectors).
template <int U>
__device__ __forceinline__ void mfma_units_tile(const uint32_t (&d)[12], uint32_t lo0,
                                               uint32_t lo1, uint32_t hi0, uint32_t hi1,
                                               const unsigned char* xrow, int piece0, int swz,
                                               f32x4_t& acc) {
    if constexpr (U < 4) {
        uint32_t sel[8];
        stream::unit_selectors_sel(d[3 * U], d[3 * U + 1], d[3 * U + 2], sel);
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t la = __builtin_amdgcn_perm(lo1, lo0, sel[2 * p]);
            const uint32_t ha = __builtin_amdgcn_perm(hi1, hi0, sel[2 * p]);
            const uint32_t lb = __builtin_amdgcn_perm(lo1, lo0, sel[2 * p + 1]);
            const uint32_t hb = __builtin_amdgcn_perm(hi1, hi0, sel[2 * p + 1]);
            u32x4_t a;
            a.x = __builtin_amdgcn_perm(ha, la, 0x05010400u);  // (w0, w1)
            a.y = __builtin_amdgcn_perm(ha, la, 0x07030602u);  // (w2, w3)
            a.z = __builtin_amdgcn_perm(hb, lb, 0x05010400u);  // (w4, w5)
            a.w = __builtin_amdgcn_perm(hb, lb, 0x07030602u);  // (w6, w7)
            const u32x4_t b =
                *reinterpret_cast<const u32x4_t*>(xrow + 16 * ((piece0 + 4 * U + p) ^ swz));
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                          __builtin_bit_cast(bf16x8_t, b), acc,
                                                          0, 0, 0);
        }
        mfma_units_tile<U + 1>(d, lo0, lo1, hi0, hi1, xrow, piece0, swz, acc);
    }
}

// global_load_lds_dwordx4: 16 bytes per lane from `src` to
// LDS address m0 + 16 * lane (m0 = the wave-uniform `lds`).  Completion is
// tracked by vmcnt only; the compiler does not see the LDS write, so the
// waits below are explicit.
__device__ __forceinline__ void dma16(uint32_t lds, const void* src) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(lds), "v"(src)
                 : "memory", "m0");
}

// The same load marked non-temporal: weights are read once per launch.
__device__ __forceinline__ void dma16_nt(uint32_t lds, const void* src) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off nt"
                 :
                 : "s"(lds), "v"(src)
                 : "memory", "m0");
}

// Waits until at most N vector-memory operations of this wave are
// outstanding (they complete in issue order).
template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// wait_vm for a wave-uniform n (a scalar branch to the immediate form;
// n outside 1..24 waits for everything, which is always enough).
__device__ __forceinline__ void wait_vm_n(int n) {
    switch (n) {
#define NB_SK_CASE(k) \
    case k:           \
        wait_vm<k>(); \
        break;
        NB_SK_CASE(1) NB_SK_CASE(2) NB_SK_CASE(3) NB_SK_CASE(4) NB_SK_CASE(5) NB_SK_CASE(6)
        NB_SK_CASE(7) NB_SK_CASE(8) NB_SK_CASE(9) NB_SK_CASE(10) NB_SK_CASE(11) NB_SK_CASE(12)
        NB_SK_CASE(13) NB_SK_CASE(14) NB_SK_CASE(15) NB_SK_CASE(16) NB_SK_CASE(17)
        NB_SK_CASE(18) NB_SK_CASE(19) NB_SK_CASE(20) NB_SK_CASE(21) NB_SK_CASE(22)
        NB_SK_CASE(23) NB_SK_CASE(24)
#undef NB_SK_CASE
        default:
            wait_vm<0>();
    }
}

// Workgroup barrier that waits for this wave's LDS operations only, not
// for its loads in flight (a __syncthreads would drain the prefetch).
__device__ __forceinline__ void wg_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory");
}

template <typename T>
__device__ __forceinline__ uint32_t lds_addr(T* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) T*)p;
}

struct SkinnyArgs {
    const StreamProblem* probs;
    SkinnyTasks tasks;
    int32_t wg_task0[kStreamMaxGroups + 1];  // task range of workgroup g
    int M, y_dtype;
};

// A position in the workgroup's (task, slice) sequence and the fields of
// its problem (wave-uniform).
struct Cursor {
    int p;        // problem index (relative to tasks.prob0)
    int task;     // task index of the launch
    int s;        // slice of the task
    int h;        // 128-row half of the task (item (s, h))
    int ns;       // slices of the problem
    int row0;     // first row of the wave's group
    int N, K, bpr;
    const uint8_t* packed;
    const float* cb;
    const uint16_t* x;
};

// The problem table is read through the constant address space with a
// wave-uniform index: scalar loads, counted on lgkmcnt, so they never make
// the compiler wait on vmcnt (which would drain the weight prefetch).
typedef const __attribute__((address_space(4))) StreamProblem* prob_cptr;
__device__ __forceinline__ prob_cptr problem(const SkinnyArgs& a, int p) {
    return (prob_cptr)a.probs + (a.tasks.prob0 + p);
}

__device__ __forceinline__ void cursor_load(const SkinnyArgs& a, Cursor& c) {
    const prob_cptr P = problem(a, c.p);
    c.N = P->N;
    c.K = P->K;
    c.bpr = P->K >> 7;
    c.ns = (c.bpr + 3) >> 2;
    c.packed = P->packed;
    c.cb = P->codebook;
    c.x = static_cast<const uint16_t*>(P->x);
}

template <int R>
__device__ __forceinline__ void cursor_rows(const SkinnyArgs& a, Cursor& c, int wave) {
    c.row0 = (c.task - a.tasks.task_begin[c.p]) * (R * kSkRows) + c.h * kSkRows + wave * 16;
}

// the next slice (h stays 0: the x cursor, one step per slice)
template <int R>
__device__ __forceinline__ void cursor_next_slice(const SkinnyArgs& a, Cursor& c, int wave) {
    if (++c.s < c.ns) return;
    c.s = 0;
    ++c.task;
    if (c.p + 1 < a.tasks.nprob && c.task >= a.tasks.task_begin[c.p + 1]) {
        ++c.p;
        cursor_load(a, c);
    }
    cursor_rows<R>(a, c, wave);
}

// the next item
template <int R>
__device__ __forceinline__ void cursor_next(const SkinnyArgs& a, Cursor& c, int wave) {
    if (++c.h < R) {
        cursor_rows<R>(a, c, wave);
        return;
    }
    c.h = 0;
    cursor_rows<R>(a, c, wave);
    cursor_next_slice<R>(a, c, wave);
}

template <int NXB, bool TILE>
__global__ __launch_bounds__(kSkThreads) void gemv_skinny_kernel(SkinnyArgs a) {
    constexpr int kSkR = skinny_r(TILE);
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int r = lane & 15;
    const int q = lane >> 4;
    const int M = a.M;
    const int t0 = a.wg_task0[blockIdx.x], t1 = a.wg_task0[blockIdx.x + 1];
    if (t0 >= t1) return;

    // ---- the first task's problem (binary search over the task prefix) ----
    Cursor cc;
    {
        int lo = 0, hi = a.tasks.nprob - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (a.tasks.task_begin[mid] <= t0) lo = mid; else hi = mid - 1;
        }
        cc.p = lo;
        cc.task = t0;
        cc.s = 0;
        cc.h = 0;
        cursor_load(a, cc);
        cursor_rows<kSkR>(a, cc, wave);
    }
    // items (task, slice) of the workgroup
    int nitems = 0;
    {
        Cursor c = cc;
        for (int t = t0; t < t1; ++t) {
            if (c.p + 1 < a.tasks.nprob && t >= a.tasks.task_begin[c.p + 1]) {
                ++c.p;
                cursor_load(a, c);
            }
            nitems += c.ns * kSkR;
        }
    }

    // LDS: the waves' rings, then NXB x buffers of M rows
    const uint32_t base = lds_addr(smem);
    const uint32_t ring = base + wave * kSkDepth * kSkSlot;
    const unsigned char* ring_p = smem + wave * kSkDepth * kSkSlot;
    const int xbuf_bytes = M * kSkXRow;

    // Per-lane constants of the weight loads: load i < 3 (indices) puts
    // piece P = 64 i + lane of the slot at row P / 12, place P % 12, which
    // holds piece (place - 3 (idx_rot(row) & 3)) mod 12 of the row; load
    // 3 + i (codebooks) puts P = 64 i + lane at row P / 8, place P % 8,
    // holding piece (place - cb_rot(row)) & 7.
    int w_row[5], w_blk[5], w_off[5];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int P = 64 * i + lane;
        const int rr = P / 12, place = P % 12;
        const int piece = (place - 3 * (idx_rot(rr) & 3) + 12) % 12;
        w_row[i] = rr;
        w_blk[i] = piece / 3;
        w_off[i] = (piece % 3) * 16;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int P = 64 * i + lane;
        const int rr = P >> 3, place = P & 7;
        const int piece = (place - cb_rot(rr)) & 7;
        w_row[3 + i] = rr;
        w_blk[3 + i] = piece >> 1;
        w_off[3 + i] = (piece & 1) * 16;
    }
    // Row bases of the weight loads of the W cursor's item rows (recomputed
    // when they change): per load, the row's first index byte or codebook
    // byte plus the lane's offset inside a block.
    const unsigned char* wbase[5];
    int wtask = -1, wh = -1;
    auto w_rows = [&](const Cursor& c) {
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const int64_t row = min(c.row0 + w_row[i], c.N - 1);
            wbase[i] = i < 3 ? c.packed + row * c.bpr * 48 + w_off[i]
                             : reinterpret_cast<const unsigned char*>(c.cb) + row * c.bpr * 32 +
                                   w_off[i];
        }
        wtask = c.task;
        wh = c.h;
    };
    auto issue_w = [&](const Cursor& c, int slot) {
        const uint32_t dst = __builtin_amdgcn_readfirstlane(ring + slot * kSkSlot);
        if constexpr (TILE) {
            // the slot's image: tile (group, slice), groups past the
            // layer's last read its last (their rows are not stored)
            const int64_t g = min(c.row0 >> 4, (c.N - 1) >> 4);
            const int64_t tile = g * c.ns + c.s;
            const unsigned char* ib = c.packed + tile * kSkIdxBytes + 16 * lane;
            const unsigned char* cp =
                reinterpret_cast<const unsigned char*>(c.cb) + tile * (kSkSlot - kSkIdxBytes) +
                16 * lane;
            dma16_nt(dst, ib);
            dma16_nt(dst + 1024, ib + 1024);
            dma16_nt(dst + 2048, ib + 2048);
            dma16_nt(dst + 3072, cp);
            dma16_nt(dst + 4096, cp + 1024);
        } else {
            if (c.task != wtask || c.h != wh) w_rows(c);
#pragma unroll
            for (int i = 0; i < 5; ++i) {
                const int blk = min(4 * c.s + w_blk[i], c.bpr - 1);
                dma16(dst + 1024 * i, wbase[i] + blk * (i < 3 ? 48 : 32));
            }
        }
    };
    // x slice of slice c.s into buffer `buf`: wave w loads activation rows
    // min(2w + j, M - 1), j = 0, 1 -- always two loads, so the wait counts
    // below are exact (a clamped row rewrites row M - 1 with the same bytes,
    // before anyone reads that buffer).  Lane l takes the 16 bytes of
    // column piece l ^ (m & 15), so piece p of row m sits at place
    // p ^ (m & 15): the 16 rows of one B-operand read fall in 16 different
    // 4-bank groups (and each 8 of them in 8 groups of 32 banks).  Columns
    // past K repeat the last 8 (their weights are zero).
    auto issue_x = [&](const Cursor& c, int buf) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int m = min(2 * wave + j, M - 1);
            const int piece = lane ^ (m & 15);
            const int k = min(c.s * kSkSliceK + piece * 8, c.K - 8);
            dma16(__builtin_amdgcn_readfirstlane(base + kSkRing + buf * xbuf_bytes + m * kSkXRow),
                  c.x + (int64_t)m * c.K + k);
        }
    };

    // MFMA column r reads activation row min(r, M - 1)
    const int xm = r < M ? r : M - 1;
    // this lane's pieces of a slot (rotated places, see above)
    const int idx_off = r * 192 + ((q + idx_rot(r)) & 3) * 48;
    const int cb_off0 = kSkIdxBytes + r * 128 + ((2 * q + cb_rot(r)) & 7) * 16;
    const int cb_off1 = kSkIdxBytes + r * 128 + ((2 * q + 1 + cb_rot(r)) & 7) * 16;
    const int x_off = xm * kSkXRow;
    const int x_swz = xm & 15;
    // one accumulator per 128-row half of the task
    f32x4_t acc[kSkR];
#pragma unroll
    for (int h = 0; h < kSkR; ++h) acc[h] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // A finished task's outputs wait in `pend` and are stored after the
    // next item's loads are issued.  acc[h] lane (q, r) holds C[4q + v][r]:
    // y[r][row0 + 128 h + 4q + v], row0 the first row of the wave in half 0.
    f32x4_t pend[kSkR];
    int pend_p = 0, pend_row0 = 0, pend_n = 0;
    bool pending = false;
    auto store = [&]() {
        pending = false;
        if (r >= M) return;
        const prob_cptr P = problem(a, pend_p);
        const bool add = P->y_mode == NB_Y_ADD;
        void* y = P->y;
#pragma unroll
        for (int h = 0; h < kSkR; ++h) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int n = pend_row0 + h * kSkRows + 4 * q + v;
                if (n >= pend_n) continue;
                const int64_t yi = (int64_t)r * pend_n + n;
                if (a.y_dtype == NB_BF16) {
                    *as_global_mut(static_cast<bf16_bits*>(y) + yi) =
                        f32_to_bf16_rne(pend[h][v]);
                } else if (add) {
                    auto* yp = as_global_mut(static_cast<float*>(y) + yi);
                    *yp = *yp + pend[h][v];
                } else {
                    *as_global_mut(static_cast<float*>(y) + yi) = pend[h][v];
                }
            }
        }
    };

    // ---- the pipeline -----------------------------------------------------
    // Item i's weights W(i) (five loads) go to slot i % kSkDepth; slice g's x
    // X(g) (two loads, g = i / R for item i) to buffer g % NXB.  Before the
    // loop: X(0 .. kLead - 1), then W(0 .. kSkDepth - 1).  Item i's step
    // waits until W(i) is in -- and for the first item of a slice X(g) too,
    // then passes the workgroup barrier (every wave's x pieces of slice g
    // are in, and every wave is done with slice g - 1, whose x buffer
    // X(g + kLead) refills) -- reads slot i into registers, issues
    // X(g + kLead) (first item of a slice), computes, and then issues
    // W(i + kSkDepth) into the slot it read.  kSkDepth slices of weights
    // are in flight while one is computed.  Loads complete in issue order,
    // so what a step needs is in once at most after(i) loads are
    // outstanding: those issued after the later of W(i) and X(g).  (Output
    // stores, issued after a step's loads, only make the waits longer.)
    constexpr int kLead = NXB - 1;  // slices between X's issue and use
    const int nslices = nitems / kSkR;
    auto x_at = [&](int j) {  // x loads issued in step j
        return (j % kSkR == 0 && j / kSkR + kLead < nslices) ? 2 : 0;
    };
    auto w_at = [&](int j) { return j + kSkDepth < nitems ? 5 : 0; };  // in step j
    auto after = [&](int i) {
        int nw = 0;  // loads issued after W(i)
        if (i < kSkDepth) {
            for (int d = i + 1; d < kSkDepth && d < nitems; ++d) nw += 5;
            for (int j = 0; j < i; ++j) nw += x_at(j) + w_at(j);
        } else {
            for (int j = i - kSkDepth + 1; j < i; ++j) nw += x_at(j) + w_at(j);
        }
        if (i % kSkR != 0) return nw;
        const int g = i / kSkR;
        int nx = 0;  // loads issued after X(g)
        if (g < kLead) {
            for (int gg = g + 1; gg < kLead && gg < nslices; ++gg) nx += 2;
            for (int d = 0; d < kSkDepth && d < nitems; ++d) nx += 5;
            for (int j = 0; j < i; ++j) nx += x_at(j) + w_at(j);
        } else {
            const int j0 = (g - kLead) * kSkR;  // the step that issued X(g)
            nx = w_at(j0);
            for (int j = j0 + 1; j < i; ++j) nx += x_at(j) + w_at(j);
        }
        return min(nw, nx);
    };
    Cursor cx = cc, cw = cc;
    for (int g = 0; g < kLead && g < nslices; ++g) {
        issue_x(cx, g % NXB);
        cursor_next_slice<kSkR>(a, cx, wave);
    }
    for (int d = 0; d < kSkDepth && d < nitems; ++d) {
        issue_w(cw, d);
        cursor_next<kSkR>(a, cw, wave);
    }

    // item i (half H of its slice) into acc[H]
    auto step = [&](int i, auto h_c) {
        constexpr int H = decltype(h_c)::value;
        const int g = i / kSkR;
        wait_vm_n(after(i));
        if (H == 0) wg_barrier();
        // ---- slot i into registers, then this step's loads ----
        const int si = i % kSkDepth;
        const unsigned char* slot = ring_p + si * kSkSlot;
        uint32_t d[12];
        {
            const u32x4_t* ip = reinterpret_cast<const u32x4_t*>(slot + idx_off);
#pragma unroll
            for (int v = 0; v < 3; ++v) {
                const u32x4_t u = ip[v];
                d[4 * v] = u.x;
                d[4 * v + 1] = u.y;
                d[4 * v + 2] = u.z;
                d[4 * v + 3] = u.w;
            }
        }
        const f32x4_t c0 = *reinterpret_cast<const f32x4_t*>(slot + cb_off0);
        const f32x4_t c1 = *reinterpret_cast<const f32x4_t*>(slot + cb_off1);
        // the slot's bytes are in registers before its refill is issued
        asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
        if (H == 0 && g + kLead < nslices) {
            issue_x(cx, (g + kLead) % NXB);
            cursor_next_slice<kSkR>(a, cx, wave);
        }
        if (pending) store();
        // ---- compute item (cc.s, H) of the task ----
        const bool live = cc.row0 + r < cc.N && 4 * cc.s + q < cc.bpr;
        const uint32_t p0 = pack_bf16x2(c0.x, c0.y);
        const uint32_t p1 = pack_bf16x2(c0.z, c0.w);
        const uint32_t p2 = pack_bf16x2(c1.x, c1.y);
        const uint32_t p3 = pack_bf16x2(c1.z, c1.w);
        uint32_t lo0 = __builtin_amdgcn_perm(p1, p0, 0x06040200u);
        uint32_t hi0 = __builtin_amdgcn_perm(p1, p0, 0x07050301u);
        uint32_t lo1 = __builtin_amdgcn_perm(p3, p2, 0x06040200u);
        uint32_t hi1 = __builtin_amdgcn_perm(p3, p2, 0x07050301u);
        lo0 = live ? lo0 : 0u;
        hi0 = live ? hi0 : 0u;
        lo1 = live ? lo1 : 0u;
        hi1 = live ? hi1 : 0u;
        const unsigned char* xb = smem + kSkRing + (g % NXB) * xbuf_bytes + x_off;
        if constexpr (TILE) {
            mfma_units_tile<0>(d, lo0, lo1, hi0, hi1, xb, q * 16, x_swz, acc[H]);
        } else {
            mfma_groups<0>(d, lo0, lo1, hi0, hi1, xb, q * 16, x_swz, acc[H]);
        }
        // the weights of step i + kSkDepth into the slot read above, after
        // the MFMAs: issued before them, the five loads can stall at issue
        // behind a full memory queue, and the wave with them
        if (i + kSkDepth < nitems) {
            issue_w(cw, si);
            cursor_next<kSkR>(a, cw, wave);
        }
        if (H == kSkR - 1 && cc.s == cc.ns - 1) {
#pragma unroll
            for (int h = 0; h < kSkR; ++h) {
                pend[h] = acc[h];
                acc[h] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            }
            pend_p = cc.p;
            pend_row0 = cc.row0 - H * kSkRows;
            pend_n = cc.N;
            pending = true;
        }
        cursor_next<kSkR>(a, cc, wave);
    };
    for (int i = 0; i < nitems; i += kSkR) {
        step(i, std::integral_constant<int, 0>{});
        if constexpr (kSkR > 1) step(i + 1, std::integral_constant<int, 1>{});
        if constexpr (kSkR > 2) step(i + 2, std::integral_constant<int, 2>{});
        if constexpr (kSkR > 3) step(i + 3, std::integral_constant<int, 3>{});
    }
    if (pending) store();
}

// Index position of index i (= 4s + t) of a 32-index unit in the tile
// layout: o(s) + 8t, o(s) = stream::sel_offset(s).
__host__ __device__ constexpr int sel_position(int i) {
    return stream::sel_offset(i >> 2) + 8 * (i & 3);
}

// 3-bit field at index position i of a 12-byte unit (dwords u[0..2])
template <int I>
__device__ __forceinline__ uint32_t unit_field(const uint32_t* u) {
    constexpr int bit = 3 * I, w = bit >> 5, off = bit & 31;
    if constexpr (off <= 29) {
        return (u[w] >> off) & 7u;
    } else {
        return ((u[w] >> off) | (u[w + 1] << (32 - off))) & 7u;
    }
}

template <int I>
__device__ __forceinline__ void unit_put(uint32_t* u, uint32_t f) {
    constexpr int bit = 3 * I, w = bit >> 5, off = bit & 31;
    u[w] |= f << off;
    if constexpr (off > 29) u[w + 1] |= f >> (32 - off);
}

template <int I>
__device__ __forceinline__ void sel_unit(const uint32_t* in, uint32_t* out) {
    if constexpr (I < 32) {
        unit_put<sel_position(I)>(out, unit_field<I>(in));
        sel_unit<I + 1>(in, out);
    }
}

// One thread per block place of a tile (64 per tile: row rr, block blk of
// the slice): the block's 48 index bytes (each 12-byte unit the
// selector-ordered unit whose selector s holds indices 4s .. 4s + 3) at the rotated
// place the kernel's slot holds them, its 8 codebook entries as two
// rotated 16-byte pieces; zeros where the row or block is past the layer.
__global__ __launch_bounds__(256) void tile_layout_kernel(const uint8_t* packed,
                                                          const float* codebook, int N, int bpr,
                                                          int ns, int64_t nthreads, uint8_t* tp,
                                                          float* tc) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= nthreads) return;
    const int64_t tile = t >> 6;
    const int rr = (int)(t >> 2) & 15, blk = (int)t & 3;
    const int64_t row = tile / ns * 16 + rr;
    const int kb = (int)(tile % ns) * 4 + blk;
    uint32_t o[12] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    u32x4_t c0 = {0u, 0u, 0u, 0u}, c1 = c0;
    if (row < N && kb < bpr) {
        const int64_t b = row * bpr + kb;
        const u32x4_t* src = reinterpret_cast<const u32x4_t*>(packed + b * 48);
        uint32_t d[12];
#pragma unroll
        for (int v = 0; v < 3; ++v) {
            const u32x4_t u = src[v];
            d[4 * v] = u.x;
            d[4 * v + 1] = u.y;
            d[4 * v + 2] = u.z;
            d[4 * v + 3] = u.w;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            // selector s = indices 4s .. 4s + 3, stored as the
            // selector-ordered unit (nb_stream_common.h, sel_unit_pack)
            uint32_t so[3] = {0u, 0u, 0u}, sel[8];
            sel_unit<0>(d + 3 * u, so);
            stream::unit_selectors(so[0], so[1], so[2], sel);
            stream::sel_unit_pack(sel, o[3 * u], o[3 * u + 1], o[3 * u + 2]);
        }
        const u32x4_t* cs = reinterpret_cast<const u32x4_t*>(codebook + b * 8);
        c0 = cs[0];
        c1 = cs[1];
    }
    u32x4_t* di = reinterpret_cast<u32x4_t*>(tp + tile * kSkIdxBytes + rr * 192 +
                                             ((blk + idx_rot(rr)) & 3) * 48);
#pragma unroll
    for (int v = 0; v < 3; ++v) {
        di[v] = u32x4_t{o[4 * v], o[4 * v + 1], o[4 * v + 2], o[4 * v + 3]};
    }
    unsigned char* dc = reinterpret_cast<unsigned char*>(tc) + tile * (kSkSlot - kSkIdxBytes) +
                        rr * 128;
    *reinterpret_cast<u32x4_t*>(dc + ((2 * blk + cb_rot(rr)) & 7) * 16) = c0;
    *reinterpret_cast<u32x4_t*>(dc + ((2 * blk + 1 + cb_rot(rr)) & 7) * 16) = c1;
}

}  // namespace

int64_t tile_layout_tiles(int N, int K) {
    return (int64_t)((N + 15) / 16) * ((K / 128 + 3) / 4);
}

int launch_tile_layout(const uint8_t* packed, const float* codebook, int N, int K,
                       uint8_t* tpacked, float* tcodebook, hipStream_t stream) {
    const int64_t nthreads = tile_layout_tiles(N, K) * 64;
    if (nthreads == 0) return NB_OK;
    const int64_t grid = (nthreads + 255) / 256;
    if (grid > 0x7fffffff) return fail(NB_EUNSUPPORTED, "nb_tile_layout: layer too large");
    hipLaunchKernelGGL(tile_layout_kernel, dim3((unsigned)grid), dim3(256), 0, stream, packed,
                       codebook, N, K / 128, (K / 128 + 3) / 4, nthreads, tpacked, tcodebook);
    return check_launch("nb_tile_layout");
}

int launch_gemv_skinny(const StreamProblem* dev_probs, const StreamProblem* host_probs,
                       int nprob, int M, int y_dtype, bool tile, hipStream_t stream) {
    const char* fn = tile ? "nb_gemm_skinny_tile_batched" : "nb_gemm_skinny_batched";
    const int cus = std::max(1, std::min(device_cu_count(), kStreamMaxGroups));
    // launches of at most kSkinnyMaxProbs problems each
    for (int p0 = 0; p0 < nprob; p0 += kSkinnyMaxProbs) {
        const int n = std::min(kSkinnyMaxProbs, nprob - p0);
        SkinnyArgs A;
        A.probs = dev_probs;
        A.tasks.prob0 = p0;
        A.tasks.nprob = n;
        A.M = M;
        A.y_dtype = y_dtype;
        // tasks and their slice counts, then contiguous task ranges, one per
        // workgroup, whose largest slice count is the least possible: the
        // smallest capacity C for which filling workgroups in order up to C
        // slices needs at most G of them (binary search), then that filling
        std::vector<int> slices;
        int64_t total_slices = 0;
        int max_slices = 0;
        for (int i = 0; i < n; ++i) {
            A.tasks.task_begin[i] = (int32_t)slices.size();
            const StreamProblem& P = host_probs[p0 + i];
            const int R = skinny_r(tile);
            const int nt = (P.N + R * kSkRows - 1) / (R * kSkRows);
            const int ns = (((P.K >> 7) + 3) >> 2) * R;  // items of a task
            for (int t = 0; t < nt; ++t) slices.push_back(ns);
            total_slices += (int64_t)nt * ns;
            max_slices = std::max(max_slices, ns);
            if (slices.size() > (size_t)0x7fffffff) {
                return fail(NB_EUNSUPPORTED, "%s: too many rows", fn);
            }
        }
        const int ntask = (int)slices.size();
        if (ntask == 0) continue;
        const int G = std::min(cus, ntask);
        auto groups_for = [&](int64_t cap) {
            int g = 1;
            int64_t acc = 0;
            for (int t = 0; t < ntask; ++t) {
                if (acc + slices[t] > cap) {
                    ++g;
                    acc = 0;
                }
                acc += slices[t];
            }
            return g;
        };
        int64_t lo = std::max<int64_t>(max_slices, (total_slices + G - 1) / G), hi = total_slices;
        while (lo < hi) {
            const int64_t mid = (lo + hi) / 2;
            if (groups_for(mid) <= G) hi = mid; else lo = mid + 1;
        }
        int used = 0;
        {
            int64_t acc = 0;
            A.wg_task0[0] = 0;
            for (int t = 0; t < ntask; ++t) {
                if (acc + slices[t] > lo) {
                    A.wg_task0[++used] = t;
                    acc = 0;
                }
                acc += slices[t];
            }
            A.wg_task0[++used] = ntask;
        }
        const size_t lds = (size_t)kSkRing + (size_t)skinny_xbufs(M) * M * kSkXRow;
        auto kernel = skinny_xbufs(M) == 3 ? (tile ? gemv_skinny_kernel<3, true>
                                                   : gemv_skinny_kernel<3, false>)
                                           : (tile ? gemv_skinny_kernel<2, true>
                                                   : gemv_skinny_kernel<2, false>);
        hipLaunchKernelGGL(kernel, dim3((unsigned)used), dim3(kSkThreads), lds, stream, A);
        const int st = check_launch(fn);
        if (st) return st;
    }
    return NB_OK;
}

}  // namespace nb
