// Batched packed skinny GEMM on gfx950: many 3-bit layers, M <= 16
// activation rows, one launch.
//
//   for every problem p:  y_p[m][n] = sum_k x_p[m][k] * bf16(W_p[n][k]),  m < M
//
// The batched branch of PackedLinear.forward (inference/triton_kernel.py:
// 258-275) in its bf16 form (inference/eval_ppl.py:149-174) for the few
// token rows of a small-batch decode step, over all layers of the step.
//
// Work split.  A task is 128 rows of one problem over all of K, taken in
// slices of 512 (4 blocks of 128); wave w of a workgroup owns rows 16w ..
// 16w + 15 of the task.  The grid is one workgroup per CU, each walking a
// contiguous range of tasks balanced by slice count, so a workgroup's loads
// run on from one task into the next without a ramp.
//
// Memory side.  Each wave keeps a ring of three LDS slots, one slice each
// (16 rows x 4 blocks: 3 KiB of indices, 2 KiB of codebook), filled by
// global_load_lds_dwordx4: five instructions of 1 KiB, in which the lanes of
// one row read that row's contiguous 192 (128) bytes, so every instruction
// touches a few whole cache lines.  Within a row the 16-byte pieces land
// rotated -- index blocks by (r >> 1) & 3 blocks, codebook pieces by r & 7
// pieces -- which makes the compute side's LDS reads conflict-free.  Slices
// i + 1 and i + 2 are in flight while slice i is computed.  The x slice
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
// Weights are rounded to bf16 (RNE), as the reference's bf16 path;
// accumulation is fp32.
#include <algorithm>
#include <vector>

#include "nb_device.h"
#include "nb_internal.h"

namespace nb {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;

constexpr int kSkWaves = 8;
constexpr int kSkThreads = 64 * kSkWaves;
constexpr int kSkRows = 16 * kSkWaves;         // rows of one task
constexpr int kSkSliceK = 512;                 // K of one slice (4 blocks)
constexpr int kSkMaxM = 16;
constexpr int kSkXRow = kSkSliceK * 2;         // LDS bytes of one staged x row
constexpr int kSkIdxBytes = 16 * 192;          // indices of one slot
constexpr int kSkSlot = kSkIdxBytes + 16 * 128;  // + codebooks
constexpr int kSkDepth = 3;                    // slots per wave
constexpr int kSkRing = kSkWaves * kSkDepth * kSkSlot;
constexpr int kSkLdsMax = 160 * 1024;
static_assert(kSkRing + 2 * kSkMaxM * kSkXRow <= kSkLdsMax, "LDS");
static_assert(kSkSlot == 5 * 1024, "five 1 KiB loads per slot");
// x buffers of a launch: three (x two slices ahead) when M rows of them fit
// beside the ring, else two (one slice ahead)
__host__ __device__ constexpr int skinny_xbufs(int M) {
    return kSkRing + 3 * M * kSkXRow <= kSkLdsMax ? 3 : 2;
}

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

// Waits until at most N vector-memory operations of this wave are
// outstanding (they complete in issue order).
template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
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

__device__ __forceinline__ void cursor_rows(const SkinnyArgs& a, Cursor& c, int wave) {
    c.row0 = (c.task - a.tasks.task_begin[c.p]) * kSkRows + wave * 16;
}

__device__ __forceinline__ void cursor_next(const SkinnyArgs& a, Cursor& c, int wave) {
    if (++c.s < c.ns) return;
    c.s = 0;
    ++c.task;
    if (c.p + 1 < a.tasks.nprob && c.task >= a.tasks.task_begin[c.p + 1]) {
        ++c.p;
        cursor_load(a, c);
    }
    cursor_rows(a, c, wave);
}

template <int NXB>
__global__ __launch_bounds__(kSkThreads) void gemv_skinny_kernel(SkinnyArgs a) {
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
        cursor_load(a, cc);
        cursor_rows(a, cc, wave);
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
            nitems += c.ns;
        }
    }

    // LDS: the waves' rings, then NXB x buffers of M rows
    const uint32_t base = lds_addr(smem);
    const uint32_t ring = base + wave * kSkDepth * kSkSlot;
    const unsigned char* ring_p = smem + wave * kSkDepth * kSkSlot;
    const int xbuf_bytes = M * kSkXRow;

    // Per-lane constants of the weight loads: load i < 3 (indices) puts
    // piece P = 64 i + lane of the slot at row P / 12, place P % 12, which
    // holds piece (place - 3 rot) mod 12 of the row, rot = (row >> 1) & 3;
    // load 3 + i (codebooks) puts P = 64 i + lane at row P / 8, place
    // P % 8, holding piece (place - row) & 7.
    int w_row[5], w_blk[5], w_off[5];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int P = 64 * i + lane;
        const int rr = P / 12, place = P % 12;
        const int piece = (place - 3 * ((rr >> 1) & 3) + 12) % 12;
        w_row[i] = rr;
        w_blk[i] = piece / 3;
        w_off[i] = (piece % 3) * 16;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int P = 64 * i + lane;
        const int rr = P >> 3, place = P & 7;
        const int piece = (place - rr) & 7;
        w_row[3 + i] = rr;
        w_blk[3 + i] = piece >> 1;
        w_off[3 + i] = (piece & 1) * 16;
    }
    // Row bases of the weight loads of the W cursor's task (recomputed when
    // the task changes): per load, the row's first index byte or codebook
    // byte plus the lane's offset inside a block.
    const unsigned char* wbase[5];
    int wtask = -1;
    auto w_rows = [&](const Cursor& c) {
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const int64_t row = min(c.row0 + w_row[i], c.N - 1);
            wbase[i] = i < 3 ? c.packed + row * c.bpr * 48 + w_off[i]
                             : reinterpret_cast<const unsigned char*>(c.cb) + row * c.bpr * 32 +
                                   w_off[i];
        }
        wtask = c.task;
    };
    auto issue_w = [&](const Cursor& c, int slot) {
        if (c.task != wtask) w_rows(c);
        const uint32_t dst = __builtin_amdgcn_readfirstlane(ring + slot * kSkSlot);
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const int blk = min(4 * c.s + w_blk[i], c.bpr - 1);
            dma16(dst + 1024 * i, wbase[i] + blk * (i < 3 ? 48 : 32));
        }
    };
    // x slice of item c into buffer `buf`: wave w loads activation rows
    // min(2w + j, M - 1), j = 0, 1 -- always two loads, so the wait counts
    // below are exact (a clamped row rewrites row M - 1 with the same bytes,
    // before anyone reads that buffer).  Lane l takes the 16 bytes of
    // column piece l ^ (m & 7), so piece p of row m sits at place
    // p ^ (m & 7): the 16 rows of one B-operand read fall in different
    // banks.  Columns past K repeat the last 8 (their weights are zero).
    auto issue_x = [&](const Cursor& c, int buf) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int m = min(2 * wave + j, M - 1);
            const int piece = lane ^ (m & 7);
            const int k = min(c.s * kSkSliceK + piece * 8, c.K - 8);
            dma16(__builtin_amdgcn_readfirstlane(base + kSkRing + buf * xbuf_bytes + m * kSkXRow),
                  c.x + (int64_t)m * c.K + k);
        }
    };

    // MFMA column r reads activation row min(r, M - 1)
    const int xm = r < M ? r : M - 1;
    // this lane's pieces of a slot (rotated places, see above)
    const int idx_off = r * 192 + ((q + (r >> 1)) & 3) * 48;
    const int cb_off0 = kSkIdxBytes + r * 128 + ((2 * q + r) & 7) * 16;
    const int cb_off1 = kSkIdxBytes + r * 128 + ((2 * q + 1 + r) & 7) * 16;
    const int x_off = xm * kSkXRow;
    const int x_swz = xm & 7;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    // A finished task's outputs wait in `pend` and are stored after the
    // next item's loads are issued.  acc lane (q, r) holds C[4q + v][r]:
    // y[r][row0 + 4q + v].
    f32x4_t pend = acc;
    int pend_p = 0, pend_row0 = 0, pend_n = 0;
    bool pending = false;
    auto store = [&]() {
        pending = false;
        if (r >= M) return;
        const prob_cptr P = problem(a, pend_p);
        const bool add = P->y_mode == NB_Y_ADD;
        void* y = P->y;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int n = pend_row0 + 4 * q + v;
            if (n >= pend_n) continue;
            const int64_t yi = (int64_t)r * pend_n + n;
            if (a.y_dtype == NB_BF16) {
                *as_global_mut(static_cast<bf16_bits*>(y) + yi) = f32_to_bf16_rne(pend[v]);
            } else if (add) {
                auto* yp = as_global_mut(static_cast<float*>(y) + yi);
                *yp = *yp + pend[v];
            } else {
                *as_global_mut(static_cast<float*>(y) + yi) = pend[v];
            }
        }
    };

    // ---- the pipeline -----------------------------------------------------
    // Loads complete in issue order.  With three x buffers the issue order
    // is X(0) W(0) X(1) W(1), then item i issues X(i + 2) W(i + 2) after its
    // barrier, and W(i), X(i) are in once at most the 7 loads of X(i + 1)
    // and W(i + 1) are outstanding.  With two, the order is X(0) W(0) W(1),
    // then item i issues X(i + 1) W(i + 2), and W(i), X(i) are in once at
    // most the 5 loads of W(i + 1) are.  Either way the weights are
    // requested two items ahead.  (Output stores, issued after an item's
    // loads, only make the next wait longer.)
    constexpr int kLead = NXB == 3 ? 2 : 1;  // items between X's issue and use
    constexpr int kAfter = NXB == 3 ? 7 : 5;
    Cursor cx = cc, cw = cc;
    issue_x(cx, 0);
    cursor_next(a, cx, wave);
    issue_w(cw, 0);
    cursor_next(a, cw, wave);
    if (nitems > 1) {
        if (NXB == 3) {
            issue_x(cx, 1);
            cursor_next(a, cx, wave);
        }
        issue_w(cw, 1);
        cursor_next(a, cw, wave);
    }

    for (int i = 0; i < nitems; ++i) {
        if (i + 1 < nitems) {
            wait_vm<kAfter>();
        } else {
            wait_vm<0>();
        }
        // every wave's x pieces of item i are in, and every wave is done
        // with item i - 1 (the buffers the next loads overwrite)
        wg_barrier();
        if (i + kLead < nitems) {
            issue_x(cx, (i + kLead) % NXB);
            cursor_next(a, cx, wave);
        }
        if (i + 2 < nitems) {
            issue_w(cw, (i + 2) % kSkDepth);
            cursor_next(a, cw, wave);
        }
        if (pending) store();
        // ---- compute slice cc.s of the task ----
        const unsigned char* slot = ring_p + (i % kSkDepth) * kSkSlot;
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
        const unsigned char* xb = smem + kSkRing + (i % NXB) * xbuf_bytes + x_off;
        mfma_groups<0>(d, lo0, lo1, hi0, hi1, xb, q * 16, x_swz, acc);
        if (cc.s == cc.ns - 1) {
            pend = acc;
            pend_p = cc.p;
            pend_row0 = cc.row0;
            pend_n = cc.N;
            pending = true;
            acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
        cursor_next(a, cc, wave);
    }
    if (pending) store();
}

}  // namespace

int launch_gemv_skinny(const StreamProblem* dev_probs, const StreamProblem* host_probs,
                       int nprob, int M, int y_dtype, hipStream_t stream) {
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
        // tasks and their slice counts, then contiguous task ranges of about
        // equal slice count, one per workgroup
        std::vector<int> slices;
        int64_t total_slices = 0;
        for (int i = 0; i < n; ++i) {
            A.tasks.task_begin[i] = (int32_t)slices.size();
            const StreamProblem& P = host_probs[p0 + i];
            const int nt = (P.N + kSkRows - 1) / kSkRows;
            const int ns = ((P.K >> 7) + 3) >> 2;
            for (int t = 0; t < nt; ++t) slices.push_back(ns);
            total_slices += (int64_t)nt * ns;
            if (slices.size() > (size_t)0x7fffffff) {
                return fail(NB_EUNSUPPORTED, "nb_gemm_skinny_batched: too many rows");
            }
        }
        const int ntask = (int)slices.size();
        if (ntask == 0) continue;
        const int G = std::min(cus, ntask);
        int t = 0;
        int64_t acc = 0;
        A.wg_task0[0] = 0;
        for (int g = 1; g <= G; ++g) {
            const int64_t goal = total_slices * g / G;
            // (a task goes to the workgroup that holds its midpoint)
            while (t < ntask && 2 * acc + slices[t] <= 2 * goal) acc += slices[t++];
            // every workgroup keeps at least one task while tasks remain
            if (t == A.wg_task0[g - 1] && t < ntask) acc += slices[t++];
            A.wg_task0[g] = g == G ? ntask : t;
        }
        const size_t lds = (size_t)kSkRing + (size_t)skinny_xbufs(M) * M * kSkXRow;
        if (skinny_xbufs(M) == 3) {
            hipLaunchKernelGGL(gemv_skinny_kernel<3>, dim3((unsigned)G), dim3(kSkThreads), lds,
                               stream, A);
        } else {
            hipLaunchKernelGGL(gemv_skinny_kernel<2>, dim3((unsigned)G), dim3(kSkThreads), lds,
                               stream, A);
        }
        const int st = check_launch("nb_gemm_skinny_batched");
        if (st) return st;
    }
    return NB_OK;
}

}  // namespace nb
