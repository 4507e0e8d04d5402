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
// Compute side (nb_stream_common.h).  Lane l takes block l of the chunk
// and forms its private dot product with the staged activations.
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
#include "nb_stream_common.h"

namespace nb {
namespace {

using namespace stream;

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
// One problem of the workgroup's range as the set-up, the activation
// staging, the chunk loop and the output phase read it, copied into LDS at
// set-up (96 bytes): after the set-up no phase reads the device table.
struct ProbL {
    const uint8_t* packed;
    const float* codebook;
    void* y;
    const void* x;          // activations in the form x_mode names
    const float* norm_w;    // NB_X_RMSNORM weights
    int32_t nblocks, bpr, nchunks, chunk_begin;
    int32_t x_off;      // byte offset of this problem's x (permuted) in LDS
    int32_t y_off;      // float offset of its row sums (rows row_a..row_b-1)
    int32_t row_a;      // first row of this problem in the range
    int32_t row_b;      // one past the last row
    int32_t carry_off;  // float offset of its carries (chunks ca..)
    int32_t ca;         // first chunk of this problem in the range
    int32_t x_mode, y_mode;
    float eps;
    int32_t pad;
};
static_assert(sizeof(ProbL) == 96, "ProbL is 96 bytes");

// The fields the loop needs, in scalar registers.
struct Prob {
    const uint8_t* packed;
    const float* codebook;
    int nblocks, bpr, chunk_begin, chunk_end, x_off, y_off, row_a, carry_off, ca;
    float inv_bpr;
};

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

__device__ __forceinline__ float wave_sum(float v) { return wave64_sum(v); }

// Halfword position, inside a column block's staged activations, of
// element e (0..7) of 8-element group g (0..15) of the block: the group's
// unit u = g / 4 and quarter q = g % 4, element e = index offset o of
// selector s with sel_offset(s) = e; selector s sits in 16-byte unit
// 4u + s / 2, halves (s & 1) * 4 + q (stage_unit's layout).
__device__ __forceinline__ int staged_half(int g, int e) {
    const int s = e == 0 ? 0 : e == 1 ? 1 : e == 2 ? 6 : e == 3 ? 2 : e == 4 ? 3 : e == 5 ? 7
                : e == 6 ? 4 : 5;
    return (4 * (g >> 2) + (s >> 1)) * 8 + (s & 1) * 4 + (g & 3);
}

// The K activations of problem s in the form its x_mode names, rounded to
// bf16 (nearest even) and written in selector order to the column blocks
// at `col0` (kXColBytes each).  Every thread of the workgroup calls it.
//   NB_X_BF16      a = x                      (K bf16)
//   NB_X_RMSNORM   a = (x / sqrt(mean(x^2) + eps)) * w   (K fp32; the
//                  expression of RMSNorm.forward, generate_torch.py:29-38)
//   NB_X_SILU_MUL  a = silu(gate) * up, gate | up = x   (2K fp32;
//                  generate_torch.py:116-117)
// The fp32 forms spread 8-element groups over all threads with every load
// issued up front, so a launch pays one memory round trip for them (plus
// two workgroup barriers for the norm's sum of squares).  exp(-g) in silu
// is v_exp_f32 of -g * log2(e) (__expf; a few ulp in fp32, below the bf16
// rounding that follows).
__device__ __forceinline__ void stage_problem(const ProbL* sp, unsigned char* col0,
                                              float* red, int tid) {
    constexpr int NT = 64 * kWaves;
    constexpr int kMaxG = (8192 / 8 + NT - 1) / NT;  // groups per thread (K <= 8192)
    const int K = sp->bpr * 128, mode = sp->x_mode;
    if (mode == NB_X_BF16) {
        for (int q = tid; q < (K >> 5); q += NT) {
            const int c = q >> 2, u = q & 3;
            const u32x4_t* src = reinterpret_cast<const u32x4_t*>(
                static_cast<const uint16_t*>(sp->x) + c * 128 + u * 32);
            uint32_t w[16];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const u32x4_t t = *as_global(src + v);
                w[4 * v] = t.x;
                w[4 * v + 1] = t.y;
                w[4 * v + 2] = t.z;
                w[4 * v + 3] = t.w;
            }
            stage_unit(col0 + c * kXColBytes, u, w);
        }
        return;
    }
    const int ng = K >> 3;
    const float* xf = static_cast<const float*>(sp->x);
    // second operand: the norm weights, or the up half of gate | up
    const float* bf = mode == NB_X_RMSNORM ? sp->norm_w : xf + K;
    f32x4_t a[kMaxG][2], b[kMaxG][2];
#pragma unroll
    for (int j = 0; j < kMaxG; ++j) {
        const int g = tid + j * NT;
        if (g < ng) {
            const f32x4_t* xa = reinterpret_cast<const f32x4_t*>(xf + 8 * g);
            const f32x4_t* xb = reinterpret_cast<const f32x4_t*>(bf + 8 * g);
            a[j][0] = *as_global(xa);
            a[j][1] = *as_global(xa + 1);
            b[j][0] = *as_global(xb);
            b[j][1] = *as_global(xb + 1);
        }
    }
    float norm = 1.f;
    if (mode == NB_X_RMSNORM) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < kMaxG; ++j) {
            if (tid + j * NT < ng) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) ss += a[j][h][e] * a[j][h][e];
                }
            }
        }
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        float t = 0.f;
        for (int w = 0; w < kWaves; ++w) t += red[w];  // same order in every thread
        __syncthreads();  // red is free for the next problem
        norm = sqrtf(t / (float)K + sp->eps);
    }
    uint16_t* out = reinterpret_cast<uint16_t*>(col0);
#pragma unroll
    for (int j = 0; j < kMaxG; ++j) {
        const int g = tid + j * NT;
        if (g < ng) {
            uint16_t* col = out + (g >> 4) * (kXColBytes / 2);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float xv = a[j][e >> 2][e & 3], bv = b[j][e >> 2][e & 3];
                const float r = mode == NB_X_RMSNORM ? (xv / norm) * bv
                                                     : (xv / (1.0f + __expf(-xv))) * bv;
                col[staged_half(g & 15, e)] = f32_to_bf16_rne(r);
            }
        }
    }
}

// kSel: every problem's index stream is in the selector-ordered unit layout
// (nb_stream_layout); the products are the same.
template <bool kSel>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(kWaves / 4, kWaves / 4)))
void gemv_stream_kernel(
    const StreamProblem* __restrict__ probs, StreamRanges ranges, int y_dtype) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    // ---- set-up: the workgroup's chunks, problems and counter -------------
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
            d.x = s.x;
            d.norm_w = s.norm_w;
            d.x_mode = s.x_mode;
            d.y_mode = s.y_mode;
            d.eps = s.eps;
            pl[i] = d;
        }
        x_bytes += s.bpr * kXColBytes;
        y_floats += (rb - ra) + (cb - ca);
    }
    float* ybuf = reinterpret_cast<float*>(xregion + x_bytes);
    int* next_chunk = reinterpret_cast<int*>(ybuf + y_floats);
    float* red = reinterpret_cast<float*>(next_chunk + 4);  // kWaves floats
    for (int e = tid; e < y_floats; e += 64 * kWaves) ybuf[e] = 0.f;
    if (tid == 0) *next_chunk = C0;
    __syncthreads();

    // ---- ring state: waves take chunks from the counter until none is left
    auto grab = [&]() -> int {
        int t = 0;
        if (lane == 0) t = atomicAdd(next_chunk, 1);
        return __builtin_amdgcn_readfirstlane(t);
    };
    unsigned char* my_ring = ring + wave * kDepth * kSlotBytes;
    const uint32_t my_ring_lds = lds_addr(my_ring);

    // load cursor (runs kDepth chunks ahead of computation)
    int li = 0;
    Prob LP = {};
    int lchunk = 0;
    bool lvalid = false;

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

    // The first kDepth chunks of each wave are requested before the
    // activations are formed: the weights do not depend on them, so the
    // two memory latencies overlap (a small launch pays one, not two).
    Meta ma = {0, 0, false}, mb = {0, 0, false}, mc = {0, 0, false};
    auto start = [&]() {
        const int c_first = grab();
        if (c_first < C1) {
            read_prob(pl, 0, LP);
            while (c_first >= LP.chunk_end) read_prob(pl, ++li, LP);
            lchunk = c_first;
            lvalid = true;
            issue(0, ma, grab());
            issue(1, mb, lvalid ? grab() : C1);
            if constexpr (kDepth == 3) issue(2, mc, lvalid ? grab() : C1);
        }
    };
    start();

    // ---- activations of the range's problems, staged in LDS ---------------
    // (16-byte unit j = 4u + m of column block c, at c * kXColBytes + j * 16,
    // holds the activations of selectors 2m and 2m+1 of unit u)
    {
        for (int i = 0; i < np; ++i) stage_problem(pl + i, xregion + pl[i].x_off, red, tid);
    }
    __syncthreads();

    // ---- steady state -------------------------------------------------------
    // A wait the compiler sees: its scoreboard otherwise still counts the
    // staging loads above as pending (their registers are reused in the
    // loop), and it would wait for every vector-memory operation -- the
    // ring's loads too -- at that reuse in every step.
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0), expcnt and lgkmcnt not waited
    if (ma.valid) {
        int ci = -1;  // problem whose fields are in CP
        Prob CP = {};

        // Per-chunk lane state computed before the chunk's bytes arrive.
        struct Lane {
            int row;
            int col;  // the block's column block in its row
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
            L.col = rem;
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
            // a block that is not live computes garbage on its own diagonal only
            const f32x4_t a = block_dot<kSel>(r.d0, r.d1, r.d2, r.c0, r.c1, xv);
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
                // chunk's carry slot: its first block is lane - col < 0 of
                // this chunk (the chunk starts at block lc * 64)
                const int cbase = __builtin_amdgcn_readfirstlane(CP.carry_off + m.lc - CP.ca);
                const int ybase = __builtin_amdgcn_readfirstlane(CP.y_off - CP.row_a);
                const int slot = L.col > lane ? cbase : ybase + L.row;
                atomicAdd(ybuf + slot, quad_row ? s4 : dot);
            }
        };

        // Ring of kDepth slots, unrolled so each slot index is a constant.
        // One step: take the next chunk number from the counter and request
        // this chunk's activations (both LDS, in flight while the wave waits
        // for the chunk), read the slot into registers, refill it with the
        // chunk kDepth ahead, and compute -- kDepth chunks are in flight
        // during the arithmetic.  Validity is monotonic: the first invalid
        // slot ends the wave's work.  From here on the wave issues no other
        // vector-memory instruction (the staging loads above have all been
        // consumed), so the vmcnt waits count ring loads exactly (each valid
        // slot holds kLoadsPerChunk loads).
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
        if constexpr (kDepth == 2) {
            while (true) {
                if (!ma.valid) break;
                step(0, ma, mb.valid ? 1 : 0);
                if (!mb.valid) break;
                step(1, mb, ma.valid ? 1 : 0);
            }
        } else {
            while (true) {
                if (!ma.valid) break;
                step(0, ma, (int)mb.valid + (int)mc.valid);
                if (!mb.valid) break;
                step(1, mb, (int)mc.valid + (int)ma.valid);
                if (!mc.valid) break;
                step(2, mc, (int)ma.valid + (int)mb.valid);
            }
        }
    }
    wait_vm<0>();  // (nothing is in flight here; kept as a guard)

    // ---- write the range's outputs (coalesced, after every wave is done) --
    __syncthreads();
    for (int i = 0; i < np; ++i) {
        const ProbL& P = pl[i];
        const bool add = P.y_mode == NB_Y_ADD;
        for (int e = tid; e < P.row_b - P.row_a; e += 64 * kWaves) {
            const int row = P.row_a + e;
            float val = ybuf[P.y_off + e];
            // the row's tail, if its last block lies in a later chunk
            const int c_first = (row * P.bpr) / kChunkBlocks;
            const int c_last = (row * P.bpr + P.bpr - 1) / kChunkBlocks;
            if (c_last != c_first) val += ybuf[P.carry_off + c_last - P.ca];
            if (y_dtype == NB_BF16) {
                *as_global_mut(static_cast<bf16_bits*>(P.y) + row) = f32_to_bf16_rne(val);
            } else if (add) {
                // residual add: the row belongs to this workgroup alone
                auto* yp = as_global_mut(static_cast<float*>(P.y) + row);
                *yp = *yp + val;
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
    return n + 16 + 64;  // chunk counter, then the norm's partial sums
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

namespace {

// nb_stream_layout: one thread per 12-byte unit; the unit's eight selectors
// (unit_selectors) packed back as the selector-ordered unit (sel_unit_pack).
// A thread reads its unit before writing it, so in == out is allowed.
__global__ __launch_bounds__(256) void stream_layout_kernel(const uint32_t* in, uint32_t* out,
                                                            int64_t units) {
    for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < units;
         u += (int64_t)gridDim.x * blockDim.x) {
        const uint32_t d0 = in[3 * u], d1 = in[3 * u + 1], d2 = in[3 * u + 2];
        uint32_t sel[8];
        unit_selectors(d0, d1, d2, sel);
        uint32_t e0, e1, e2;
        sel_unit_pack(sel, e0, e1, e2);
        out[3 * u] = e0;
        out[3 * u + 1] = e1;
        out[3 * u + 2] = e2;
    }
}

}  // namespace

int launch_stream_layout(const uint8_t* in, uint8_t* out, int64_t units, hipStream_t stream) {
    if (units == 0) return NB_OK;
    const int64_t grid = std::min<int64_t>((units + 255) / 256, (int64_t)device_cu_count() * 8);
    hipLaunchKernelGGL(stream_layout_kernel, dim3((int)grid), dim3(256), 0, stream,
                       reinterpret_cast<const uint32_t*>(in), reinterpret_cast<uint32_t*>(out),
                       units);
    return check_launch("nb_stream_layout");
}

int launch_gemv_stream(const StreamProblem* dev_probs, const StreamProblem* host_probs,
                       int nprob, int y_dtype, bool sel, hipStream_t stream) {
    if (nprob == 0) return NB_OK;
    // a single problem (a decode step's launch) takes the whole-row kernel
    if (nprob == 1 && gemv_rows_fits(host_probs[0])) {
        return launch_gemv_rows(host_probs[0], y_dtype, sel, stream);
    }
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
        if (sel) {
            hipLaunchKernelGGL(gemv_stream_kernel<true>, dim3(n), dim3(64 * kWaves), (size_t)lds,
                               stream, dev_probs, R, y_dtype);
        } else {
            hipLaunchKernelGGL(gemv_stream_kernel<false>, dim3(n), dim3(64 * kWaves), (size_t)lds,
                               stream, dev_probs, R, y_dtype);
        }
        const int st = check_launch("nb_gemv_batched");
        if (st) return st;
    }
    return NB_OK;
}

}  // namespace nb
