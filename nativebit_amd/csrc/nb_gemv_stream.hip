// Persistent streaming GEMV over a batch of packed 3-bit layers (gfx950).
//
//   for every problem p:  y_p[n] = sum_k x_p[k] * bf16(W_p[n][k])   (M = 1)
//
// One launch streams the packed weights of all problems.  The batch is cut
// into 16-row tiles (tile t of problem p = rows 16t..16t+15, all of K),
// numbered consecutively across problems.  Each workgroup owns a contiguous
// tile range holding 1/G of all steps (a K=6912 tile costs 14 steps, a
// K=2560 tile 5); inside it, its waves take tiles one at a time from a
// counter in LDS.  (Static per-wave ranges leave half of the kernel's time
// to one wave per SIMD: the arbiter favours the older of two waves, which
// finishes its share in about half the time of the other.)  A tile is
// computed by one wave from start to end -- full rows, no cross-wave
// reduction, no barrier after the counter is set up -- so results do not
// depend on which wave took which tile.
//
// Each tile is consumed in steps of 4 blocks (512 columns): lane l = q*16 + r
// loads row r's block 4*step + q (48 bytes of indices, 32 bytes of fp32
// codebook), turns its 128 weights into 16 bf16 MFMA A-operands with the
// register byte-plane lookup of nb_gemv_mfma.hip, and multiplies them by
// x (B operand, from the wave's own LDS copy of x_p) with
// v_mfma_f32_16x16x32_bf16.  The loads of the next two steps -- which may
// belong to the next tile or the next problem -- are in flight while the
// current step is consumed, so HBM requests stay in flight across tile
// boundaries.
//
// Weights are rounded to bf16 (RNE) as in the reference's bf16 path
// (inference/eval_ppl.py:149-174); accumulation is fp32.
#include <algorithm>
#include <utility>
#include <vector>

#include "nb_device.h"
#include "nb_internal.h"

namespace nb {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;

// waves per workgroup (two per SIMD)
#ifndef NB_STREAM_WAVES
#define NB_STREAM_WAVES 8
#endif
constexpr int kWaves = NB_STREAM_WAVES;

#ifndef NB_STREAM_WG_PER_CU
#define NB_STREAM_WG_PER_CU 1
#endif

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
    bf16x2_t v;
    v.x = (__bf16)lo;
    v.y = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
}

// 8 bf16 weights (natural order) of one 24-bit index group from the byte
// planes of the block's codebook.  Two selectors of four 3-bit indices (one
// per byte) are built in 9 VALU ops; v_perm_b32 on the low-byte and
// high-byte planes looks up four entries at once, and two more v_perm_b32
// interleave low and high bytes into bf16x2 pairs.
__device__ __forceinline__ u32x4_t lookup8(uint32_t g, uint32_t lo0, uint32_t lo1,
                                           uint32_t hi0, uint32_t hi1) {
    // h = indices 0-3 in the low half, 4-7 in the high half (bits 0,3,6,9):
    //   h  = bfi(0xffff, g, g << 4)
    //   sa = (h & 0x00070007) | ((h << 5) & 0x07000700)   bytes (i0,i1,i4,i5)
    //   sb = ((h >> 6) & 0x00070007) | ((h >> 1) & 0x07000700)   (i2,i3,i6,i7)
    // Written as one asm block (VALU only, no memory) because the compiler
    // otherwise rebuilds h in pieces and spends 11 ops instead of 9.
    // (VOP3 forms take no literal on gfx9: the masks come in as SGPRs.)
    uint32_t sa, sb, t0, t1;
    asm("v_lshlrev_b32 %2, 4, %4\n\t"
        "v_bfi_b32 %2, %5, %4, %2\n\t"
        "v_lshlrev_b32 %3, 5, %2\n\t"
        "v_and_b32 %0, %6, %2\n\t"
        "v_and_or_b32 %0, %3, %7, %0\n\t"
        "v_lshrrev_b32 %3, 1, %2\n\t"
        "v_lshrrev_b32 %2, 6, %2\n\t"
        "v_and_b32 %3, %7, %3\n\t"
        "v_and_or_b32 %1, %2, %6, %3"
        : "=&v"(sa), "=&v"(sb), "=&v"(t0), "=&v"(t1)
        : "v"(g), "s"(0xffffu), "s"(0x00070007u), "s"(0x07000700u));
    const uint32_t la = __builtin_amdgcn_perm(lo1, lo0, sa);
    const uint32_t ha = __builtin_amdgcn_perm(hi1, hi0, sa);
    const uint32_t lb = __builtin_amdgcn_perm(lo1, lo0, sb);
    const uint32_t hb = __builtin_amdgcn_perm(hi1, hi0, sb);
    u32x4_t w;
    w.x = __builtin_amdgcn_perm(ha, la, 0x05010400u);
    w.y = __builtin_amdgcn_perm(hb, lb, 0x05010400u);
    w.z = __builtin_amdgcn_perm(ha, la, 0x07030602u);
    w.w = __builtin_amdgcn_perm(hb, lb, 0x07030602u);
    return w;
}

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

// One lane's loads of one step: 48 bytes of indices, 32 bytes of codebook.
struct Regs {
    u32x4_t d0, d1, d2, c0, c1;
};

// The three register sets of the prefetch ring sit in fixed VGPRs
// (v[100:119], v[120:139], v[140:159]); their loads are issued with inline
// asm and waited for with an explicit s_waitcnt vmcnt.  Left to itself, the
// compiler moves a set that is still in flight into other registers in one
// of the three unrolled copies of the step, and a move of an in-flight
// register must first wait for it: that drains the ring every third step.
// With the sets pinned, nothing touches a set between its load and its wait.
// The loop issues no other vector-memory instruction, so the count is exact:
// when a set is consumed, it and the two sets issued after it -- 15 loads --
// are the only ones outstanding.
#define NB_RING_LOAD(R0, R1, R2, R3, R4)                                                      \
    __device__ __forceinline__ void load_set(const uint8_t* p, const float* c, Regs& s) {     \
        asm volatile("global_load_dwordx4 %0, %1, off" : "={v[" #R0 "]}"(s.d0) : "v"(p));          \
        asm volatile("global_load_dwordx4 %0, %1, off offset:16" : "={v[" #R1 "]}"(s.d1) : "v"(p)); \
        asm volatile("global_load_dwordx4 %0, %1, off offset:32" : "={v[" #R2 "]}"(s.d2) : "v"(p)); \
        asm volatile("global_load_dwordx4 %0, %1, off" : "={v[" #R3 "]}"(s.c0) : "v"(c));          \
        asm volatile("global_load_dwordx4 %0, %1, off offset:16" : "={v[" #R4 "]}"(s.c1) : "v"(c)); \
    }                                                                                          \
    __device__ __forceinline__ void wait_set(Regs& s) {                                        \
        asm volatile("s_waitcnt vmcnt(10)"                                                     \
                     : "+{v[" #R0 "]}"(s.d0), "+{v[" #R1 "]}"(s.d1), "+{v[" #R2 "]}"(s.d2),       \
                       "+{v[" #R3 "]}"(s.c0), "+{v[" #R4 "]}"(s.c1));                            \
    }

namespace set0 { NB_RING_LOAD(100:103, 104:107, 108:111, 112:115, 116:119) }
namespace set1 { NB_RING_LOAD(120:123, 124:127, 128:131, 132:135, 136:139) }
namespace set2 { NB_RING_LOAD(140:143, 144:147, 148:151, 152:155, 156:159) }
#undef NB_RING_LOAD

// Waits for every set (the loads issued past the wave's last step land
// before their registers are released).
__device__ __forceinline__ void wait_all(Regs& a, Regs& b, Regs& c) {
    asm volatile("s_waitcnt vmcnt(0)"
                 : "+{v[100:103]}"(a.d0), "+{v[104:107]}"(a.d1), "+{v[108:111]}"(a.d2),
                   "+{v[112:115]}"(a.c0), "+{v[116:119]}"(a.c1),
                   "+{v[120:123]}"(b.d0), "+{v[124:127]}"(b.d1), "+{v[128:131]}"(b.d2),
                   "+{v[132:135]}"(b.c0), "+{v[136:139]}"(b.c1),
                   "+{v[140:143]}"(c.d0), "+{v[144:147]}"(c.d1), "+{v[148:151]}"(c.d2),
                   "+{v[152:155]}"(c.c0), "+{v[156:159]}"(c.c1));
}

template <int J>
__device__ __forceinline__ void mfma_groups(const uint32_t (&d)[12], uint32_t lo0, uint32_t lo1,
                                            uint32_t hi0, uint32_t hi1,
                                            const u32x4_t (&bv)[16], f32x4_t& acc0,
                                            f32x4_t& acc1) {
    if constexpr (J < 16) {
        const u32x4_t a = lookup8(group24<J>(d), lo0, lo1, hi0, hi1);
        const u32x4_t b = bv[J];
        // two accumulators halve the dependent-MFMA chain
        if constexpr (J % 2 == 0) {
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                           __builtin_bit_cast(bf16x8_t, b),
                                                           acc0, 0, 0, 0);
        } else {
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                           __builtin_bit_cast(bf16x8_t, b),
                                                           acc1, 0, 0, 0);
        }
        mfma_groups<J + 1>(d, lo0, lo1, hi0, hi1, bv, acc0, acc1);
    }
}

__device__ __forceinline__ void consume(const Regs& s, bool live,
                                        const u32x4_t* __restrict__ bsrc, f32x4_t& acc0,
                                        f32x4_t& acc1) {
    // all 16 B operands (x at this lane's 128 columns) requested at once, so
    // their LDS latency overlaps the codebook planes and the first lookups
    u32x4_t bv[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) bv[j] = bsrc[j];
    // keep the scheduler from sinking the reads back next to their MFMAs
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t p0 = pack_bf16x2(__uint_as_float(s.c0.x), __uint_as_float(s.c0.y));
    const uint32_t p1 = pack_bf16x2(__uint_as_float(s.c0.z), __uint_as_float(s.c0.w));
    const uint32_t p2 = pack_bf16x2(__uint_as_float(s.c1.x), __uint_as_float(s.c1.y));
    const uint32_t p3 = pack_bf16x2(__uint_as_float(s.c1.z), __uint_as_float(s.c1.w));
    uint32_t lo0 = __builtin_amdgcn_perm(p1, p0, 0x06040200u);
    uint32_t hi0 = __builtin_amdgcn_perm(p1, p0, 0x07050301u);
    uint32_t lo1 = __builtin_amdgcn_perm(p3, p2, 0x06040200u);
    uint32_t hi1 = __builtin_amdgcn_perm(p3, p2, 0x07050301u);
    lo0 = live ? lo0 : 0u;
    hi0 = live ? hi0 : 0u;
    lo1 = live ? lo1 : 0u;
    hi1 = live ? hi1 : 0u;
    const uint32_t d[12] = {s.d0.x, s.d0.y, s.d0.z, s.d0.w, s.d1.x, s.d1.y,
                            s.d1.z, s.d1.w, s.d2.x, s.d2.y, s.d2.z, s.d2.w};
    mfma_groups<0>(d, lo0, lo1, hi0, hi1, bv, acc0, acc1);
}

// One problem of the workgroup's range as the step loop reads it, copied
// into LDS at set-up (64 bytes).
struct ProbL {
    const uint8_t* packed;
    const float* codebook;
    void* y;
    int32_t N, K, bpr, nsteps, tiles, tile_begin;
    int32_t x_off;  // byte offset of this problem's x in the LDS x region
    int32_t pad[3];
};
static_assert(sizeof(ProbL) == 64, "ProbL is 64 bytes");

// The same fields in scalar registers.
struct Prob {
    const uint8_t* packed;
    const float* codebook;
    int N, bpr, nsteps, tiles, tile_begin, x_off;
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
    P.N = __builtin_amdgcn_readfirstlane(s.N);
    P.bpr = __builtin_amdgcn_readfirstlane(s.bpr);
    P.nsteps = __builtin_amdgcn_readfirstlane(s.nsteps);
    P.tiles = __builtin_amdgcn_readfirstlane(s.tiles);
    P.tile_begin = __builtin_amdgcn_readfirstlane(s.tile_begin);
    P.x_off = __builtin_amdgcn_readfirstlane(s.x_off);
}

// Where one loaded register set belongs: problem (index in the workgroup's
// range), tile inside it, step inside the tile.  `valid` is false for loads
// issued after the wave ran out of tiles (they repeat the last address and
// are never consumed).
struct Meta {
    int li, tile, step;
    bool valid;
};

__global__ __launch_bounds__(64 * kWaves) void gemv_stream_kernel(
    const StreamProblem* __restrict__ probs, StreamRanges ranges, int y_dtype) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int r = lane & 15;
    const int q = lane >> 4;

    // ---- set-up: the workgroup's tiles, problems, x vectors and counter ----
    const int g = blockIdx.x;
    const int T0 = ranges.tile0[g];
    const int T1 = ranges.tile0[g + 1];
    const int p0 = ranges.prob0[g];
    const int np = ranges.prob1[g] - p0 + 1;
    ProbL* pl = reinterpret_cast<ProbL*>(smem);
    unsigned char* xregion = smem + np * (int)sizeof(ProbL);
    int x_bytes = 0;  // every thread sums the K of the range (few problems)
    for (int i = 0; i < np; ++i) x_bytes += probs[p0 + i].K * 2;
    float* ybuf = reinterpret_cast<float*>(xregion + x_bytes);
    int* next_tile = reinterpret_cast<int*>(ybuf + (T1 - T0) * 16);
    if (tid < np) {
        const StreamProblem& s = probs[p0 + tid];
        ProbL d;
        d.packed = s.packed;
        d.codebook = s.codebook;
        d.y = s.y;
        d.N = s.N;
        d.K = s.K;
        d.bpr = s.bpr;
        d.nsteps = s.nsteps;
        d.tiles = s.tiles;
        d.tile_begin = s.tile_begin;
        int off = 0;
        for (int i = 0; i < tid; ++i) off += probs[p0 + i].K * 2;
        d.x_off = off;
        d.pad[0] = d.pad[1] = d.pad[2] = 0;
        pl[tid] = d;
    }
    {
        int off = 0;
        for (int i = 0; i < np; ++i) {
            const int K = probs[p0 + i].K;
            const u32x4_t* src = reinterpret_cast<const u32x4_t*>(probs[p0 + i].x);
            u32x4_t* dst = reinterpret_cast<u32x4_t*>(xregion + off);
            for (int c = tid; c < K / 8; c += 64 * kWaves) dst[c] = *as_global(src + c);
            off += K * 2;
        }
    }
    if (tid == 0) *next_tile = T0;
    __syncthreads();

    // ---- steady state: waves take tiles from the counter until none is left
    auto grab = [&]() -> int {
        int t = 0;
        if (lane == 0) t = atomicAdd(next_tile, 1);
        return __builtin_amdgcn_readfirstlane(t);
    };

    int t_first = grab();
    if (t_first < T1) {
        // load cursor (runs two steps ahead of consumption)
        int li = 0;
        Prob LP;
        read_prob(pl, 0, LP);
        while (t_first >= LP.tile_begin + LP.tiles) read_prob(pl, ++li, LP);
        int ltile = t_first - LP.tile_begin, lstep = 0;
        bool lvalid = true;

        // Loads the step at the load cursor into s (always: after the last
        // tile the cursor stays put and the load is a repeat), records where
        // it belongs and moves the cursor on, taking a new tile when one ends.
        auto issue = [&](auto load, Regs& s, Meta& m) {
            const int row = ltile * 16 + r;
            const int64_t lrow = row < LP.N ? row : LP.N - 1;
            const int b = lstep * 4 + q;
            const int bc = b < LP.bpr ? b : LP.bpr - 1;
            const int64_t blk = lrow * LP.bpr + bc;
            load(LP.packed + blk * 48, LP.codebook + blk * 8, s);
            m.li = li;
            m.tile = ltile;
            m.step = lstep;
            m.valid = lvalid;
            if (!lvalid) return;
            if (++lstep == LP.nsteps) {
                const int t = grab();
                if (t >= T1) {
                    lvalid = false;
                    lstep = LP.nsteps - 1;  // repeat the last step's address
                } else {
                    lstep = 0;
                    while (t >= LP.tile_begin + LP.tiles) read_prob(pl, ++li, LP);
                    ltile = t - LP.tile_begin;
                }
            }
        };

        int ci = -1;  // problem whose fields are in CP
        Prob CP = {};
        f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};

        auto step = [&](const Regs& s, const Meta& m) {
            if (m.li != ci) {
                read_prob(pl, m.li, CP);
                ci = m.li;
            }
            const int row = m.tile * 16 + r;
            const int b = m.step * 4 + q;
            const bool live = row < CP.N && b < CP.bpr;
            const int bc = b < CP.bpr ? b : CP.bpr - 1;
            const u32x4_t* xb = reinterpret_cast<const u32x4_t*>(xregion + CP.x_off) + bc * 16;
            consume(s, live, xb, acc0, acc1);
            if (m.step == CP.nsteps - 1) {
                // tile done: lanes (c = 0, g = q) hold rows 4q .. 4q+3 of
                // column 0; they go to the LDS output buffer (a global store
                // here would lock its data registers until it completes, in
                // order behind the weight loads in flight)
                if (r == 0) {
                    f32x4_t v;
                    v.x = acc0.x + acc1.x;
                    v.y = acc0.y + acc1.y;
                    v.z = acc0.z + acc1.z;
                    v.w = acc0.w + acc1.w;
                    const int slot = CP.tile_begin + m.tile - T0;
                    *reinterpret_cast<f32x4_t*>(ybuf + slot * 16 + 4 * q) = v;
                }
                acc0 = f32x4_t{0.f, 0.f, 0.f, 0.f};
                acc1 = f32x4_t{0.f, 0.f, 0.f, 0.f};
            }
        };

        // Three-register ring, unrolled so the sets rotate without copies:
        // the loads of the two steps after the current one are in flight
        // while it is consumed.  Validity is monotonic, so the first invalid
        // set ends the wave's work.
        Regs ra = {}, rb = {}, rc = {};
        // (initialised: an undefined wave-uniform value is materialised with
        // a v_readfirstlane of an arbitrary VGPR, which can be a load in
        // flight)
        Meta ma = {0, 0, 0, false}, mb = {0, 0, 0, false}, mc = {0, 0, 0, false};
        const auto la = [](const uint8_t* p, const float* c, Regs& s) { set0::load_set(p, c, s); };
        const auto lb = [](const uint8_t* p, const float* c, Regs& s) { set1::load_set(p, c, s); };
        const auto lc = [](const uint8_t* p, const float* c, Regs& s) { set2::load_set(p, c, s); };
        issue(la, ra, ma);
        issue(lb, rb, mb);
        while (true) {
            issue(lc, rc, mc);
            if (!ma.valid) break;
            set0::wait_set(ra);
            step(ra, ma);
            issue(la, ra, ma);
            if (!mb.valid) break;
            set1::wait_set(rb);
            step(rb, mb);
            issue(lb, rb, mb);
            if (!mc.valid) break;
            set2::wait_set(rc);
            step(rc, mc);
        }
        wait_all(ra, rb, rc);
    }

    // ---- write the range's outputs (coalesced, after every wave is done) --
    __syncthreads();
    int li = 0;
    for (int e = tid; e < (T1 - T0) * 16; e += 64 * kWaves) {
        const int t = T0 + (e >> 4);
        while (t >= pl[li].tile_begin + pl[li].tiles) ++li;
        const ProbL& P = pl[li];
        const int row = (t - P.tile_begin) * 16 + (e & 15);
        if (row < P.N) {
            const float val = ybuf[e];
            if (y_dtype == NB_BF16) {
                *as_global_mut(static_cast<bf16_bits*>(P.y) + row) = f32_to_bf16_rne(val);
            } else {
                *as_global_mut(static_cast<float*>(P.y) + row) = val;
            }
        }
    }
}

}  // namespace

// LDS bytes the kernel uses for a range of tiles [a, b) over problems
// [pa, pb] (same layout as the kernel's set-up).
static int64_t range_lds(const StreamProblem* hp, int pa, int pb, int a, int b) {
    int64_t n = (int64_t)(pb - pa + 1) * (int64_t)sizeof(ProbL);
    for (int p = pa; p <= pb; ++p) n += (int64_t)hp[p].K * 2;
    return n + (int64_t)(b - a) * 16 * 4 + 16;
}

// Problem holding tile t (host copy of the table; binary search).
static int prob_of_tile(const StreamProblem* hp, int nprob, int t) {
    int lo = 0, hi = nprob - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (hp[mid].tile_begin <= t) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// First tile whose first step is at or after global step s.
static int tile_at_step(const StreamProblem* hp, int nprob, int64_t s) {
    int lo = 0, hi = nprob - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (hp[mid].step_begin <= s) lo = mid; else hi = mid - 1;
    }
    const StreamProblem& P = hp[lo];
    int64_t t = (s - P.step_begin + P.nsteps - 1) / P.nsteps;
    if (t > P.tiles) t = P.tiles;
    return P.tile_begin + (int)t;
}

int launch_gemv_stream(const StreamProblem* dev_probs, const StreamProblem* host_probs,
                       int nprob, int y_dtype, hipStream_t stream) {
    if (nprob == 0) return NB_OK;
    const StreamProblem& last = host_probs[nprob - 1];
    const int total_tiles = last.tile_begin + last.tiles;
    const int64_t total_steps = (int64_t)last.step_begin + (int64_t)last.tiles * last.nsteps;
    if (total_tiles == 0) return NB_OK;
    const int64_t lds_max = device_lds_bytes();

    // Ranges balanced by steps, one per workgroup; a range whose problems,
    // x vectors and outputs do not fit in LDS is halved (by steps) until
    // they do.
    const int64_t G = std::min<int64_t>((int64_t)device_cu_count() * NB_STREAM_WG_PER_CU,
                                        total_tiles);
    std::vector<int> bounds;
    bounds.reserve((size_t)G + 1);
    for (int64_t g = 0; g <= G; ++g) bounds.push_back(tile_at_step(host_probs, nprob, g * total_steps / G));
    std::vector<int> out;
    out.push_back(bounds[0]);
    for (int64_t g = 0; g < G; ++g) {
        // split [bounds[g], bounds[g+1]) as needed (explicit stack)
        std::vector<std::pair<int, int>> todo{{bounds[(size_t)g], bounds[(size_t)g + 1]}};
        while (!todo.empty()) {
            auto [a, b] = todo.back();
            todo.pop_back();
            if (a >= b) continue;
            const int pa = prob_of_tile(host_probs, nprob, a);
            const int pb = prob_of_tile(host_probs, nprob, b - 1);
            if (range_lds(host_probs, pa, pb, a, b) <= lds_max) {
                out.push_back(b);
                continue;
            }
            if (b - a == 1) {
                return fail(NB_EUNSUPPORTED, "nb_gemv_batched: one tile needs more LDS than %lld bytes",
                            (long long)lds_max);
            }
            const int mid = a + (b - a) / 2;
            todo.push_back({mid, b});  // popped second
            todo.push_back({a, mid});
        }
    }
    // launch in chunks of at most kStreamMaxGroups workgroups
    const int nranges = (int)out.size() - 1;
    for (int c0 = 0; c0 < nranges; c0 += kStreamMaxGroups) {
        const int n = std::min(kStreamMaxGroups, nranges - c0);
        StreamRanges R;
        int64_t lds = 0;
        for (int i = 0; i <= n; ++i) R.tile0[i] = out[(size_t)(c0 + i)];
        for (int i = 0; i < n; ++i) {
            R.prob0[i] = prob_of_tile(host_probs, nprob, R.tile0[i]);
            R.prob1[i] = prob_of_tile(host_probs, nprob, R.tile0[i + 1] - 1);
            lds = std::max(lds, range_lds(host_probs, R.prob0[i], R.prob1[i], R.tile0[i], R.tile0[i + 1]));
        }
        hipLaunchKernelGGL(gemv_stream_kernel, dim3(n), dim3(64 * kWaves), (size_t)lds, stream,
                           dev_probs, R, y_dtype);
        const int st = check_launch("nb_gemv_batched");
        if (st) return st;
    }
    return NB_OK;
}

}  // namespace nb
