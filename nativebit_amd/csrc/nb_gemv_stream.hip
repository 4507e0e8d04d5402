// Persistent streaming GEMV over a batch of packed 3-bit layers (gfx950).
//
//   for every problem p:  y_p[n] = sum_k x_p[k] * bf16(W_p[n][k])   (M = 1)
//
// One launch streams the packed weights of all problems.  Every wave is an
// independent worker: the batch is cut into 16-row tiles (tile t of problem p
// = rows 16t..16t+15, all of K), numbered consecutively across problems, and
// each wave of the grid owns a contiguous tile range holding 1/W of all
// steps (a K=6912 tile costs 14 steps, a K=2560 tile 5).  A wave therefore
// never waits for another wave: there is no barrier and no cross-wave
// reduction (it accumulates full rows and writes them itself).
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
#include "nb_device.h"
#include "nb_internal.h"

namespace nb {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;

// waves per workgroup (independent workers)
#ifndef NB_STREAM_WAVES
#define NB_STREAM_WAVES 4
#endif
constexpr int kWaves = NB_STREAM_WAVES;

#ifndef NB_STREAM_WG_PER_CU
#define NB_STREAM_WG_PER_CU 2
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

struct Regs {
    uint32_t d[12];
    float c[8];
};

// Loads of one step of one lane (no waits).
__device__ __forceinline__ void load_regs(const uint8_t* __restrict__ packed,
                                          const float* __restrict__ cb, int64_t row,
                                          int bcol, int bpr, Regs& s) {
    const u32x4_t* p = reinterpret_cast<const u32x4_t*>(packed + (row * bpr + bcol) * 48);
#pragma unroll
    for (int v = 0; v < 3; ++v) {
        const u32x4_t u = stream_load(p + v);
        s.d[4 * v] = u.x;
        s.d[4 * v + 1] = u.y;
        s.d[4 * v + 2] = u.z;
        s.d[4 * v + 3] = u.w;
    }
    const f32x4_t* c = reinterpret_cast<const f32x4_t*>(cb + (row * bpr + bcol) * 8);
#pragma unroll
    for (int v = 0; v < 2; ++v) {
        const f32x4_t f = stream_load(c + v);
        s.c[4 * v] = f.x;
        s.c[4 * v + 1] = f.y;
        s.c[4 * v + 2] = f.z;
        s.c[4 * v + 3] = f.w;
    }
}

template <int J>
__device__ __forceinline__ void mfma_groups(const Regs& s, uint32_t lo0, uint32_t lo1,
                                            uint32_t hi0, uint32_t hi1,
                                            const u32x4_t (&bv)[16], f32x4_t& acc0,
                                            f32x4_t& acc1) {
    if constexpr (J < 16) {
        const u32x4_t a = lookup8(group24<J>(s.d), lo0, lo1, hi0, hi1);
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
        mfma_groups<J + 1>(s, lo0, lo1, hi0, hi1, bv, acc0, acc1);
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
    const uint32_t p0 = pack_bf16x2(s.c[0], s.c[1]);
    const uint32_t p1 = pack_bf16x2(s.c[2], s.c[3]);
    const uint32_t p2 = pack_bf16x2(s.c[4], s.c[5]);
    const uint32_t p3 = pack_bf16x2(s.c[6], s.c[7]);
    uint32_t lo0 = __builtin_amdgcn_perm(p1, p0, 0x06040200u);
    uint32_t hi0 = __builtin_amdgcn_perm(p1, p0, 0x07050301u);
    uint32_t lo1 = __builtin_amdgcn_perm(p3, p2, 0x06040200u);
    uint32_t hi1 = __builtin_amdgcn_perm(p3, p2, 0x07050301u);
    lo0 = live ? lo0 : 0u;
    hi0 = live ? hi0 : 0u;
    lo1 = live ? lo1 : 0u;
    hi1 = live ? hi1 : 0u;
    mfma_groups<0>(s, lo0, lo1, hi0, hi1, bv, acc0, acc1);
}

// The fields of one problem the step loop needs, held in registers (scalar,
// wave-uniform) and refreshed only when the cursor moves to another problem.
struct Prob {
    const uint8_t* packed;
    const float* codebook;
    const uint16_t* x;
    void* y;
    int N, K, bpr, nsteps, tiles;
};

__device__ __forceinline__ void fetch_prob(const StreamProblem* __restrict__ probs, int p,
                                           Prob& P) {
    const StreamProblem& s = probs[p];
    P.packed = s.packed;
    P.codebook = s.codebook;
    P.x = s.x;
    P.y = s.y;
    P.N = s.N;
    P.K = s.K;
    P.bpr = s.bpr;
    P.nsteps = s.nsteps;
    P.tiles = s.tiles;
}

// A position in a wave's stream of steps, with its problem's fields.
struct Cursor {
    int p;       // problem
    int tile;    // tile inside the problem
    int step;    // step inside the tile
    int left;    // steps left in this wave's range (incl. this one)
    Prob P;
};

__device__ __forceinline__ void advance(Cursor& c, const StreamProblem* __restrict__ probs) {
    --c.left;
    if (++c.step == c.P.nsteps) {
        c.step = 0;
        if (++c.tile == c.P.tiles) {
            c.tile = 0;
            ++c.p;
            if (c.left > 0) fetch_prob(probs, c.p, c.P);
        }
    }
}

// First tile (in batch order) whose first step is at or after global step s.
__device__ __forceinline__ int tile_at(const StreamProblem* __restrict__ probs, int nprob,
                                       int s) {
    int p = 0;
    while (p + 1 < nprob && probs[p + 1].step_begin <= s) ++p;
    const StreamProblem& P = probs[p];
    int t = (s - P.step_begin + P.nsteps - 1) / P.nsteps;
    if (t > P.tiles) t = P.tiles;
    return P.tile_begin + t;
}

__global__ __launch_bounds__(64 * kWaves) void gemv_stream_kernel(
    const StreamProblem* __restrict__ probs, int nprob, int total_steps, int x_slot,
    int y_dtype) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int r = lane & 15;
    const int q = lane >> 4;
    bf16_bits* xs = reinterpret_cast<bf16_bits*>(smem + (size_t)wave * x_slot);

    // This wave's tiles: a contiguous range holding about 1/nw of all steps
    // (tiles of different K cost different numbers of steps).  Tile i goes
    // to the wave whose step range contains the tile's first step.
    const int gw = blockIdx.x * kWaves + wave;
    const int nw = gridDim.x * kWaves;
    const int t0 = tile_at(probs, nprob, (int)(((int64_t)gw * total_steps) / nw));
    const int t1 = tile_at(probs, nprob, (int)(((int64_t)(gw + 1) * total_steps) / nw));
    if (t0 >= t1) return;

    // locate t0 (problem tables hold only problems with at least one tile)
    Cursor cc;
    cc.p = 0;
    while (cc.p + 1 < nprob && probs[cc.p + 1].tile_begin <= t0) ++cc.p;
    cc.tile = t0 - probs[cc.p].tile_begin;
    cc.step = 0;
    {
        int left = 0, p = cc.p, t = t0;
        while (t < t1) {
            const int end = probs[p].tile_begin + probs[p].tiles;
            const int n = (end < t1 ? end : t1) - t;
            left += n * probs[p].nsteps;
            t += n;
            ++p;
        }
        cc.left = left;
    }
    fetch_prob(probs, cc.p, cc.P);
    Cursor lc = cc;  // load cursor: runs up to two steps ahead of cc

    auto issue = [&](const Cursor& c, Regs& s) {
        const int row = c.tile * 16 + r;
        const int64_t lrow = row < c.P.N ? row : c.P.N - 1;
        const int b = c.step * 4 + q;
        const int bc = b < c.P.bpr ? b : c.P.bpr - 1;
        load_regs(c.P.packed, c.P.codebook, lrow, bc, c.P.bpr, s);
    };
    // The load cursor stops at the wave's last step (re-issuing it is a
    // harmless cache hit), so no load leaves the wave's range.
    auto issue_next = [&](Regs& s) {
        issue(lc, s);
        if (lc.left > 1) advance(lc, probs);
    };

    int xp = -1;  // problem whose x is in this wave's LDS slot
    f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};

    auto step = [&](const Regs& s) {
        const Prob& P = cc.P;
        if (cc.p != xp) {
            // stage x_p in this wave's LDS slot (wave-local: no barrier)
            const int chunks = P.K >> 3;
            const u32x4_t* src = reinterpret_cast<const u32x4_t*>(P.x);
            for (int i = lane; i < chunks; i += 64) {
                reinterpret_cast<u32x4_t*>(xs)[i] = *as_global(src + i);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            xp = cc.p;
        }
        const int row = cc.tile * 16 + r;
        const int b = cc.step * 4 + q;
        const bool live = row < P.N && b < P.bpr;
        const int bc = b < P.bpr ? b : P.bpr - 1;
        consume(s, live, reinterpret_cast<const u32x4_t*>(xs + bc * 128), acc0, acc1);
        if (cc.step == P.nsteps - 1) {
            // tile done: lanes (c = 0, g = q) hold rows 4q .. 4q+3 of column 0
            if (r == 0) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int orow = cc.tile * 16 + 4 * q + v;
                    if (orow < P.N) {
                        const float val = acc0[v] + acc1[v];
                        if (y_dtype == NB_BF16) {
                            *as_global_mut(static_cast<bf16_bits*>(P.y) + orow) = f32_to_bf16_rne(val);
                        } else {
                            *as_global_mut(static_cast<float*>(P.y) + orow) = val;
                        }
                    }
                }
            }
            acc0 = f32x4_t{0.f, 0.f, 0.f, 0.f};
            acc1 = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
        advance(cc, probs);
    };

    // Three-register ring, unrolled so the sets rotate without copies: the
    // loads of the two steps after the current one are in flight while it
    // is consumed.
    Regs ra, rb, rc;
    issue_next(ra);
    issue_next(rb);
    while (true) {
        issue_next(rc);
        step(ra);
        if (cc.left <= 0) break;
        issue_next(ra);
        step(rb);
        if (cc.left <= 0) break;
        issue_next(rb);
        step(rc);
        if (cc.left <= 0) break;
    }
}

}  // namespace

int launch_gemv_stream(const StreamProblem* dev_probs, int nprob, int total_steps,
                       int max_k, int y_dtype, hipStream_t stream) {
    if (nprob == 0 || total_steps == 0) return NB_OK;
    const int x_slot = ((max_k * 2 + 255) / 256) * 256;
    const size_t lds = (size_t)x_slot * kWaves;
    if (lds > (size_t)device_lds_bytes()) {
        return fail(NB_EUNSUPPORTED, "nb_gemv_batched: K=%d needs %zu bytes of LDS", max_k, lds);
    }
    const int cus = device_cu_count();
    int64_t grid = (int64_t)cus * NB_STREAM_WG_PER_CU;
    const int64_t need = (total_steps + kWaves - 1) / kWaves;
    if (grid > need) grid = need;
    hipLaunchKernelGGL(gemv_stream_kernel, dim3((int)grid), dim3(64 * kWaves), lds, stream,
                       dev_probs, nprob, total_steps, x_slot, y_dtype);
    return check_launch("nb_gemv_batched");
}

}  // namespace nb
