// Batched packed skinny GEMM for M <= 4 activation rows on the row-quad
// layout (gfx950).
//
//   for every problem p:  y_p[m][n] = sum_k x_p[m][k] * bf16(W_p[n][k]),  m < M <= 4
//
// The batched branch of PackedLinear.forward (inference/triton_kernel.py:
// 258-275) in its bf16 form (inference/eval_ppl.py:149-174), for the two to
// four token rows of a small-batch decode step.
//
// Row-quad layout.  The weights are the same 128-weight blocks (48 bytes of
// 3-bit indices, 8 fp32 codebook entries) in another order: rows are taken
// four at a time (N rounded up to a multiple of 4 with zero blocks), and a
// quad's blocks are stored column by column, the four rows' blocks of one
// column block kb side by side:
//     block 4 (q * bpr + kb) + i  =  row 4q + i, column block kb.
// nb_quad_layout writes it from the reference layout (one pass, HBM-bound).
//
// Why: v_mfma_f32_4x4x4_16b_bf16 computes, in each group of four lanes,
// D[i][j] = sum_k A_i[k] B_j[k] with lane 4g+i supplying A row i and lane
// 4g+j supplying B column j.  The M = 1 kernel (nb_gemv_stream.hip) gives
// each lane its own block and keeps only the diagonal.  Here the four lanes
// of a group hold the four rows of a quad at one column block (one 64-block
// chunk of the layout = 16 such groups, read by the same contiguous 1 KiB
// direct-to-LDS loads), and lane 4g+j supplies token j's activations of that
// column block: every entry of D is used, so up to four tokens cost what
// one does -- the same dequantization and MFMAs per weight as M = 1
// (nb_stream_common.h, block_dot).
//
// Work split.  The problems' quads form one sequence; each workgroup takes
// a contiguous run balanced by blocks (host), and each wave a contiguous
// run of whole quads of its workgroup's run, again balanced by blocks
// (device).  A wave streams the chunks that hold its quads through a ring
// of two LDS slots (five 1 KiB loads each, as M = 1), so no other wave
// touches its rows: a quad's 4 x M results are summed over the quad's
// chunks inside one wave, in a fixed order, and stored by that wave.
// (Units of a few quads handed out from an LDS counter, which keep a
// workgroup's waves on neighbouring bytes, measured about 5 % slower.)
//
// Row sums.  Group g of chunk c holds pair 16c + g = q * bpr + kb.  Each
// lane keeps one accumulator for the quad of its latest pair; with
// bpr >= 16 a lane's pair moves to the next quad at most once a chunk, in
// the chunk where the previous quad ends.  In that chunk the quad's sums
// are the lanes still in it (with this chunk's products) plus the lanes
// already past it (their accumulators from earlier chunks), summed over
// the 16 groups in a fixed tree, and stored one step later (after the next
// ring wait, so the stores do not sit between a slot's loads and its wait).
//
// Weights are rounded to bf16 (RNE), as the reference's bf16 path;
// accumulation is fp32.
#include <algorithm>
#include <vector>

#include "nb_device.h"
#include "nb_internal.h"
#include "nb_stream_common.h"

namespace nb {
namespace {

using namespace stream;

constexpr int kQChunkBlocks = 64;
constexpr int kQChunkIdx = kQChunkBlocks * 48;   // 3 KiB
constexpr int kQChunkCb = kQChunkBlocks * 32;    // 2 KiB
constexpr int kQSlot = kQChunkIdx + kQChunkCb;
constexpr int kQDepth = 2;
constexpr int kQLoads = 5;
constexpr int kQMaxM = 4;
constexpr int kQMinBpr = 16;                     // at most two quads per chunk
constexpr int kQMaxProbs = 256;                  // problems per launch (kernel-argument size)

struct QuadArgs {
    const StreamProblem* probs;                    // table (packed/codebook: quad layout)
    int32_t wg_q0[kStreamMaxGroups + 1];           // global quad run of workgroup g
    int32_t wg_p0[kStreamMaxGroups];               // problem holding quad wg_q0[g]
    int32_t quad_begin[kQMaxProbs + 1];            // first global quad of problem p
    int nprob, M, y_dtype;
};

// The fields of one problem a wave needs, in scalar registers.
struct QProb {
    const uint8_t* packed;
    const float* codebook;
    void* y;
    int N, bpr, nblocks, x_off, y_mode;
};

// Sum of v over the 16 lane groups of a wave with the same lane & 3; the
// total lands in lanes 0..3 (the other lanes hold partial sums).
__device__ __forceinline__ float group_sum(float v) {
    // rotate within each row of 16 lanes by 4 and 8 lanes: the row's four
    // groups, then across the four rows
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xf, 0xf, false));
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

template <int W>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(W / 4, W / 4)))
void gemv_quad_kernel(QuadArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = blockIdx.x;
    const int GQ0 = a.wg_q0[g], GQ1 = a.wg_q0[g + 1];
    const int pA = a.wg_p0[g];
    const int M = a.M;
    // the workgroup's problems pA .. pB
    int pB = pA;
    while (pB + 1 < a.nprob && a.quad_begin[pB + 1] < GQ1) ++pB;

    unsigned char* ring = smem;
    unsigned char* xreg = smem + W * kQDepth * kQSlot;
    const uint32_t ring_lds = lds_addr(ring) + wave * kQDepth * kQSlot;

    // x offsets in LDS: problems pA.. in order, M rows of bpr column blocks
    auto x_offset = [&](int p) -> int {
        int off = 0;
        for (int q = pA; q < p; ++q) off += M * a.probs[q].bpr * kXColBytes;
        return off;
    };
    auto load_prob = [&](int p, QProb& P) {
        const StreamProblem& s = a.probs[p];
        P.packed = uniform_ptr(s.packed);
        P.codebook = uniform_ptr(s.codebook);
        P.y = uniform_ptr(s.y);
        P.N = __builtin_amdgcn_readfirstlane(s.N);
        P.bpr = __builtin_amdgcn_readfirstlane(s.bpr);
        P.nblocks = ((P.N + 3) >> 2) * 4 * P.bpr;
        P.x_off = __builtin_amdgcn_readfirstlane(x_offset(p));
        P.y_mode = __builtin_amdgcn_readfirstlane(s.y_mode);
    };

    // ---- this wave's run of quads [S0, S1), balanced by pairs ---------------
    auto quad_at = [&](int64_t target) -> int {   // first quad at or past `target` pairs
        int64_t cum = 0;
        for (int p = pA; p <= pB; ++p) {
            const int lo = max(GQ0, a.quad_begin[p]), hi = min(GQ1, a.quad_begin[p + 1]);
            const int bpr = a.probs[p].bpr;
            const int64_t n = (int64_t)(hi - lo) * bpr;
            if (target < cum + n) return lo + (int)((target - cum + bpr - 1) / bpr);
            cum += n;
        }
        return GQ1;
    };
    int64_t total = 0;
    for (int p = pA; p <= pB; ++p) {
        const int lo = max(GQ0, a.quad_begin[p]), hi = min(GQ1, a.quad_begin[p + 1]);
        total += (int64_t)(hi - lo) * a.probs[p].bpr;
    }
    const int S0 = __builtin_amdgcn_readfirstlane(quad_at(total * wave / W));
    const int S1 = __builtin_amdgcn_readfirstlane(quad_at(total * (wave + 1) / W));
    struct Part {
        int p, qa, qb;   // problem, local quads [qa, qb)
    };
    // the run's part in its k-th problem (in order) -> (problem, quads);
    // false past the last
    auto part_of = [&](int k, Part& u) -> bool {
        for (int p = pA; p <= pB; ++p) {
            const int qb0 = a.quad_begin[p];
            const int lo = max(S0, qb0) - qb0, hi = min(S1, a.quad_begin[p + 1]) - qb0;
            if (hi <= lo) continue;
            if (k-- == 0) {
                u.p = p;
                u.qa = lo;
                u.qb = hi;
                return true;
            }
        }
        return false;
    };
    int kseg = 0;           // next part number

    // ---- load cursor: the next chunk of the run's current problem part -----
    // A ring slot records the part's number and the chunk (-1: past the
    // run's end, nothing loaded).
    int lf = -1;            // part being loaded
    Part lu = {0, 0, 0};    // its problem and quads
    int lc = 0, lc_end = 0; // its next chunk, one past its last
    QProb LP;
    int lp = -1;            // problem in LP
    auto next_part = [&]() {
        lf = kseg++;
        if (!part_of(lf, lu)) {
            lf = -1;
            return;
        }
        if (lu.p != lp) {
            load_prob(lu.p, LP);
            lp = lu.p;
        }
        lc = lu.qa * LP.bpr / 16;
        lc_end = (lu.qb * LP.bpr - 1) / 16 + 1;
    };
    next_part();
    struct Meta {
        int f, c;
        Part u;
    };
    auto issue = [&](int slot, Meta& m) {
        m.f = lf;
        m.c = lc;
        m.u = lu;
        if (lf < 0) return;
        const uint32_t dst = __builtin_amdgcn_readfirstlane(ring_lds + slot * kQSlot);
        const uint8_t* ip = LP.packed + (int64_t)lc * kQChunkIdx + 16 * lane;
        const uint8_t* cp =
            reinterpret_cast<const uint8_t*>(LP.codebook) + (int64_t)lc * kQChunkCb + 16 * lane;
        if ((lc + 1) * kQChunkBlocks <= LP.nblocks) {
            dma16<0>(dst, ip);
            dma16<1024>(dst, ip);
            dma16<2048>(dst, ip);
            dma16<0>(dst + kQChunkIdx, cp);
            dma16<1024>(dst + kQChunkIdx, cp);
        } else {
            // the layout's last, partial chunk: lanes past its end re-read
            // the last 16 bytes (blocks that are never used)
            const uint8_t* ilast = LP.packed + (int64_t)LP.nblocks * 48 - 16;
            const uint8_t* clast =
                reinterpret_cast<const uint8_t*>(LP.codebook) + (int64_t)LP.nblocks * 32 - 16;
            dma16<0>(dst, min(ip, ilast));
            dma16<0>(dst + 1024, min(ip + 1024, ilast));
            dma16<0>(dst + 2048, min(ip + 2048, ilast));
            dma16<0>(dst + kQChunkIdx, min(cp, clast));
            dma16<0>(dst + kQChunkIdx + 1024, min(cp + 1024, clast));
        }
        if (++lc == lc_end) next_part();
    };
    Meta ma = {-1, 0, {0, 0, 0}}, mb = {-1, 0, {0, 0, 0}};
    issue(0, ma);
    issue(1, mb);

    // ---- activations of the workgroup's problems, staged in LDS ------------
    // token t, column block c of problem p at x_off(p) + (t * bpr + c) * kXColBytes
    {
        int off = 0;
        for (int p = pA; p <= pB; ++p) {
            const StreamProblem& s = a.probs[p];
            const int bpr = s.bpr, K = s.K;
            const uint16_t* xp = static_cast<const uint16_t*>(s.x);
            for (int q = tid; q < M * bpr * 4; q += 64 * W) {
                const int u = q & 3, tc = q >> 2;   // tc = t * bpr + c
                const int t = tc / bpr, c = tc - t * bpr;
                const u32x4_t* src =
                    reinterpret_cast<const u32x4_t*>(xp + (int64_t)t * K + c * 128 + u * 32);
                uint32_t w[16];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const u32x4_t d = *as_global(src + v);
                    w[4 * v] = d.x;
                    w[4 * v + 1] = d.y;
                    w[4 * v + 2] = d.z;
                    w[4 * v + 3] = d.w;
                }
                stage_unit(xreg + off + tc * kXColBytes, u, w);
            }
            off += M * bpr * kXColBytes;
        }
    }
    __syncthreads();
    if (ma.f < 0) return;

    // ---- steady state: the run's chunks, in order ----------------------------
    const int grp = lane >> 2, j = lane & 3;
    const int tok = min(j, M - 1);
    int cf = -1;             // part being computed
    int ci = -1;             // problem in CP
    QProb CP = {};
    int qbeg = 0, pend = 0;  // the part's pairs
    int fq = 0, fchunk = 0;  // next quad to complete, the chunk holding its last pair
    // the column block of this lane's pair 16c + grp, advanced by 16 pairs a
    // chunk (bpr >= 16: at most one wrap)
    int lkb = 0;
    int xlane = 0;           // LDS offset of this lane's token's x rows
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};

    // A completed quad's sums wait in registers (lanes 0..3) and are stored
    // by the next step right after its ring wait: the stores then sit
    // before that step's ring loads in the wave's vector-memory order, so
    // the following wait (vmcnt <= one slot's loads) covers them without
    // draining the loads just issued.
    float pr0 = 0.f, pr1 = 0.f, pr2 = 0.f, pr3 = 0.f;
    int pq = -1;             // quad of the pending sums, -1: none
    QProb PP = {};           // its problem
    auto store_pending = [&]() {
        if (pq < 0) return;
        const float r[4] = {pr0, pr1, pr2, pr3};
        // lane j (< 4) holds token j; accumulator i holds row 4q + i
        if (lane < M) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 4 * pq + i;
                if (row < PP.N) {
                    const int64_t e = (int64_t)lane * PP.N + row;
                    if (a.y_dtype == NB_BF16) {
                        *as_global_mut(static_cast<bf16_bits*>(PP.y) + e) = f32_to_bf16_rne(r[i]);
                    } else if (PP.y_mode == NB_Y_ADD) {
                        // the element belongs to this wave alone: one add onto
                        // the prior value, without waiting for a load
                        unsafeAtomicAdd(static_cast<float*>(PP.y) + e, r[i]);
                    } else {
                        *as_global_mut(static_cast<float*>(PP.y) + e) = r[i];
                    }
                }
            }
        }
        pq = -1;
    };

    auto step = [&](int slot, Meta& m, bool other_valid) {
        if (m.f != cf) {
            // a new part (rare): its problem, pairs and the lane's position
            const Part u = m.u;
            cf = m.f;
            if (u.p != ci) {
                load_prob(u.p, CP);
                ci = u.p;
                xlane = CP.x_off + tok * CP.bpr * kXColBytes;
            }
            qbeg = u.qa * CP.bpr;
            pend = u.qb * CP.bpr;
            fq = u.qa;
            fchunk = ((fq + 1) * CP.bpr - 1) >> 4;
            const int pi0 = m.c * 16 + grp;
            lkb = pi0 % CP.bpr;
        } else {
            lkb += 16;
            if (lkb >= CP.bpr) lkb -= CP.bpr;
        }
        const int pi = m.c * 16 + grp;
        const bool live = pi >= qbeg && pi < pend;
        u32x4_t xv[16];
        {
            const unsigned char* xb = xreg + xlane + (live ? lkb : 0) * kXColBytes;
#pragma unroll
            for (int u = 0; u < 16; ++u) xv[u] = *reinterpret_cast<const u32x4_t*>(xb + 16 * u);
        }
        if (other_valid) {
            wait_vm<kQLoads>();
        } else {
            wait_vm<0>();
        }
        const unsigned char* src = ring + (wave * kQDepth + slot) * kQSlot;
        const u32x4_t* pi4 = reinterpret_cast<const u32x4_t*>(src + 48 * lane);
        const u32x4_t* pc4 = reinterpret_cast<const u32x4_t*>(src + kQChunkIdx + 32 * lane);
        const u32x4_t d0 = pi4[0], d1 = pi4[1], d2 = pi4[2], e0 = pc4[0], e1 = pc4[1];
        wait_lds();
        store_pending();
        const int c = m.c;
        issue(slot, m);
        const f32x4_t d = block_dot<true>(d0, d1, d2, e0, e1, xv);
        // lane 4g+j, accumulator i: row 4q+i, token j.  acc holds the lane's
        // sums for the quad of its latest pair; a lane's pair moves to the
        // next quad at most once a chunk (bpr >= 16), in the chunk where
        // that quad's predecessor ends.
        const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
        const f32x4_t dd = live ? d : z;
        if (c == fchunk) {
            // quad fq's last pair is in this chunk: lanes whose pair is still
            // in fq add this chunk's products, the others (already past it)
            // hold fq's sums from earlier chunks; sum over the 16 groups
            const bool in_fq = pi < (fq + 1) * CP.bpr;
            const f32x4_t v = acc + (in_fq ? dd : z);
            pr0 = group_sum(v.x);
            pr1 = group_sum(v.y);
            pr2 = group_sum(v.z);
            pr3 = group_sum(v.w);
            pq = fq;
            PP = CP;
            acc = in_fq ? z : dd;
            ++fq;
            fchunk = ((fq + 1) * CP.bpr - 1) >> 4;
        } else {
            acc += dd;
        }
    };
    while (true) {
        if (ma.f < 0) break;
        step(0, ma, mb.f >= 0);
        if (mb.f < 0) break;
        step(1, mb, ma.f >= 0);
    }
    store_pending();
    wait_vm<0>();
}

}  // namespace

// LDS bytes of workgroup g's x staging (M rows of each of its problems).
static int64_t quad_x_bytes(const StreamProblem* hp, const int* qbeg, int nprob, int q0, int q1,
                            int M) {
    int64_t n = 0;
    for (int p = 0; p < nprob; ++p) {
        if (qbeg[p + 1] <= q0 || qbeg[p] >= q1) continue;
        n += (int64_t)M * hp[p].bpr * kXColBytes;
    }
    return n;
}

bool gemv_quad_supported(const StreamProblem* hp, int nprob, int M) {
    if (M < 1 || M > kQMaxM) return false;
    for (int p = 0; p < nprob; ++p) {
        if (hp[p].bpr < kQMinBpr || hp[p].x_mode != NB_X_BF16 ||
            hp[p].y_mode == NB_Y_SILU_PAIRS) {
            return false;
        }
        // one problem's x must fit beside the smallest ring
        if ((int64_t)8 * kQDepth * kQSlot + (int64_t)M * hp[p].bpr * kXColBytes >
            device_lds_bytes()) {
            return false;
        }
    }
    return true;
}

// One launch (or more, past kStreamMaxGroups workgroup runs) over at most
// kQMaxProbs problems.
static int launch_quad_group(const StreamProblem* dev_probs, const StreamProblem* hp, int nprob,
                             int M, int y_dtype, hipStream_t stream) {
    std::vector<int> qbeg((size_t)nprob + 1, 0);
    std::vector<int64_t> pairs_before((size_t)nprob + 1, 0);
    for (int p = 0; p < nprob; ++p) {
        const int nq = (hp[p].N + 3) / 4;
        qbeg[p + 1] = qbeg[p] + nq;
        pairs_before[p + 1] = pairs_before[p] + (int64_t)nq * hp[p].bpr;
    }
    const int total_q = qbeg[nprob];
    const int64_t total_pairs = pairs_before[nprob];
    const int64_t lds_max = device_lds_bytes();
    const int64_t ring8 = (int64_t)8 * kQDepth * kQSlot, ring12 = (int64_t)12 * kQDepth * kQSlot;
    // pairs before global quad q
    auto pairs_at = [&](int q) -> int64_t {
        const int p = (int)(std::upper_bound(qbeg.begin(), qbeg.end(), q) - qbeg.begin()) - 1;
        if (p >= nprob) return total_pairs;
        return pairs_before[p] + (int64_t)(q - qbeg[p]) * hp[p].bpr;
    };
    // the first quad at or past `target` pairs
    auto quad_at = [&](int64_t target) -> int {
        if (target >= total_pairs) return total_q;
        const int p = (int)(std::upper_bound(pairs_before.begin(), pairs_before.end(), target) -
                            pairs_before.begin()) - 1;
        const int64_t r = target - pairs_before[p];
        return qbeg[p] + (int)((r + hp[p].bpr - 1) / hp[p].bpr);
    };
    // Workgroup runs balanced by pairs (each an equal share of what is left);
    // a run whose x staging does not fit beside the ring ends at the start
    // of its last problem (one problem's always fits the 8-wave ring:
    // checked above).  The 12-wave ring is planned first; when its runs
    // would need more workgroups than the device has CUs, the 8-wave one.
    const int G = std::max(1, std::min(device_cu_count(), total_q));
    auto plan = [&](int64_t ring) {
        std::vector<int> wq{0};
        while (wq.back() < total_q) {
            const int q0 = wq.back();
            const int64_t done = pairs_at(q0);
            const int left = std::max(1, G - ((int)wq.size() - 1));
            int q1 = std::max(q0 + 1,
                              std::min(total_q, quad_at(done + (total_pairs - done) / left)));
            while (ring + quad_x_bytes(hp, qbeg.data(), nprob, q0, q1, M) > lds_max) {
                const int p = (int)(std::upper_bound(qbeg.begin(), qbeg.end(), q1 - 1) -
                                    qbeg.begin()) - 1;
                if (qbeg[p] <= q0) return std::vector<int>();   // one problem does not fit
                q1 = qbeg[p];
            }
            wq.push_back(q1);
        }
        return wq;
    };
    std::vector<int> wq = plan(ring12);
    if (wq.empty() || (int)wq.size() - 1 > G) wq = plan(ring8);
    const int nruns = (int)wq.size() - 1;
    for (int r0 = 0; r0 < nruns; r0 += kStreamMaxGroups) {
        const int n = std::min(kStreamMaxGroups, nruns - r0);
        QuadArgs args;
        args.probs = dev_probs;
        args.nprob = nprob;
        args.M = M;
        args.y_dtype = y_dtype;
        for (int p = 0; p <= nprob; ++p) args.quad_begin[p] = qbeg[p];
        int64_t xmax = 0;
        for (int i = 0; i <= n; ++i) args.wg_q0[i] = wq[(size_t)(r0 + i)];
        for (int i = 0; i < n; ++i) {
            args.wg_p0[i] = (int)(std::upper_bound(qbeg.begin(), qbeg.end(), args.wg_q0[i]) -
                                  qbeg.begin()) - 1;
            xmax = std::max(xmax, quad_x_bytes(hp, qbeg.data(), nprob, args.wg_q0[i],
                                               args.wg_q0[i + 1], M));
        }
        if (ring12 + xmax <= lds_max) {
            hipLaunchKernelGGL(gemv_quad_kernel<12>, dim3(n), dim3(64 * 12),
                               (size_t)(ring12 + xmax), stream, args);
        } else {
            hipLaunchKernelGGL(gemv_quad_kernel<8>, dim3(n), dim3(64 * 8), (size_t)(ring8 + xmax),
                               stream, args);
        }
        const int st = check_launch("nb_gemm_skinny_quad_batched");
        if (st) return st;
    }
    return NB_OK;
}

int launch_gemv_quad(const StreamProblem* dev_probs, const StreamProblem* hp, int nprob, int M,
                     int y_dtype, hipStream_t stream) {
    if (!gemv_quad_supported(hp, nprob, M)) {
        return fail(NB_EUNSUPPORTED, "nb_gemm_skinny_quad_batched: needs M <= %d, K >= %d and "
                    "bf16 activations", kQMaxM, kQMinBpr * 128);
    }
    for (int p0 = 0; p0 < nprob; p0 += kQMaxProbs) {
        const int n = std::min(kQMaxProbs, nprob - p0);
        const int st = launch_quad_group(dev_probs + p0, hp + p0, n, M, y_dtype, stream);
        if (st) return st;
    }
    return NB_OK;
}

// ---- the row-quad layout ----------------------------------------------------

namespace {

// Thread t copies one 16-byte piece: pieces 0..2 of a block's indices, 3..4
// of its codebook.  Destination block b = 4 (q * bpr + kb) + i is row 4q + i,
// column block kb of the source (zero past row N).
__global__ __launch_bounds__(256) void quad_layout_kernel(const uint8_t* __restrict__ packed,
                                                          const float* __restrict__ codebook,
                                                          int N, int bpr, int64_t nblocks,
                                                          uint8_t* __restrict__ qpacked,
                                                          float* __restrict__ qcodebook) {
    // three threads a block: its 48 index bytes (four 12-byte units, each
    // rewritten as the selector-ordered unit) and the two halves of its
    // eight codebook entries
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= nblocks * 3) return;
    const int64_t b = t / 3;
    const int piece = (int)(t - b * 3);
    const int64_t pr = b >> 2;
    const int i = (int)(b & 3);
    const int64_t q = pr / bpr;
    const int kb = (int)(pr - q * bpr);
    const int64_t row = 4 * q + i;
    typedef __attribute__((ext_vector_type(4))) uint32_t v4;
    if (piece == 0) {
        uint32_t w[12] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
        if (row < N) {
            const v4* src = reinterpret_cast<const v4*>(packed + (row * bpr + kb) * 48);
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                const v4 v = src[j];
                w[4 * j] = v.x;
                w[4 * j + 1] = v.y;
                w[4 * j + 2] = v.z;
                w[4 * j + 3] = v.w;
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            uint32_t sel[8];
            unit_selectors(w[3 * u], w[3 * u + 1], w[3 * u + 2], sel);
            sel_unit_pack(sel, w[3 * u], w[3 * u + 1], w[3 * u + 2]);
        }
        v4* dst = reinterpret_cast<v4*>(qpacked + b * 48);
#pragma unroll
        for (int j = 0; j < 3; ++j) dst[j] = v4{w[4 * j], w[4 * j + 1], w[4 * j + 2], w[4 * j + 3]};
    } else {
        const int h = piece - 1;
        v4 v = {0u, 0u, 0u, 0u};
        if (row < N) v = *reinterpret_cast<const v4*>(codebook + (row * bpr + kb) * 8 + 4 * h);
        *reinterpret_cast<v4*>(qcodebook + b * 8 + 4 * h) = v;
    }
}

}  // namespace

int launch_quad_layout(const uint8_t* packed, const float* codebook, int N, int K,
                       uint8_t* qpacked, float* qcodebook, hipStream_t stream) {
    const int bpr = K / 128;
    const int64_t nblocks = (int64_t)((N + 3) / 4) * 4 * bpr;
    const int64_t threads = nblocks * 3;
    if (threads == 0) return NB_OK;
    hipLaunchKernelGGL(quad_layout_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       stream, packed, codebook, N, bpr, nblocks, qpacked, qcodebook);
    return check_launch("nb_quad_layout");
}

}  // namespace nb
