// Batched packed skinny GEMM on gfx950: many 3-bit layers, M <= 16
// activation rows, one launch.
//
//   for every problem p:  y_p[m][n] = sum_k x_p[m][k] * bf16(W_p[n][k]),  m < M
//
// The batched branch of PackedLinear.forward (inference/triton_kernel.py:
// 258-275) in its bf16 form (inference/eval_ppl.py:149-174) for the few
// token rows of a small-batch decode step, over all layers of the step.
//
// Work split.  A workgroup task is 128 rows of one problem (8 waves, one
// 16-row group each) over all of K, taken in slices of 512 (4 blocks of
// 128).  Per slice, lane l = q*16 + r of a wave takes row r of its group and
// block q of the slice: 48 bytes of indices and 8 fp32 codebook entries
// (the 4 lanes of a row read 192 contiguous bytes), turned into 16 MFMA
// A-operands of v_mfma_f32_16x16x32_bf16 by register codebook lookups
// (v_perm_b32 on byte planes of the bf16-rounded entries, 17 VALU ops per 8
// weights).  B is the slice of x: MFMA column c = activation row c, staged
// once per slice in LDS for the whole workgroup (rows padded by 16 bytes so
// the 16 columns of one read fall in different banks; columns c >= M repeat
// row M-1 and are not stored).  The accumulator (16 rows x 16 columns per
// wave) stays in registers over all of K: no cross-wave reduction.
//
// Pipelining.  While slice s is computed, the weights of slices s+1 and s+2
// and the x of slice s+1 are in flight; the x registers are written to the
// other LDS buffer after the MFMAs (vector-memory loads complete in order,
// so that waits for the loads issued up to then, not for slice s+2's), and
// one barrier per slice hands the buffer over.
//
// Weights are rounded to bf16 (RNE), as the reference's bf16 path;
// accumulation is fp32.
#include <algorithm>

#include "nb_device.h"
#include "nb_internal.h"

namespace nb {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;

constexpr int kSkWaves = 8;
constexpr int kSkThreads = 64 * kSkWaves;
constexpr int kSkRows = 16 * kSkWaves;       // rows of one workgroup task
constexpr int kSkSliceK = 512;               // K of one slice (4 blocks)
constexpr int kSkMaxM = 16;
constexpr int kSkXPitch = kSkSliceK * 2 + 16;  // LDS bytes of one staged x row
constexpr int kSkXGran = kSkMaxM * kSkSliceK / 8 / kSkThreads;  // 16-byte x pieces per thread

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

// One lane's block of one slice: 48 index bytes and the 8 codebook entries.
struct Tile {
    uint32_t d[12];
    float c[8];
};

__device__ __forceinline__ void load_tile(const uint8_t* __restrict__ packed,
                                          const float* __restrict__ cb, int64_t row, int bcol,
                                          int bpr, Tile& t) {
    const u32x4_t* p =
        reinterpret_cast<const u32x4_t*>(packed + (row * bpr + bcol) * (int64_t)48);
#pragma unroll
    for (int v = 0; v < 3; ++v) {
        const u32x4_t u = stream_load(p + v);
        t.d[4 * v] = u.x;
        t.d[4 * v + 1] = u.y;
        t.d[4 * v + 2] = u.z;
        t.d[4 * v + 3] = u.w;
    }
    const f32x4_t* c = reinterpret_cast<const f32x4_t*>(cb + (row * bpr + bcol) * 8);
#pragma unroll
    for (int v = 0; v < 2; ++v) {
        const f32x4_t f = stream_load(c + v);
        t.c[4 * v] = f.x;
        t.c[4 * v + 1] = f.y;
        t.c[4 * v + 2] = f.z;
        t.c[4 * v + 3] = f.w;
    }
}

template <int J>
__device__ __forceinline__ void mfma_groups(const Tile& t, uint32_t lo0, uint32_t lo1,
                                            uint32_t hi0, uint32_t hi1,
                                            const unsigned char* bsrc, f32x4_t& acc) {
    if constexpr (J < 16) {
        const u32x4_t a = lookup8(group24<J>(t.d), lo0, lo1, hi0, hi1);
        const u32x4_t b = *reinterpret_cast<const u32x4_t*>(bsrc + 16 * J);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                      __builtin_bit_cast(bf16x8_t, b), acc,
                                                      0, 0, 0);
        mfma_groups<J + 1>(t, lo0, lo1, hi0, hi1, bsrc, acc);
    }
}

// The 128 weights of the lane's block times the staged x (zero weights when
// the block is not live).
__device__ __forceinline__ void compute_tile(const Tile& t, bool live, const unsigned char* bsrc,
                                             f32x4_t& acc) {
    const uint32_t p0 = pack_bf16x2(t.c[0], t.c[1]);
    const uint32_t p1 = pack_bf16x2(t.c[2], t.c[3]);
    const uint32_t p2 = pack_bf16x2(t.c[4], t.c[5]);
    const uint32_t p3 = pack_bf16x2(t.c[6], t.c[7]);
    uint32_t lo0 = __builtin_amdgcn_perm(p1, p0, 0x06040200u);
    uint32_t hi0 = __builtin_amdgcn_perm(p1, p0, 0x07050301u);
    uint32_t lo1 = __builtin_amdgcn_perm(p3, p2, 0x06040200u);
    uint32_t hi1 = __builtin_amdgcn_perm(p3, p2, 0x07050301u);
    lo0 = live ? lo0 : 0u;
    hi0 = live ? hi0 : 0u;
    lo1 = live ? lo1 : 0u;
    hi1 = live ? hi1 : 0u;
    mfma_groups<0>(t, lo0, lo1, hi0, hi1, bsrc, acc);
}

__global__ __launch_bounds__(kSkThreads) void gemv_skinny_kernel(
    const StreamProblem* __restrict__ probs, SkinnyTasks tasks, int M, int y_dtype) {
    __shared__ __align__(16) unsigned char xs[2][kSkMaxM * kSkXPitch];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int r = lane & 15;
    const int q = lane >> 4;

    // ---- the task's problem (binary search over the task prefix) ----------
    const int task = blockIdx.x;
    int lo = 0, hi = tasks.nprob - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (tasks.task_begin[mid] <= task) lo = mid; else hi = mid - 1;
    }
    const StreamProblem& P = probs[tasks.prob0 + lo];
    const int N = P.N, K = P.K, bpr = K >> 7;
    const uint8_t* packed = P.packed;
    const float* cb = P.codebook;
    const uint16_t* x = static_cast<const uint16_t*>(P.x);
    const int row0 = (task - tasks.task_begin[lo]) * kSkRows + wave * 16;
    const int row = row0 + r;
    const bool row_ok = row < N;
    const int64_t lrow = row_ok ? row : N - 1;  // clamped: loads stay in bounds
    const int nslices = (bpr + 3) >> 2;

    auto bcol_of = [&](int s) {
        const int b = 4 * s + q;
        return b < bpr ? b : bpr - 1;
    };
    // x pieces of slice s: piece g = tid + j * kSkThreads is row g / 64,
    // 16-byte part g % 64 of the slice (zero past K or M).  Every lane loads
    // (a clamped, in-bounds address) and the value is selected afterwards:
    // no branch around a load, so the compiler's wait counts stay exact.
    auto load_x = [&](int s, u32x4_t (&v)[kSkXGran]) {
#pragma unroll
        for (int j = 0; j < kSkXGran; ++j) {
            const int g = tid + j * kSkThreads;
            const int m = g >> 6, k = s * kSkSliceK + (g & 63) * 8;
            const int mc = m < M ? m : M - 1, kc = k < K ? k : K - 8;
            v[j] = *as_global(reinterpret_cast<const u32x4_t*>(x + (int64_t)mc * K + kc));
        }
    };
    auto keep_x = [&](int s, u32x4_t (&v)[kSkXGran]) {
#pragma unroll
        for (int j = 0; j < kSkXGran; ++j) {
            const int g = tid + j * kSkThreads;
            const bool in = (g >> 6) < M && s * kSkSliceK + (g & 63) * 8 < K;
            v[j].x = in ? v[j].x : 0u;
            v[j].y = in ? v[j].y : 0u;
            v[j].z = in ? v[j].z : 0u;
            v[j].w = in ? v[j].w : 0u;
        }
    };
    // (rows m >= M are written too, as zeros: no branch around the stores)
    auto store_x = [&](unsigned char* buf, const u32x4_t (&v)[kSkXGran]) {
#pragma unroll
        for (int j = 0; j < kSkXGran; ++j) {
            const int g = tid + j * kSkThreads;
            *reinterpret_cast<u32x4_t*>(buf + (g >> 6) * kSkXPitch + (g & 63) * 16) = v[j];
        }
    };

    // MFMA column r reads activation row min(r, M - 1)
    const int xm = r < M ? r : M - 1;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    Tile ta, tb, tc;
    u32x4_t xv[kSkXGran];
    // slice s: computes tile `now` (loaded two slices earlier) while slice
    // s + 1's x and slice s + 2's tile `ahead` load; the three tiles rotate,
    // so no register copy waits for a load.  Past the last slice the loads
    // repeat the last one (cache hits) and nothing is stored.
    auto slice = [&](int s, Tile& now, Tile& ahead) {
        const int s1 = min(s + 1, nslices - 1), s2 = min(s + 2, nslices - 1);
        load_x(s1, xv);
        load_tile(packed, cb, lrow, bcol_of(s2), bpr, ahead);
        // the loads stay ahead of the arithmetic (the scheduler would sink
        // the x loads next to their use and wait for them there)
        __builtin_amdgcn_sched_barrier(0);
        const bool live = row_ok && 4 * s + q < bpr;
        compute_tile(now, live, xs[s & 1] + xm * kSkXPitch + q * 256, acc);
        keep_x(s1, xv);
        // (after the last slice the other buffer is no longer read)
        store_x(xs[(s + 1) & 1], xv);
        __syncthreads();
    };
    load_x(0, xv);
    load_tile(packed, cb, lrow, bcol_of(0), bpr, ta);
    load_tile(packed, cb, lrow, bcol_of(min(1, nslices - 1)), bpr, tb);
    keep_x(0, xv);
    store_x(xs[0], xv);
    __syncthreads();
    for (int s = 0; s < nslices; s += 3) {
        slice(s, ta, tc);
        if (s + 1 < nslices) slice(s + 1, tb, ta);
        if (s + 2 < nslices) slice(s + 2, tc, tb);
    }

    // acc lane (q, r) holds C[4q + v][r]: y[r][row0 + 4q + v]
    if (r < M) {
        const bool add = P.y_mode == NB_Y_ADD;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int n = row0 + 4 * q + v;
            if (n >= N) continue;
            const int64_t i = (int64_t)r * N + n;
            if (y_dtype == NB_BF16) {
                *as_global_mut(static_cast<bf16_bits*>(P.y) + i) = f32_to_bf16_rne(acc[v]);
            } else if (add) {
                auto* yp = as_global_mut(static_cast<float*>(P.y) + i);
                *yp = *yp + acc[v];
            } else {
                *as_global_mut(static_cast<float*>(P.y) + i) = acc[v];
            }
        }
    }
}

}  // namespace

int launch_gemv_skinny(const StreamProblem* dev_probs, const StreamProblem* host_probs,
                       int nprob, int M, int y_dtype, hipStream_t stream) {
    // launches of at most kSkinnyMaxProbs problems each
    for (int p0 = 0; p0 < nprob; p0 += kSkinnyMaxProbs) {
        const int n = std::min(kSkinnyMaxProbs, nprob - p0);
        SkinnyTasks T;
        T.prob0 = p0;
        T.nprob = n;
        int64_t total = 0;
        for (int i = 0; i < n; ++i) {
            T.task_begin[i] = (int32_t)total;
            total += (host_probs[p0 + i].N + kSkRows - 1) / kSkRows;
        }
        if (total == 0) continue;
        if (total > 0x7fffffff) return fail(NB_EUNSUPPORTED, "nb_gemm_skinny_batched: too many rows");
        hipLaunchKernelGGL(gemv_skinny_kernel, dim3((unsigned)total), dim3(kSkThreads), 0, stream,
                           dev_probs, T, M, y_dtype);
        const int st = check_launch("nb_gemm_skinny_batched");
        if (st) return st;
    }
    return NB_OK;
}

}  // namespace nb
