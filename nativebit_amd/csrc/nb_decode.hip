// Kernels of one greedy decode step of the packed NativeBit decoder (gfx950),
// everything but the packed GEMVs:
//
//   nb_add_rmsnorm      x (+)= y (or x = embedding[token]); h = rmsnorm(x) * w
//                       (generate_torch.py:29-38, residuals 128-132, 150)
//   nb_attention_step   RoPE at the current position, K/V append, softmax
//                       attention over positions 0..pos for every head
//                       (generate_torch.py:48-60, 72-106 with T = 1)
//   nb_silu_mul         silu(gate) * up (generate_torch.py:116-117)
//   nb_lm_head_argmax   tied head, 30 tanh(l / 30) soft cap, greedy argmax,
//                       position advance (generate_torch.py:157-159, 311)
//
// The position and the current token live in a device-side nb_decode_state,
// so a whole step is a fixed sequence of launches that can be captured once
// in a HIP graph and replayed per token without a host round trip.
// Arithmetic is fp32 (activations may be handed on as bf16, rounded to
// nearest even).
#include <math.h>

#include <algorithm>
#include <mutex>

#include "nb_device.h"
#include "nb_internal.h"

namespace nb {
namespace {

__device__ __forceinline__ float load_act(const void* p, int dtype, int64_t i) {
    if (dtype == NB_BF16) return bf16_to_f32(static_cast<const bf16_bits*>(p)[i]);
    return static_cast<const float*>(p)[i];
}

__device__ __forceinline__ void store_act(void* p, int dtype, int64_t i, float v) {
    if (dtype == NB_BF16) {
        static_cast<bf16_bits*>(p)[i] = f32_to_bf16_rne(v);
    } else {
        static_cast<float*>(p)[i] = v;
    }
}

// Cross-workgroup hand-over inside one launch.  Values another workgroup
// will read are written and read with agent-scope atomic accesses, which
// are coherent across the XCDs' separate L2 caches, and the writer waits
// for its stores to complete (vmcnt counts stores on gfx9) before it bumps
// the counter that publishes them.  A __threadfence() would instead write
// back the whole L2 of the XCD, which costs tens of microseconds when the
// decode step leaves much dirty data behind.
__device__ __forceinline__ void put_agent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float get_agent(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" : : : "memory"); }

__device__ __forceinline__ float wave_sum(float v) { return wave64_sum(v); }

__device__ __forceinline__ float wave_max(float v) { return wave64_max(v); }

// Block-wide sum of one value per thread (blockDim.x a multiple of 64,
// at most 1024).
__device__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
    for (int w = 0; w < nw; ++w) t += red[w];  // same order in every thread
    return t;
}

// ---------------------------------------------------------------------------
// RMSNorm with the residual add or the embedding lookup in front
// ---------------------------------------------------------------------------
constexpr int kNormThreads = 1024;

__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(
    float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ emb,
    const nb_decode_state* __restrict__ st, const float* __restrict__ w, void* __restrict__ h,
    int h_dtype, int n, float eps) {
    __shared__ float red[kNormThreads / 64];
    const float* src_row = nullptr;
    if (emb) src_row = emb + (int64_t)st->token * n;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float v;
        if (src_row) {
            v = src_row[i];
        } else {
            v = x[i];
            if (y) v = v + y[i];
        }
        if (src_row || y) x[i] = v;
        ss += v * v;
    }
    const float mean = block_sum(ss, red) / (float)n;
    const float norm = sqrtf(mean + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        // (x / norm) * w, as generate_torch.py:37
        store_act(h, h_dtype, i, (x[i] / norm) * w[i]);
    }
}

// ---------------------------------------------------------------------------
// attention for one new token, split over positions
// ---------------------------------------------------------------------------
// Caches: keys transposed, [n_head][D][ctx] (position fastest), values
// [n_head][ctx][D].  Grid (n_head, kAttnSplits); workgroup (hd, s) takes the
// contiguous positions [s*Lp, min(pos+1, (s+1)*Lp)), Lp = ceil((pos+1)/S)
// <= 64.  Scores: lane i takes position t0 + i and each of the 4 waves a
// quarter of the head dimension, so every key load is 64 consecutive
// positions (coalesced); the quarters are summed in wave order.  Softmax
// partials (max, sum) and the weighted sum of values (thread d takes
// dimension d, reading value rows whole) go to the workspace; the last
// workgroup of a head (atomic counter) combines the splits in split order.
// Every workgroup rotates the new query and key itself; the workgroup whose
// range holds pos uses the new key/value directly and is the only one that
// writes them to the caches, so nothing reads what another workgroup writes
// in the same launch.
constexpr int kAttnSplits = 16;
constexpr int kAttnThreads = 256;
constexpr int kAttnMaxSplitLen = 64;
constexpr int kMaxHeadDim = 256;
constexpr int kMaxCtx = kAttnSplits * kAttnMaxSplitLen;

__global__ __launch_bounds__(kAttnThreads) void attention_step_kernel(
    const float* __restrict__ qkv, float* __restrict__ k_cache, float* __restrict__ v_cache,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    const nb_decode_state* __restrict__ st, float* __restrict__ work, unsigned* __restrict__ done,
    void* __restrict__ out, int out_dtype, int n_head, int D, int ctx) {
    __shared__ float q[kMaxHeadDim], kn[kMaxHeadDim], vn[kMaxHeadDim];
    __shared__ float sc[kAttnThreads / 64][kAttnMaxSplitLen];
    __shared__ float p[kAttnMaxSplitLen];
    __shared__ float ml[2];
    __shared__ unsigned last;
    const int hd = blockIdx.x, s = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pos = st->pos;
    if (pos < 0 || pos >= ctx) return;  // past the cache: nothing to do
    const int C = n_head * D;
    const float scale = 1.0f / sqrtf((float)D);
    const int n = pos + 1;
    const int Lp = (n + kAttnSplits - 1) / kAttnSplits;
    const int t0 = min(n, s * Lp), t1 = min(n, t0 + Lp);
    // RoPE of the new query and key (pairs (2i, 2i+1) rotated by angle i)
    for (int i = tid; i < D / 2; i += kAttnThreads) {
        const float c = cos_t[(int64_t)pos * (D / 2) + i], sn = sin_t[(int64_t)pos * (D / 2) + i];
        const float q0 = qkv[hd * D + 2 * i], q1 = qkv[hd * D + 2 * i + 1];
        const float k0 = qkv[C + hd * D + 2 * i], k1 = qkv[C + hd * D + 2 * i + 1];
        // q * cos2 + rotate(q) * sin2, then the reference's (q * scale)
        q[2 * i] = __fmul_rn(__fadd_rn(__fmul_rn(q0, c), __fmul_rn(-q1, sn)), scale);
        q[2 * i + 1] = __fmul_rn(__fadd_rn(__fmul_rn(q1, c), __fmul_rn(q0, sn)), scale);
        kn[2 * i] = __fadd_rn(__fmul_rn(k0, c), __fmul_rn(-k1, sn));
        kn[2 * i + 1] = __fadd_rn(__fmul_rn(k1, c), __fmul_rn(k0, sn));
    }
    for (int d = tid; d < D; d += kAttnThreads) vn[d] = qkv[2 * C + hd * D + d];
    __syncthreads();
    const float* kt = k_cache + (int64_t)hd * D * ctx;  // [D][ctx]
    const float* vc = v_cache + (int64_t)hd * ctx * D;  // [ctx][D]
    if (pos >= t0 && pos < t1) {
        for (int d = tid; d < D; d += kAttnThreads) {
            k_cache[((int64_t)hd * D + d) * ctx + pos] = kn[d];
            v_cache[((int64_t)hd * ctx + pos) * D + d] = vn[d];
        }
    }
    // partial scores of this wave's quarter of the dimensions
    const int t = t0 + lane;
    const int dq = (D + 3) / 4;
    const int d0 = wave * dq, d1 = min(D, d0 + dq);
    float part = 0.f;
    if (t < t1) {
        if (t == pos) {
            for (int d = d0; d < d1; ++d) part += q[d] * kn[d];
        } else {
#pragma unroll 8
            for (int d = d0; d < d1; ++d) part += q[d] * kt[(int64_t)d * ctx + t];
        }
    }
    sc[wave][lane] = part;
    __syncthreads();
    float* wk = work + ((int64_t)hd * kAttnSplits + s) * (kMaxHeadDim + 2);
    if (wave == 0) {
        float score = -INFINITY;
        if (t < t1) {
            score = 0.f;
            for (int w = 0; w < kAttnThreads / 64; ++w) score += sc[w][lane];
        }
        const float m = wave_max(score);
        const float e = t < t1 ? __expf(score - m) : 0.f;
        const float l = wave_sum(e);
        p[lane] = e;
        if (lane == 0) {
            ml[0] = m;
            ml[1] = l;
        }
    }
    __syncthreads();
    for (int d = tid; d < D; d += kAttnThreads) {
        float o = 0.f;
        for (int i = 0; i < t1 - t0; ++i) {
            const int tt = t0 + i;
            o += p[i] * (tt == pos ? vn[d] : vc[(int64_t)tt * D + d]);
        }
        put_agent(wk + 2 + d, o);
    }
    if (tid == 0) {
        put_agent(wk, ml[0]);
        put_agent(wk + 1, ml[1]);
    }
    // the last workgroup of this head combines the splits
    wait_stores();
    __syncthreads();
    if (tid == 0) {
        last = __hip_atomic_fetch_add(done + hd, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                       kAttnSplits - 1
                   ? 1u
                   : 0u;
    }
    __syncthreads();
    if (!last) return;
    const float* base = work + (int64_t)hd * kAttnSplits * (kMaxHeadDim + 2);
    for (int d = tid; d < D; d += kAttnThreads) {
        float M = -INFINITY;
        for (int j = 0; j < kAttnSplits; ++j) {
            M = fmaxf(M, get_agent(base + j * (kMaxHeadDim + 2)));
        }
        float L = 0.f, O = 0.f;
        for (int j = 0; j < kAttnSplits; ++j) {
            const float* pj = base + j * (kMaxHeadDim + 2);
            const float mj = get_agent(pj);
            const float f = mj == -INFINITY ? 0.f : __expf(mj - M);
            L += f * get_agent(pj + 1);
            O += f * get_agent(pj + 2 + d);
        }
        store_act(out, out_dtype, hd * D + d, O / L);
    }
    if (tid == 0) done[hd] = 0u;  // ready for the next step
}

// The same step for head_dim <= 128 with every global load of a workgroup
// issued before the first is used: the query/key/value of the head and the
// RoPE row first, then all of the split's cached keys (lane = position,
// wave = a quarter of the dimensions, up to 32 loads per thread) and values
// (thread = dimension and half of the positions, up to 32 loads), so a
// workgroup pays one memory latency instead of one per dependent loop.
// Scores, softmax partials, the weighted values and the split combine are
// those of attention_step_kernel, in the same order.
constexpr int kAttn2MaxD = 128;

__global__ __launch_bounds__(kAttnThreads) void attention_step2_kernel(
    const float* __restrict__ qkv, float* __restrict__ k_cache, float* __restrict__ v_cache,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    const nb_decode_state* __restrict__ st, float* __restrict__ work, unsigned* __restrict__ done,
    void* __restrict__ out, int out_dtype, int n_head, int D, int ctx) {
    __shared__ float q[kAttn2MaxD], kn[kAttn2MaxD], vn[kAttn2MaxD];
    __shared__ float sc[kAttnThreads / 64][kAttnMaxSplitLen];
    __shared__ float p[kAttnMaxSplitLen];
    __shared__ float oh[2][kAttn2MaxD];
    __shared__ float ml[2];
    __shared__ unsigned last;
    const int hd = blockIdx.x, s = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pos = st->pos;
    if (pos < 0 || pos >= ctx) return;  // past the cache: nothing to do
    const int C = n_head * D;
    const float scale = 1.0f / sqrtf((float)D);
    const int n = pos + 1;
    const int Lp = (n + kAttnSplits - 1) / kAttnSplits;
    const int t0 = min(n, s * Lp), t1 = min(n, t0 + Lp);
    const int len = t1 - t0;

    // ---- loads: the head's new q, k, v and the RoPE row, then the split's
    //      cached keys and values (clamped addresses; unused values are
    //      never read)
    const int half = D / 2;
    float q0 = 0.f, q1 = 0.f, k0 = 0.f, k1 = 0.f, c = 0.f, sn = 0.f, v0 = 0.f;
    if (tid < half) {
        q0 = qkv[hd * D + 2 * tid];
        q1 = qkv[hd * D + 2 * tid + 1];
        k0 = qkv[C + hd * D + 2 * tid];
        k1 = qkv[C + hd * D + 2 * tid + 1];
        c = cos_t[(int64_t)pos * half + tid];
        sn = sin_t[(int64_t)pos * half + tid];
    }
    if (tid < D) v0 = qkv[2 * C + hd * D + tid];
    const int dq = (D + 3) / 4;
    const int d0 = wave * dq;
    const int t = t0 + lane;
    const int tk = lane < len ? t : t0;           // a position of the split
    float kr[kAttn2MaxD / 4];
    const float* kt = k_cache + (int64_t)hd * D * ctx;  // [D][ctx]
    // values: thread (vh, d), vh = tid / 128: positions of half vh
    const int vd = tid & (kAttn2MaxD - 1), vh = tid >> 7;
    const int vlen = (len + 1) / 2;
    const int vt0 = t0 + vh * vlen;
    const int vcnt = max(0, min(vlen, t1 - vt0));
    float vr[kAttnMaxSplitLen / 2];
    const float* vc = v_cache + (int64_t)hd * ctx * D;  // [ctx][D]
    if (len > 0) {
#pragma unroll
        for (int j = 0; j < kAttn2MaxD / 4; ++j) {
            const int d = min(d0 + j, D - 1);
            kr[j] = kt[(int64_t)d * ctx + tk];
        }
        const int dv = min(vd, D - 1);
#pragma unroll
        for (int j = 0; j < kAttnMaxSplitLen / 2; ++j) {
            const int tt = min(vt0 + j, t1 - 1);
            vr[j] = vc[(int64_t)tt * D + dv];
        }
    }
    // RoPE of the new query and key (pairs (2i, 2i+1) rotated by angle i),
    // then the reference's (q * scale)
    if (tid < half) {
        q[2 * tid] = __fmul_rn(__fadd_rn(__fmul_rn(q0, c), __fmul_rn(-q1, sn)), scale);
        q[2 * tid + 1] = __fmul_rn(__fadd_rn(__fmul_rn(q1, c), __fmul_rn(q0, sn)), scale);
        kn[2 * tid] = __fadd_rn(__fmul_rn(k0, c), __fmul_rn(-k1, sn));
        kn[2 * tid + 1] = __fadd_rn(__fmul_rn(k1, c), __fmul_rn(k0, sn));
    }
    if (tid < D) vn[tid] = v0;
    __syncthreads();
    if (pos >= t0 && pos < t1 && tid < D) {
        k_cache[((int64_t)hd * D + tid) * ctx + pos] = kn[tid];
        v_cache[((int64_t)hd * ctx + pos) * D + tid] = vn[tid];
    }
    // partial scores of this wave's quarter of the dimensions
    float part = 0.f;
    if (lane < len) {
        const bool is_new = t == pos;
#pragma unroll
        for (int j = 0; j < kAttn2MaxD / 4; ++j) {
            if (j < dq && d0 + j < D) part += q[d0 + j] * (is_new ? kn[d0 + j] : kr[j]);
        }
    }
    sc[wave][lane] = part;
    __syncthreads();
    float* wk = work + ((int64_t)hd * kAttnSplits + s) * (kMaxHeadDim + 2);
    if (wave == 0) {
        float score = -INFINITY;
        if (lane < len) {
            score = 0.f;
            for (int w = 0; w < kAttnThreads / 64; ++w) score += sc[w][lane];
        }
        const float m = wave_max(score);
        const float e = lane < len ? __expf(score - m) : 0.f;
        const float l = wave_sum(e);
        p[lane] = e;
        if (lane == 0) {
            ml[0] = m;
            ml[1] = l;
        }
    }
    __syncthreads();
    // weighted values: thread (vh, vd) over its half of the positions
    float o = 0.f;
    if (vd < D) {
#pragma unroll
        for (int j = 0; j < kAttnMaxSplitLen / 2; ++j) {
            if (j < vcnt) {
                const int tt = vt0 + j;
                o += p[tt - t0] * (tt == pos ? vn[vd] : vr[j]);
            }
        }
    }
    oh[vh][vd] = o;
    __syncthreads();
    if (tid < D) put_agent(wk + 2 + tid, oh[0][tid] + oh[1][tid]);
    if (tid == 0) {
        put_agent(wk, ml[0]);
        put_agent(wk + 1, ml[1]);
    }
    // the last workgroup of this head combines the splits
    wait_stores();
    __syncthreads();
    if (tid == 0) {
        last = __hip_atomic_fetch_add(done + hd, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                       kAttnSplits - 1
                   ? 1u
                   : 0u;
    }
    __syncthreads();
    if (!last) return;
    const float* base = work + (int64_t)hd * kAttnSplits * (kMaxHeadDim + 2);
    if (tid < D) {
        float M = -INFINITY;
        float mj[kAttnSplits], lj[kAttnSplits], oj[kAttnSplits];
#pragma unroll
        for (int j = 0; j < kAttnSplits; ++j) {
            const float* pj = base + j * (kMaxHeadDim + 2);
            mj[j] = get_agent(pj);
            lj[j] = get_agent(pj + 1);
            oj[j] = get_agent(pj + 2 + tid);
        }
#pragma unroll
        for (int j = 0; j < kAttnSplits; ++j) M = fmaxf(M, mj[j]);
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int j = 0; j < kAttnSplits; ++j) {
            const float f = mj[j] == -INFINITY ? 0.f : __expf(mj[j] - M);
            L += f * lj[j];
            O += f * oj[j];
        }
        store_act(out, out_dtype, hd * D + tid, O / L);
    }
    if (tid == 0) done[hd] = 0u;  // ready for the next step
}

// ---------------------------------------------------------------------------
// attention in TP-position tiles, head_dim 128 (the decode model's shape)
// ---------------------------------------------------------------------------
// Workgroup (hd, s) of 512 threads takes positions [TP s, TP s + TP) of head
// hd; only ceil((pos + 1) / TP) tiles are in use.  All global loads are
// issued before the first is used, as 16-byte loads: keys as (4 positions x
// DPG dimensions) per thread, values as (PPG positions x 4 dimensions), so
// one memory latency and the tile's bytes bound the launch.  Scores: DG
// partial sums over DPG dimensions, added in order; softmax partials per
// wave of 64 positions (max, sum of exp); the weighted values per group of
// PPG positions, merged in group order with the waves' factors exp(m_w -
// M).  With more than one tile in use, each writes (M, L, O) and the last to
// finish (agent-scope counter) merges them in tile order.  Keys
// [n_head][128][ctx] and values [n_head][ctx][128] fp32, ctx % 4 == 0,
// 16-byte aligned.
constexpr int kTileD = 128;
constexpr int kTileThreads = 512;
#ifndef NB_ATT_TILE
#define NB_ATT_TILE 128
#endif
constexpr int kTilePos = NB_ATT_TILE;
static_assert(kMaxCtx / kTilePos <= kAttnSplits, "tiles fit the partials buffer");

template <int TP>
__global__ __launch_bounds__(kTileThreads) void attention_tile_kernel(
    const float* __restrict__ qkv, float* __restrict__ k_cache, float* __restrict__ v_cache,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    const nb_decode_state* __restrict__ st, float* __restrict__ work, unsigned* __restrict__ done,
    void* __restrict__ out, int out_dtype, int n_head, int ctx) {
    typedef __attribute__((ext_vector_type(4))) float f4;
    constexpr int D = kTileD;
    constexpr int PQ = TP / 4;                 // key position quads
    constexpr int DG = kTileThreads / PQ;      // key dimension groups
    constexpr int DPG = D / DG;                // dimensions per group
    constexpr int G = kTileThreads / (D / 4);  // value position groups (16)
    constexpr int PPG = TP / G;                // positions per value group
    constexpr int NW = TP / 64;                // softmax waves
    static_assert(DPG % 4 == 0 && PPG % 4 == 0 && NW >= 1, "tile shape");
    __shared__ __align__(16) float qs[D], kn[D], vn[D];
    __shared__ __align__(16) float sc[DG][TP];
    __shared__ __align__(16) float pl[TP];
    __shared__ __align__(16) float oh[G][D];
    __shared__ float wm[NW], wl[NW];
    __shared__ unsigned last;
    const int hd = blockIdx.x, s = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pos = st->pos;
    if (pos < 0 || pos >= ctx) return;  // past the cache: nothing to do
    const int n = pos + 1;
    const int S = (n + TP - 1) / TP;  // tiles in use
    if (s >= S) return;
    const int t0 = s * TP, len = min(TP, n - t0);
    const int C = n_head * D;
    const float scale = 1.0f / sqrtf((float)D);

    // ---- loads: the new q, k, v and RoPE row; the tile's keys and values
    //      (positions past the tile's last one read that one again)
    float q0 = 0.f, q1 = 0.f, k0 = 0.f, k1 = 0.f, c = 0.f, sn = 0.f, v0 = 0.f;
    if (tid < D / 2) {
        q0 = qkv[hd * D + 2 * tid];
        q1 = qkv[hd * D + 2 * tid + 1];
        k0 = qkv[C + hd * D + 2 * tid];
        k1 = qkv[C + hd * D + 2 * tid + 1];
        c = cos_t[(int64_t)pos * (D / 2) + tid];
        sn = sin_t[(int64_t)pos * (D / 2) + tid];
    }
    if (tid < D) v0 = qkv[2 * C + hd * D + tid];
    const int pq = tid % PQ, dg = tid / PQ;           // keys: 4 positions, DPG dims
    const int tk = t0 + min(4 * pq, (len - 1) & ~3);
    const float* kt = k_cache + (int64_t)hd * D * ctx;
    f4 kr[DPG];
#pragma unroll
    for (int j = 0; j < DPG; ++j)
        kr[j] = *reinterpret_cast<const f4*>(kt + (int64_t)(DPG * dg + j) * ctx + tk);
    const int dq = tid & 31, g = tid >> 5;               // values: PPG positions, 4 dims
    const float* vc = v_cache + (int64_t)hd * ctx * D;
    f4 vr[PPG];
#pragma unroll
    for (int j = 0; j < PPG; ++j) {
        const int tt = t0 + min(PPG * g + j, len - 1);
        vr[j] = *reinterpret_cast<const f4*>(vc + (int64_t)tt * D + 4 * dq);
    }

    // ---- RoPE of the new query and key, then the reference's (q * scale)
    if (tid < D / 2) {
        qs[2 * tid] = __fmul_rn(__fadd_rn(__fmul_rn(q0, c), __fmul_rn(-q1, sn)), scale);
        qs[2 * tid + 1] = __fmul_rn(__fadd_rn(__fmul_rn(q1, c), __fmul_rn(q0, sn)), scale);
        kn[2 * tid] = __fadd_rn(__fmul_rn(k0, c), __fmul_rn(-k1, sn));
        kn[2 * tid + 1] = __fadd_rn(__fmul_rn(k1, c), __fmul_rn(k0, sn));
    }
    if (tid < D) vn[tid] = v0;
    __syncthreads();
    if (s == S - 1 && tid < D) {  // the tile holding pos appends the new key and value
        k_cache[((int64_t)hd * D + tid) * ctx + pos] = kn[tid];
        v_cache[((int64_t)hd * ctx + pos) * D + tid] = vn[tid];
    }
    // the cache did not hold position pos yet: its key and value come from LDS
    if (pos >= tk && pos < tk + 4) {
        const int i = pos - tk;
#pragma unroll
        for (int j = 0; j < DPG; ++j) {
            const float v = kn[DPG * dg + j];
            kr[j].x = i == 0 ? v : kr[j].x;
            kr[j].y = i == 1 ? v : kr[j].y;
            kr[j].z = i == 2 ? v : kr[j].z;
            kr[j].w = i == 3 ? v : kr[j].w;
        }
    }
    if (s == S - 1) {  // (positions past the tile's end were read as pos too)
        const f4 nv = *reinterpret_cast<const f4*>(vn + 4 * dq);
#pragma unroll
        for (int j = 0; j < PPG; ++j) {
            if (t0 + min(PPG * g + j, len - 1) == pos) vr[j] = nv;
        }
    }

    // ---- scores: this thread's 4 positions over its DPG dimensions
    {
        f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j4 = 0; j4 < DPG / 4; ++j4) {
            const f4 qv = *reinterpret_cast<const f4*>(qs + DPG * dg + 4 * j4);
            acc += qv.x * kr[4 * j4];
            acc += qv.y * kr[4 * j4 + 1];
            acc += qv.z * kr[4 * j4 + 2];
            acc += qv.w * kr[4 * j4 + 3];
        }
        *reinterpret_cast<f4*>(&sc[dg][4 * pq]) = acc;
    }
    __syncthreads();
    if (wave < NW) {  // position tid: its score, the wave's max and sum of exp
        float sv = -INFINITY;
        if (tid < len) {
            sv = 0.f;
#pragma unroll
            for (int k = 0; k < DG; ++k) sv += sc[k][tid];
        }
        const float m = wave_max(sv);
        const float e = tid < len ? __expf(sv - m) : 0.f;
        pl[tid] = e;
        const float l = wave_sum(e);
        if (lane == 0) {
            wm[wave] = m;
            wl[wave] = l;
        }
    }
    __syncthreads();
    // ---- weighted values of this thread's PPG positions, 4 dimensions
    {
        f4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j4 = 0; j4 < PPG / 4; ++j4) {
            const f4 pv = *reinterpret_cast<const f4*>(pl + PPG * g + 4 * j4);
            o += pv.x * vr[4 * j4];
            o += pv.y * vr[4 * j4 + 1];
            o += pv.z * vr[4 * j4 + 2];
            o += pv.w * vr[4 * j4 + 3];
        }
        *reinterpret_cast<f4*>(&oh[g][4 * dq]) = o;
    }
    __syncthreads();
    float* wk = work + ((int64_t)hd * kAttnSplits + s) * (kMaxHeadDim + 2);
    if (tid < D) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, wm[w]);
        float f[NW], L = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            f[w] = wm[w] == -INFINITY ? 0.f : __expf(wm[w] - M);
            L += f[w] * wl[w];
        }
        float O = 0.f;
#pragma unroll
        for (int gg = 0; gg < G; ++gg) O += f[(gg * PPG) / 64] * oh[gg][tid];
        if (S == 1) {
            store_act(out, out_dtype, hd * D + tid, O / L);
        } else {
            put_agent(wk + 2 + tid, O);
            if (tid == 0) {
                put_agent(wk, M);
                put_agent(wk + 1, L);
            }
        }
    }
    if (S == 1) return;
    // ---- more than one tile: the last workgroup of the head merges them
    wait_stores();
    __syncthreads();
    if (tid == 0) {
        last = __hip_atomic_fetch_add(done + hd, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                       (unsigned)(S - 1)
                   ? 1u
                   : 0u;
    }
    __syncthreads();
    if (!last) return;
    constexpr int kT = kMaxCtx / TP;  // tiles a head can have
    const float* base = work + (int64_t)hd * kAttnSplits * (kMaxHeadDim + 2);
    if (tid < D) {
        float mj[kT], lj[kT], oj[kT];
        float M = -INFINITY;
#pragma unroll
        for (int j = 0; j < kT; ++j) {
            const float* pj = base + j * (kMaxHeadDim + 2);
            mj[j] = j < S ? get_agent(pj) : -INFINITY;
            lj[j] = j < S ? get_agent(pj + 1) : 0.f;
            oj[j] = j < S ? get_agent(pj + 2 + tid) : 0.f;
            M = fmaxf(M, mj[j]);
        }
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int j = 0; j < kT; ++j) {
            const float fj = mj[j] == -INFINITY ? 0.f : __expf(mj[j] - M);
            L += fj * lj[j];
            O += fj * oj[j];
        }
        store_act(out, out_dtype, hd * D + tid, O / L);
    }
    if (tid == 0) done[hd] = 0u;  // ready for the next step
}

// ---------------------------------------------------------------------------
// silu(gate) * up
// ---------------------------------------------------------------------------
__global__ void silu_mul_kernel(const float* __restrict__ gu, void* __restrict__ act, int dtype,
                                int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const float g = gu[i];
        const float sg = g / (1.0f + expf(-g));
        store_act(act, dtype, i, sg * gu[n + i]);
    }
}

// ---------------------------------------------------------------------------
// tied LM head, soft cap, greedy argmax, position advance
// ---------------------------------------------------------------------------
// One 1024-thread workgroup per CU (fewer workgroups: fewer same-address
// atomics at the end; 16 waves of 2 rows measured 0.2 % more tokens/s than 8
// waves of 4); a wave takes kHeadRows rows at a time and has all their 16-byte
// pieces of a kHeadSpan-column span in flight together (lane i: pieces i,
// i + 64, ...), against h staged in LDS as fp32.  The argmax key is
// (order-preserving bits of the capped logit) << 32 | (0xffffffff - row),
// so the largest key is the first row with the largest value -- torch's
// argmax -- whatever the order of the atomics.  The last workgroup to
// finish (atomic counter) turns the key into the next token.
constexpr int kHeadThreads = 1024;
constexpr int kHeadMaxC = 8192;
constexpr int kHeadRows = 2;
constexpr int kHeadPieces = 5;                     // per lane and row in one span
constexpr int kHeadSpan = 64 * 8 * kHeadPieces;    // 2560 columns

__device__ __forceinline__ uint32_t orderable(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// kNorm: the head's input is RMSNorm(x) * w of the fp32 residual x, formed
// by every workgroup with add_rmsnorm_kernel's arithmetic (the same
// per-thread sums over the same 1024 threads, the same reduction and
// expressions, rounded to bf16), so the logits are those of the two launches
// add_rmsnorm_kernel + lm_head_argmax_kernel, in one launch.  Otherwise h is
// that bf16 vector.
static_assert(kHeadThreads == kNormThreads, "the fused norm repeats add_rmsnorm_kernel's sums");
template <bool kNorm>
__global__ __launch_bounds__(kHeadThreads) void lm_head_argmax_kernel(
    const bf16_bits* __restrict__ h, const float* __restrict__ x, const float* __restrict__ nw,
    float eps, const bf16_bits* __restrict__ emb, float* __restrict__ logits,
    nb_decode_state* __restrict__ st, int32_t* __restrict__ tokens_out, int tokens_cap,
    const int32_t* __restrict__ force, int n_force, int V, int C) {
    typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
    __shared__ __align__(16) float hs[kHeadMaxC];
    __shared__ unsigned long long wkey[kHeadThreads / 64];
    __shared__ unsigned last;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if constexpr (kNorm) {
        __shared__ float red[kHeadThreads / 64];
        float ss = 0.f;
        for (int i = tid; i < C; i += kHeadThreads) {
            const float v = x[i];
            ss += v * v;
        }
        const float mean = block_sum(ss, red) / (float)C;
        const float norm = sqrtf(mean + eps);
        for (int i = tid; i < C; i += kHeadThreads)
            hs[i] = bf16_to_f32(f32_to_bf16_rne((x[i] / norm) * nw[i]));
    } else {
        for (int i = tid; i < C; i += kHeadThreads) hs[i] = bf16_to_f32(h[i]);
    }
    __syncthreads();
    unsigned long long best = 0ull;
    const int nwaves = gridDim.x * (kHeadThreads / 64);
    for (int r0 = (blockIdx.x * (kHeadThreads / 64) + wave) * kHeadRows; r0 < V;
         r0 += nwaves * kHeadRows) {
        float acc[kHeadRows];
#pragma unroll
        for (int j = 0; j < kHeadRows; ++j) acc[j] = 0.f;
        for (int c0 = 0; c0 < C; c0 += kHeadSpan) {
            u32x4_t v[kHeadRows][kHeadPieces];
#pragma unroll
            for (int j = 0; j < kHeadRows; ++j) {
                const int r = min(r0 + j, V - 1);  // rows past V repeat the last one
#pragma unroll
                for (int q = 0; q < kHeadPieces; ++q) {
                    const int c = min(c0 + (q * 64 + lane) * 8, C - 8);  // past C: unused
                    v[j][q] = __builtin_nontemporal_load(
                        reinterpret_cast<const u32x4_t*>(emb + (int64_t)r * C + c));
                }
            }
#pragma unroll
            for (int q = 0; q < kHeadPieces; ++q) {
                const int c = c0 + (q * 64 + lane) * 8;
                if (c < C) {
                    const float4 h0 = *reinterpret_cast<const float4*>(hs + c);
                    const float4 h1 = *reinterpret_cast<const float4*>(hs + c + 4);
                    const float hv[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
                    for (int j = 0; j < kHeadRows; ++j) {
                        const uint32_t wv[4] = {v[j][q].x, v[j][q].y, v[j][q].z, v[j][q].w};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            acc[j] += hv[2 * e] * __uint_as_float(wv[e] << 16);
                            acc[j] += hv[2 * e + 1] * __uint_as_float(wv[e] & 0xffff0000u);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < kHeadRows; ++j) {
            const int r = r0 + j;
            const float sum = wave_sum(acc[j]);
            const float capped = 30.0f * tanhf(sum / 30.0f);
            if (lane == 0 && r < V) {
                if (logits) logits[r] = capped;
                const unsigned long long key =
                    ((unsigned long long)orderable(capped) << 32) | (0xffffffffu - (uint32_t)r);
                best = key > best ? key : best;
            }
        }
    }
    if (lane == 0) wkey[wave] = best;
    __syncthreads();
    if (tid == 0) {
        unsigned long long b = 0ull;
        for (int w = 0; w < kHeadThreads / 64; ++w) b = wkey[w] > b ? wkey[w] : b;
        atomicMax(&st->key, b);
        wait_stores();  // the max is performed before the count publishes it
        last = atomicAdd(&st->done, 1u) == gridDim.x - 1 ? 1u : 0u;
    }
    __syncthreads();
    if (tid == 0 && last) {
        const unsigned long long key = atomicAdd(&st->key, 0ull);
        const int token = (int)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
        const int step = st->step;
        if (tokens_out && step >= 0 && step < tokens_cap) tokens_out[step] = token;
        st->token = (step >= 0 && step < n_force) ? force[step] : token;
        st->pos += 1;
        st->step += 1;
        st->key = 0ull;
        st->done = 0u;
    }
}

__global__ void zero_u32_kernel(unsigned* __restrict__ p, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0u;
}

// ---------------------------------------------------------------------------
// Scratch of the allocation-free attention entry (nb_attention_step_static):
// the split partials of up to kStaticAttnHeads heads, then one counter per
// head, in a file-scope device array -- one copy on every GPU the library
// runs on, held until the process ends.  Host code never passes the
// array's name to a kernel (on the host it is only a stand-in for the
// symbol): the device address comes from hipGetSymbolAddress, once per
// device, with that device current.
// ---------------------------------------------------------------------------
constexpr int kStaticAttnHeads = 64;
constexpr size_t kStaticAttnWorkBytes =
    (size_t)kStaticAttnHeads * kAttnSplits * (kMaxHeadDim + 2) * sizeof(float);
constexpr size_t kStaticAttnBytes = kStaticAttnWorkBytes + kStaticAttnHeads * sizeof(unsigned);
static __device__ __align__(256) unsigned char scratch[kStaticAttnBytes];

constexpr int kMaxScratchDevices = 64;
unsigned char* g_scratch_ptr[kMaxScratchDevices];
std::mutex g_scratch_mutex;

}  // namespace

int static_attention_max_heads() { return kStaticAttnHeads; }
int64_t static_attention_scratch_bytes() { return (int64_t)kStaticAttnBytes; }

int static_attention_scratch(hipStream_t stream, float** work, unsigned** done) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) {
        return fail(NB_ENODEV, "nb_attention_step_static: no usable current device");
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            return fail(NB_ELAUNCH, "nb_attention_step_static: hipGetSymbolAddress failed: %s",
                        hipGetErrorString(e));
        }
        // the head counters start at zero (every completed call leaves them
        // at zero); cleared by a kernel on the caller's stream, once
        hipLaunchKernelGGL(zero_u32_kernel, dim3(1), dim3(64), 0, stream,
                           reinterpret_cast<unsigned*>(static_cast<unsigned char*>(p) +
                                                       kStaticAttnWorkBytes),
                           kStaticAttnHeads);
        const int st = check_launch("nb_attention_step_static");
        if (st) return st;
        g_scratch_ptr[dev] = static_cast<unsigned char*>(p);
    }
    *work = reinterpret_cast<float*>(g_scratch_ptr[dev]);
    *done = reinterpret_cast<unsigned*>(g_scratch_ptr[dev] + kStaticAttnWorkBytes);
    return NB_OK;
}

int launch_add_rmsnorm(float* x, const float* y, const float* emb, const nb_decode_state* st,
                       const float* w, void* h, int h_dtype, int n, float eps, hipStream_t stream) {
    hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(1), dim3(kNormThreads), 0, stream, x, y, emb, st, w,
                       h, h_dtype, n, eps);
    return check_launch("nb_add_rmsnorm");
}

int launch_attention_step(const float* qkv, float* k_cache, float* v_cache, const float* cos_t,
                          const float* sin_t, const nb_decode_state* st, float* work,
                          unsigned* done, void* out, int out_dtype, int n_head, int head_dim,
                          int ctx, hipStream_t stream) {
    if (head_dim == kTileD && ctx % 4 == 0 && reinterpret_cast<uintptr_t>(k_cache) % 16 == 0 &&
        reinterpret_cast<uintptr_t>(v_cache) % 16 == 0) {
        hipLaunchKernelGGL(attention_tile_kernel<kTilePos>, dim3(n_head, kMaxCtx / kTilePos),
                           dim3(kTileThreads), 0, stream, qkv, k_cache, v_cache, cos_t, sin_t, st,
                           work, done, out, out_dtype, n_head, ctx);
    } else if (head_dim <= kAttn2MaxD) {
        hipLaunchKernelGGL(attention_step2_kernel, dim3(n_head, kAttnSplits), dim3(kAttnThreads),
                           0, stream, qkv, k_cache, v_cache, cos_t, sin_t, st, work, done, out,
                           out_dtype, n_head, head_dim, ctx);
    } else {
        hipLaunchKernelGGL(attention_step_kernel, dim3(n_head, kAttnSplits), dim3(kAttnThreads),
                           0, stream, qkv, k_cache, v_cache, cos_t, sin_t, st, work, done, out,
                           out_dtype, n_head, head_dim, ctx);
    }
    return check_launch("nb_attention_step");
}

int launch_silu_mul(const float* gu, void* act, int dtype, int n, hipStream_t stream) {
    const int blocks = std::min(1024, (n + 255) / 256);
    hipLaunchKernelGGL(silu_mul_kernel, dim3(blocks), dim3(256), 0, stream, gu, act, dtype, n);
    return check_launch("nb_silu_mul");
}

int launch_lm_head_argmax(const void* h, const float* x, const float* norm_w, float eps,
                          const void* emb, float* logits, nb_decode_state* st,
                          int32_t* tokens_out, int tokens_cap, const int32_t* force, int n_force,
                          int V, int C, hipStream_t stream) {
    const int rows_per_block = kHeadRows * (kHeadThreads / 64);
    const int blocks = std::max(1, std::min(device_cu_count(), (V + rows_per_block - 1) / rows_per_block));
    if (x) {
        hipLaunchKernelGGL(lm_head_argmax_kernel<true>, dim3(blocks), dim3(kHeadThreads), 0,
                           stream, nullptr, x, norm_w, eps, static_cast<const bf16_bits*>(emb),
                           logits, st, tokens_out, tokens_cap, force, n_force, V, C);
        return check_launch("nb_rmsnorm_lm_head_argmax");
    }
    hipLaunchKernelGGL(lm_head_argmax_kernel<false>, dim3(blocks), dim3(kHeadThreads), 0, stream,
                       static_cast<const bf16_bits*>(h), nullptr, nullptr, 0.f,
                       static_cast<const bf16_bits*>(emb), logits, st, tokens_out, tokens_cap,
                       force, n_force, V, C);
    return check_launch("nb_lm_head_argmax");
}

int attention_work_floats(int n_head) { return n_head * kAttnSplits * (kMaxHeadDim + 2); }
int attention_max_head_dim() { return kMaxHeadDim; }
int attention_max_ctx() { return kMaxCtx; }
int lm_head_max_c() { return kHeadMaxC; }

}  // namespace nb
