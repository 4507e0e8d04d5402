// Kernels of a batched forward pass over T tokens (the prompt pass of the
// packed decoder, gfx950), everything but the packed matmuls (those are the
// prefill GEMMs):
//
//   nb_rmsnorm_rows     per row: x = embedding[token] or x += add; then
//                       h = rmsnorm(x) * w   (generate_torch.py:29-38, 128-132, 150)
//   nb_silu_pairs_rows  act = silu(gate) * up from (gate, up) column pairs
//                       (generate_torch.py:116-117)
//   nb_rope_kv_rows     RoPE of q and k at positions pos0 .. pos0 + T - 1, k and v
//                       appended to the caches, q * D^-0.5 kept for attention
//                       (generate_torch.py:48-60, 80-88)
//   nb_attention_rows   causal attention of T queries over cache positions
//                       0 .. pos0 + t (generate_torch.py:89-98)
//
// Arithmetic is fp32; outputs that feed a packed matmul may be rounded to
// bf16 (nearest even).  The cache layout is the decode step's: keys
// transposed [n_head][D][ctx], values [n_head][ctx][D].
#include <math.h>

#include "nb_device.h"
#include "nb_internal.h"

namespace nb {
namespace {

__device__ __forceinline__ void store_out(void* p, int dtype, int64_t i, float v) {
    if (dtype == NB_BF16) {
        static_cast<bf16_bits*>(p)[i] = f32_to_bf16_rne(v);
    } else {
        static_cast<float*>(p)[i] = v;
    }
}

__device__ __forceinline__ float wsum(float v) { return wave64_sum(v); }

// ---------------------------------------------------------------------------
// rmsnorm of T rows, one workgroup per row
// ---------------------------------------------------------------------------
constexpr int kNormThreads = 256;

__global__ __launch_bounds__(kNormThreads) void rmsnorm_rows_kernel(
    float* __restrict__ x, const float* __restrict__ add, const float* __restrict__ emb,
    const int32_t* __restrict__ tokens, const float* __restrict__ w, void* __restrict__ h,
    int h_dtype, int C, float eps) {
    __shared__ float red[kNormThreads / 64];
    const int t = blockIdx.x;
    float* xr = x + (int64_t)t * C;
    const float* src = tokens ? emb + (int64_t)tokens[t] * C : nullptr;
    const float* ar = add ? add + (int64_t)t * C : nullptr;
    float ss = 0.f;
    for (int i = threadIdx.x; i < C; i += kNormThreads) {
        float v = src ? src[i] : xr[i];
        if (ar) v = v + ar[i];
        if (src || ar) xr[i] = v;
        ss += v * v;
    }
    ss = wsum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int k = 0; k < kNormThreads / 64; ++k) tot += red[k];  // same order everywhere
    const float norm = sqrtf(tot / (float)C + eps);
    for (int i = threadIdx.x; i < C; i += kNormThreads) {
        // (x / norm) * w, as generate_torch.py:37
        store_out(h, h_dtype, (int64_t)t * C + i, (xr[i] / norm) * w[i]);
    }
}

// ---------------------------------------------------------------------------
// silu(gate) * up from interleaved columns
// ---------------------------------------------------------------------------
__global__ void silu_pairs_rows_kernel(const float* __restrict__ gu, void* __restrict__ act,
                                       int act_dtype, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const float g = gu[2 * i], u = gu[2 * i + 1];
        store_out(act, act_dtype, i, (g / (1.0f + __expf(-g))) * u);
    }
}

// ---------------------------------------------------------------------------
// RoPE + cache append for T tokens: grid (T, n_head), D/2 threads (<= 128)
// ---------------------------------------------------------------------------
__global__ void rope_kv_rows_kernel(const float* __restrict__ qkv, float* __restrict__ k_cache,
                                    float* __restrict__ v_cache, const float* __restrict__ cos_t,
                                    const float* __restrict__ sin_t, int pos0,
                                    float* __restrict__ q_out, int n_head, int D, int ctx) {
    const int t = blockIdx.x, hd = blockIdx.y;
    const int pos = pos0 + t;
    const int C = n_head * D, half = D / 2;
    const float scale = 1.0f / sqrtf((float)D);
    const float* row = qkv + (int64_t)t * 3 * C;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        const float c = cos_t[(int64_t)pos * half + i], s = sin_t[(int64_t)pos * half + i];
        const float q0 = row[hd * D + 2 * i], q1 = row[hd * D + 2 * i + 1];
        const float k0 = row[C + hd * D + 2 * i], k1 = row[C + hd * D + 2 * i + 1];
        // x * cos2 + rotate(x) * sin2 (generate_torch.py:54-59), q then * scale
        float* qo = q_out + (int64_t)t * C + hd * D;
        qo[2 * i] = __fmul_rn(__fadd_rn(__fmul_rn(q0, c), __fmul_rn(-q1, s)), scale);
        qo[2 * i + 1] = __fmul_rn(__fadd_rn(__fmul_rn(q1, c), __fmul_rn(q0, s)), scale);
        k_cache[((int64_t)hd * D + 2 * i) * ctx + pos] = __fadd_rn(__fmul_rn(k0, c),
                                                                   __fmul_rn(-k1, s));
        k_cache[((int64_t)hd * D + 2 * i + 1) * ctx + pos] = __fadd_rn(__fmul_rn(k1, c),
                                                                       __fmul_rn(k0, s));
    }
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        v_cache[((int64_t)hd * ctx + pos) * D + d] = row[2 * C + hd * D + d];
    }
}

// ---------------------------------------------------------------------------
// causal attention of T queries: grid (n_head, ceil(T / kQB)), 256 threads.
// The workgroup holds kQB queries of one head and walks the keys in tiles
// of kKT positions through LDS with an online softmax (running max and sum
// per query); query t sees positions 0 .. pos0 + t.
// ---------------------------------------------------------------------------
constexpr int kQB = 16;       // queries per workgroup
constexpr int kKT = 64;       // keys per tile
constexpr int kAttThreads = 256;
constexpr int kRowsMaxD = 128;

__global__ __launch_bounds__(kAttThreads) void attention_rows_kernel(
    const float* __restrict__ q, const float* __restrict__ k_cache,
    const float* __restrict__ v_cache, int pos0, int T, void* __restrict__ out, int out_dtype,
    int n_head, int D, int ctx) {
    __shared__ float qs[kQB][kRowsMaxD + 1];
    __shared__ float ks[kRowsMaxD][kKT + 1];
    __shared__ float vs[kKT][kRowsMaxD + 1];
    __shared__ float ps[kQB][kKT + 1];
    const int hd = blockIdx.x, t0 = blockIdx.y * kQB;
    const int tid = threadIdx.x;
    const int C = n_head * D;
    const int nq = min(kQB, T - t0);
    for (int e = tid; e < kQB * D; e += kAttThreads) {
        const int i = e / D, d = e - i * D;
        qs[i][d] = i < nq ? q[(int64_t)(t0 + i) * C + hd * D + d] : 0.f;
    }
    // scores: thread (sq, sp) takes query sq and keys sp, sp + 16, sp + 32, sp + 48
    const int sq = tid >> 4, sp = tid & 15;
    // weighted values: thread (oq, og) takes query oq and dims og, og + 16, ...
    const int oq = tid >> 4, og = tid & 15;
    constexpr int kDPer = kRowsMaxD / 16;
    float o[kDPer];
#pragma unroll
    for (int j = 0; j < kDPer; ++j) o[j] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;  // per query, kept by its 16 threads alike
    const int last = pos0 + t0 + nq - 1;  // the last position any query sees
    const float* kt = k_cache + (int64_t)hd * D * ctx;
    const float* vc = v_cache + (int64_t)hd * ctx * D;
    for (int p0 = 0; p0 <= last; p0 += kKT) {
        const int np = min(kKT, last + 1 - p0);
        __syncthreads();  // the previous tile is no longer read
        for (int e = tid; e < D * kKT; e += kAttThreads) {
            const int d = e / kKT, p = e - d * kKT;
            ks[d][p] = p < np ? kt[(int64_t)d * ctx + p0 + p] : 0.f;
        }
        for (int e = tid; e < kKT * D; e += kAttThreads) {
            const int p = e / D, d = e - p * D;
            vs[p][d] = p < np ? vc[(int64_t)(p0 + p) * D + d] : 0.f;
        }
        __syncthreads();
        // scores of this tile, masked past each query's own position
        float s[4];
        float tmax = -INFINITY;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int p = sp + 16 * j;
            float acc = 0.f;
            for (int d = 0; d < D; ++d) acc += qs[sq][d] * ks[d][p];
            const bool ok = sq < nq && p < np && p0 + p <= pos0 + t0 + sq;
            s[j] = ok ? acc : -INFINITY;
            tmax = fmaxf(tmax, s[j]);
        }
        // the 16 threads of a query (consecutive lanes) agree on its tile max
        tmax = row16_max(tmax);
        const float m_new = fmaxf(m_run, tmax);
        const float alpha = m_new == -INFINITY ? 1.f : __expf(m_run - m_new);
        float lsum = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float e = s[j] == -INFINITY ? 0.f : __expf(s[j] - m_new);
            ps[sq][sp + 16 * j] = e;
            lsum += e;
        }
        lsum = row16_sum(lsum);
        l_run = l_run * alpha + lsum;
        m_run = m_new;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kDPer; ++j) {
            const int d = og + 16 * j;
            float acc = o[j] * alpha;
            if (d < D) {
                for (int p = 0; p < np; ++p) acc += ps[oq][p] * vs[p][d];
            }
            o[j] = acc;
        }
    }
    if (oq < nq) {
#pragma unroll
        for (int j = 0; j < kDPer; ++j) {
            const int d = og + 16 * j;
            if (d < D) store_out(out, out_dtype, (int64_t)(t0 + oq) * C + hd * D + d, o[j] / l_run);
        }
    }
}

}  // namespace

int launch_rmsnorm_rows(float* x, const float* add, const float* emb, const int32_t* tokens,
                        const float* w, void* h, int h_dtype, int T, int C, float eps,
                        hipStream_t stream) {
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(T), dim3(kNormThreads), 0, stream, x, add, emb,
                       tokens, w, h, h_dtype, C, eps);
    return check_launch("nb_rmsnorm_rows");
}

int launch_silu_pairs_rows(const float* gu, void* act, int act_dtype, int T, int F,
                           hipStream_t stream) {
    const int64_t n = (int64_t)T * F;
    const int blocks = (int)std::min<int64_t>(4096, (n + 255) / 256);
    hipLaunchKernelGGL(silu_pairs_rows_kernel, dim3(blocks), dim3(256), 0, stream, gu, act,
                       act_dtype, n);
    return check_launch("nb_silu_pairs_rows");
}

int launch_rope_kv_rows(const float* qkv, float* k_cache, float* v_cache, const float* cos_t,
                        const float* sin_t, int pos0, int T, float* q_out, int n_head, int D,
                        int ctx, hipStream_t stream) {
    hipLaunchKernelGGL(rope_kv_rows_kernel, dim3(T, n_head), dim3(64), 0, stream, qkv, k_cache,
                       v_cache, cos_t, sin_t, pos0, q_out, n_head, D, ctx);
    return check_launch("nb_rope_kv_rows");
}

int launch_attention_rows(const float* q, const float* k_cache, const float* v_cache, int pos0,
                          int T, void* out, int out_dtype, int n_head, int D, int ctx,
                          hipStream_t stream) {
    hipLaunchKernelGGL(attention_rows_kernel, dim3(n_head, (T + kQB - 1) / kQB),
                       dim3(kAttThreads), 0, stream, q, k_cache, v_cache, pos0, T, out,
                       out_dtype, n_head, D, ctx);
    return check_launch("nb_attention_rows");
}

int attention_rows_max_head_dim() { return kRowsMaxD; }

}  // namespace nb
