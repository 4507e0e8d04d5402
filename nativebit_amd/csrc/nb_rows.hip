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
constexpr int kNormRegs = 16;      // elements per thread kept in registers (C <= 4096)

__global__ __launch_bounds__(kNormThreads) void rmsnorm_rows_kernel(
    float* __restrict__ x, const float* __restrict__ add, const float* __restrict__ emb,
    const int32_t* __restrict__ tokens, int vocab, const float* __restrict__ w,
    void* __restrict__ h, int h_dtype, int C, float eps) {
    __shared__ float red[kNormThreads / 64];
    const int t = blockIdx.x;
    float* xr = x + (int64_t)t * C;
    const int tok = tokens ? tokens[t] : 0;
    if (tokens && (tok < 0 || tok >= vocab)) {
        // a token outside the table reads nothing: its row of x and h is NaN
        // (the whole workgroup leaves here, before any barrier)
        for (int i = threadIdx.x; i < C; i += kNormThreads) {
            xr[i] = __builtin_nanf("");
            store_out(h, h_dtype, (int64_t)t * C + i, __builtin_nanf(""));
        }
        return;
    }
    const float* src = tokens ? emb + (int64_t)tok * C : nullptr;
    const float* ar = add ? add + (int64_t)t * C : nullptr;
    // rows of up to kNormRegs * 256 elements stay in registers between the
    // sum of squares and the scaling, with every load issued up front
    float ss = 0.f;
    if (C <= kNormRegs * kNormThreads) {
        float v[kNormRegs], wv[kNormRegs];
#pragma unroll
        for (int j = 0; j < kNormRegs; ++j) {
            const int i = threadIdx.x + j * kNormThreads;
            const int ic = i < C ? i : 0;
            v[j] = src ? src[ic] : xr[ic];
            if (ar) v[j] = v[j] + ar[ic];
            wv[j] = w[ic];
        }
#pragma unroll
        for (int j = 0; j < kNormRegs; ++j) {
            const int i = threadIdx.x + j * kNormThreads;
            if (i < C) {
                if (src || ar) xr[i] = v[j];
                ss += v[j] * v[j];
            }
        }
        ss = wsum(ss);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        float tot = 0.f;
        for (int k = 0; k < kNormThreads / 64; ++k) tot += red[k];  // same order everywhere
        const float norm = sqrtf(tot / (float)C + eps);
#pragma unroll
        for (int j = 0; j < kNormRegs; ++j) {
            const int i = threadIdx.x + j * kNormThreads;
            // (x / norm) * w, as generate_torch.py:37
            if (i < C) store_out(h, h_dtype, (int64_t)t * C + i, (v[j] / norm) * wv[j]);
        }
        return;
    }
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
// per query); query t sees positions 0 .. pos0 + t.  Head dims past D (up
// to a multiple of 4) are zero in LDS, so the dot products run over float4
// pieces and add exact zeros.
// ---------------------------------------------------------------------------
constexpr int kQB = 8;        // queries per workgroup (32 threads each)
constexpr int kKT = 64;       // keys per tile
constexpr int kAttThreads = 256;
constexpr int kRowsMaxD = 128;
constexpr int kQPitch = kRowsMaxD + 4;   // floats per LDS row of q and v (16-byte rows)
constexpr int kKPitch = kKT + 4;         // floats per LDS row of k (one head dim)

__global__ __launch_bounds__(kAttThreads) void attention_rows_kernel(
    const float* __restrict__ q, const float* __restrict__ k_cache,
    const float* __restrict__ v_cache, int pos0, int T, void* __restrict__ out, int out_dtype,
    int n_head, int D, int ctx) {
    typedef __attribute__((ext_vector_type(4))) float f4;
    __shared__ __align__(16) float qs[kQB][kQPitch];
    __shared__ __align__(16) float ks[kRowsMaxD][kKPitch];   // keys transposed: [dim][position]
    __shared__ __align__(16) float vs[kKT][kQPitch];
    __shared__ __align__(16) float ps[kQB][kKPitch];
    const int hd = blockIdx.x, t0 = blockIdx.y * kQB;
    const int tid = threadIdx.x;
    const int C = n_head * D;
    const int D4 = (D + 3) & ~3;
    const int nq = min(kQB, T - t0);
    for (int e = tid; e < kQB * kQPitch; e += kAttThreads) {
        const int i = e / kQPitch, d = e - i * kQPitch;
        qs[i][d] = i < nq && d < D ? q[(int64_t)(t0 + i) * C + hd * D + d] : 0.f;
    }
    typedef __attribute__((ext_vector_type(2))) float f2;
    // scores: thread (sq, sp) takes query sq and keys 2 sp, 2 sp + 1
    const int sq = tid >> 5, sp = tid & 31;
    // weighted values: thread (oq, og) takes query oq and dims 4 og .. 4 og + 3
    const int oq = tid >> 5, og = tid & 31;
    f4 o0 = {0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f;  // per query, kept by its 32 threads alike
    const int last = pos0 + t0 + nq - 1;  // the last position any query sees
    const float* kt = k_cache + (int64_t)hd * D * ctx;
    const float* vc = v_cache + (int64_t)hd * ctx * D;
    for (int p0 = 0; p0 <= last; p0 += kKT) {
        const int np = min(kKT, last + 1 - p0);
        __syncthreads();  // the previous tile is no longer read
        // the tile's keys and values, all loads of a thread issued together
        float kv[kRowsMaxD * kKT / kAttThreads], vv[kRowsMaxD * kKT / kAttThreads];
#pragma unroll
        for (int j = 0; j < kRowsMaxD * kKT / kAttThreads; ++j) {
            const int e = tid + j * kAttThreads;
            const int d = e / kKT, p = e % kKT;            // keys: position fastest
            kv[j] = d < D && p < np ? kt[(int64_t)d * ctx + p0 + p] : 0.f;
            const int pv = e / kRowsMaxD, dv = e % kRowsMaxD;  // values: dim fastest
            vv[j] = dv < D && pv < np ? vc[(int64_t)(p0 + pv) * D + dv] : 0.f;
        }
#pragma unroll
        for (int j = 0; j < kRowsMaxD * kKT / kAttThreads; ++j) {
            const int e = tid + j * kAttThreads;
            ks[e / kKT][e % kKT] = kv[j];
            vs[e / kRowsMaxD][e % kRowsMaxD] = vv[j];
        }
        __syncthreads();
        // scores of this tile, masked past each query's own position
        f2 acc = {0.f, 0.f};
        for (int d = 0; d < D4; d += 4) {
            const f4 qv = *reinterpret_cast<const f4*>(&qs[sq][d]);
            const f2 k0 = *reinterpret_cast<const f2*>(&ks[d][2 * sp]);
            const f2 k1 = *reinterpret_cast<const f2*>(&ks[d + 1][2 * sp]);
            const f2 k2 = *reinterpret_cast<const f2*>(&ks[d + 2][2 * sp]);
            const f2 k3 = *reinterpret_cast<const f2*>(&ks[d + 3][2 * sp]);
            acc += qv.x * k0;   // head dims in order for every score
            acc += qv.y * k1;
            acc += qv.z * k2;
            acc += qv.w * k3;
        }
        float s[2] = {acc.x, acc.y};
        float tmax = -INFINITY;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int p = 2 * sp + j;
            const bool ok = sq < nq && p < np && p0 + p <= pos0 + t0 + sq;
            s[j] = ok ? s[j] : -INFINITY;
            tmax = fmaxf(tmax, s[j]);
        }
        // the 32 threads of a query (consecutive lanes, two rows of 16)
        // agree on its tile max
        tmax = row16_max(tmax);
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
        const float m_new = fmaxf(m_run, tmax);
        const float alpha = m_new == -INFINITY ? 1.f : __expf(m_run - m_new);
        float lsum = 0.f;
        f2 e2;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const float e = s[j] == -INFINITY ? 0.f : __expf(s[j] - m_new);
            e2[j] = e;
            lsum += e;
        }
        *reinterpret_cast<f2*>(&ps[sq][2 * sp]) = e2;
        lsum = row16_sum(lsum);
        lsum += __shfl_xor(lsum, 16);
        l_run = l_run * alpha + lsum;
        m_run = m_new;
        __syncthreads();
        o0 *= alpha;
        for (int p = 0; p < np; ++p) {
            o0 += ps[oq][p] * *reinterpret_cast<const f4*>(&vs[p][4 * og]);
        }
    }
    if (oq < nq) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int d = 4 * og + j;
            if (d < D) store_out(out, out_dtype, (int64_t)(t0 + oq) * C + hd * D + d, o0[j] / l_run);
        }
    }
}

}  // namespace

int launch_rmsnorm_rows(float* x, const float* add, const float* emb, const int32_t* tokens,
                        int vocab, const float* w, void* h, int h_dtype, int T, int C, float eps,
                        hipStream_t stream) {
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(T), dim3(kNormThreads), 0, stream, x, add, emb,
                       tokens, vocab, w, h, h_dtype, C, eps);
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
