// Persistent greedy decode of the packed NativeBit decoder on gfx950:
// n_steps tokens in one cooperative launch of one workgroup per CU.
//
// The model is the reference's PackedGPT (inference/generate_torch.py:
// 135-162): per layer RMSNorm -> q|k|v -> RoPE + causal attention with a KV
// cache -> out_proj -> residual -> RMSNorm -> gate|up -> silu(gate) * up ->
// down -> residual, then the final RMSNorm, the tied head with the 30 tanh
// soft cap and the greedy argmax (generate_torch.py:157-159, 298-313).
//
// A token is a fixed sequence of phases separated by grid barriers:
//
//   per layer:  QKV  (prologue: rmsnorm(x) or the embedding row; y -> qkv)
//               ATT  (RoPE, KV append, split softmax attention -> att)
//               O    (prologue: att;                 epilogue: x += y)
//               GU   (prologue: rmsnorm(x);          y -> gu)
//               DOWN (prologue: silu(gate) * up;     epilogue: x += y)
//   then        HEAD (prologue: rmsnorm(x); tied head, soft cap, argmax)
//
// Workgroup.  Eleven streaming waves and one control wave.  The packed GEMV
// phases are streamed by the streaming waves in chunks of R = 64 / bpr
// whole rows (bpr = 128-weight blocks per row), so no row is shared between
// chunks, waves or workgroups: lane l of a chunk takes block l, forms its
// dot product with the staged activations (nb_stream_common.h) and the
// lanes of a row are summed in block order -- deterministic, independent of
// scheduling.  Chunks of a phase are split evenly over the workgroups; in
// a workgroup the waves take them from an LDS counter.
//
// Prefetch across barriers.  Each streaming wave keeps two chunk slots in
// LDS filled by direct-to-LDS loads, and its load cursor runs through the
// GEMV phases of the whole sequence: the packed weights do not depend on
// the activations, so while a phase waits for the grid barrier the loads
// of the next phases' chunks are already in flight.  The streaming waves
// therefore never wait for their own global stores at a barrier (on gfx9
// that wait would also drain their prefetch): their GEMV results go to LDS
// and the control wave writes them out, waits for its stores and takes part
// in the grid barrier.
//
// Grid barrier.  Two levels of agent-scope atomic counters: the workgroups
// of group g % 8 count on their group's counter, the last of each group
// counts on the top counter, everyone polls the top counter (about 2.3 us
// on MI355X, against about 4 us for one flat counter).  Values that cross
// workgroups are written with agent-scope stores and read with agent-scope
// loads (coherent across the XCDs' L2 caches) after the barrier.  Every wait
// is bounded: a barrier that does not complete within the spin limit sets
// the error word of the workspace, and every workgroup then leaves.
//
// Numerics are those of the launch-per-kernel decode step (nb_decode.hip
// and the batched GEMV): fp32 residual stream, norms, attention and KV
// cache; bf16 activations into the packed GEMVs with bf16-rounded codebook
// entries and fp32 accumulation; bf16 tied head.
#include <math.h>

#include <algorithm>

#include "nb_device.h"
#include "nb_internal.h"
#include "nb_stream_common.h"

namespace nb {
namespace {

using namespace stream;

constexpr int kSWaves = 11;                  // streaming waves
constexpr int kCtl = kSWaves;                // the control wave
constexpr int kThreads = 64 * (kSWaves + 1);
constexpr int kDepth = 2;                    // chunk slots per streaming wave
constexpr int kChunkMax = 64;                // blocks per chunk (one per lane)
constexpr int kIdxSlot = kChunkMax * 48;     // 3 KiB of indices
constexpr int kSlotBytes = kChunkMax * 80;   // + 2 KiB of codebook
constexpr int kLoadsPerChunk = 5;            // 1 KiB each
constexpr int kMaxBpr = 64;
constexpr int kXStage = kMaxBpr * kXColBytes;
constexpr int kTmpBytes = 16384;
constexpr int kYMax = 1024;                  // GEMV outputs of one workgroup per phase
constexpr int kCntWindow = 32;               // chunk counters: GEMV phase id mod 32
constexpr int kSplitLen = 16;                // positions per attention split
constexpr int kMaxSplits = 64;               // splits per head (one per lane in the combine)
constexpr int kMaxD = 128;
constexpr int kMaxC = kTmpBytes / 4;
constexpr int kMaxF = kMaxBpr * 128;
constexpr int kAttScratch = (3 * kMaxD + kMaxSplits) * 4;  // per streaming wave
constexpr int kPerThreadC = (kMaxC + 64 * 12 - 1) / (64 * 12);  // prologue elements per thread
constexpr int kPerThreadF = (kMaxF + 64 * 12 - 1) / (64 * 12);
constexpr int kHeadPieces = (kMaxC + 511) / 512;                // 16-byte pieces of a head row per lane

// LDS layout
constexpr int kOffRing = 0;
constexpr int kOffX = kOffRing + kSWaves * kDepth * kSlotBytes;
constexpr int kOffTmp = kOffX + kXStage;  // tmp follows the staged x (attention uses both)
constexpr int kOffY = kOffTmp + kTmpBytes;
constexpr int kOffCnt = kOffY + kYMax * 4;
constexpr int kOffMisc = kOffCnt + kCntWindow * 4;
constexpr int kMaxLayers = 64;
constexpr int kOffGeo = kOffMisc + 256;   // KGeo of the four GEMV kinds
constexpr int kOffLane = kOffGeo + 128;   // per kind and lane: row, column block
constexpr int kOffPtab = kOffLane + 512;  // [layer][kind] stream and codebook pointers
constexpr int kOffArgs = kOffPtab + kMaxLayers * 8 * 8;  // the kernel arguments
constexpr int kLdsBytes = kOffArgs + 256;
static_assert(kSWaves * kAttScratch <= kXStage + kTmpBytes, "attention scratch");
static_assert(kSWaves * 64 * 4 <= kTmpBytes, "row-sum scratch");
static_assert(kLdsBytes <= 160 * 1024, "LDS");

enum Kind { kQKV = 0, kO = 1, kGU = 2, kDown = 3 };

// Byte offsets inside the control block (the workspace's first kCtlBytes):
// group counters 256 bytes apart, the top counter, the error word, the
// attention split counters.
constexpr int kCtlBytes = 4096;
constexpr int kCtlTop = 8 * 64;      // in uint32 units
constexpr int kCtlErr = 9 * 64;
constexpr int kCtlDone = 10 * 64;
constexpr int kMaxHeads = (kCtlBytes / 4 - kCtlDone);

struct PArgs {
    const nb_decode_layer* layers;
    const float* ln_f;
    const float* emb_f32;
    const bf16_bits* emb_bf16;
    const float* cos_t;
    const float* sin_t;
    float* xres;      // C   residual stream
    float* qkv;       // 3C
    uint32_t* att;    // C/2 bf16 pairs
    float* gu;        // 2F
    float* awork;     // attention partials [H][kMaxSplits][kMaxD + 2]
    unsigned* ctl;    // control block
    nb_decode_state* st;
    float* logits;
    int32_t* tokens_out;
    const int32_t* force;
    int tokens_cap, n_force;
    int L, C, H, D, F, V, ctx, n_steps;
    float eps;
    int spin_limit;
};
static_assert(sizeof(PArgs) <= 256, "arguments in LDS");

// ---------------------------------------------------------------------------
// small helpers
// ---------------------------------------------------------------------------
// Agent-scope (all XCDs) relaxed accesses through global-address-space
// pointers: a generic pointer would give flat_* instructions, which also
// count on lgkmcnt, so every LDS wait would wait for global memory too.
__device__ __forceinline__ float ld_agent(const float* p) {
    return __hip_atomic_load(as_global_mut(const_cast<float*>(p)), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_agent_u(const uint32_t* p) {
    return __hip_atomic_load(as_global_mut(const_cast<uint32_t*>(p)), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(float* p, float v) {
    __hip_atomic_store(as_global_mut(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent_u(uint32_t* p, uint32_t v) {
    __hip_atomic_store(as_global_mut(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t add_agent(uint32_t* p, uint32_t v) {
    return __hip_atomic_fetch_add(as_global_mut(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T ld_g(const T* p) {
    return *as_global(p);
}

// LDS pointers with their address space spelled out: 32-bit ds addresses
// the compiler cannot lose (a generic pointer kept live across the
// streaming loop is 64 bits and was spilled, its reload waiting on vmcnt).
#define LDS3 __attribute__((address_space(3)))
template <typename T>
__device__ __forceinline__ LDS3 T* lds_at(int off) {
    extern __shared__ __align__(16) unsigned char smem[];
    return (LDS3 T*)((LDS3 unsigned char*)smem + off);
}

// Workgroup barrier that waits for this wave's LDS operations only -- not
// for its vector-memory loads, which would drain the prefetch.
__device__ __forceinline__ void wg_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory");
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ uint32_t orderable(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Geometry of one GEMV kind: rows N, blocks per row, rows per chunk R,
// blocks per full chunk, and this workgroup's chunk range [c0, c1).
struct KGeo {
    int N, bpr, R, nbk, c0, c1;
};
// field-wise copies in and out of LDS (a struct copy through an
// address-space-qualified pointer is not allowed)
__device__ __forceinline__ KGeo kgeo_get(const __attribute__((address_space(3))) KGeo* p) {
    KGeo k;
    k.N = p->N;
    k.bpr = p->bpr;
    k.R = p->R;
    k.nbk = p->nbk;
    k.c0 = p->c0;
    k.c1 = p->c1;
    return k;
}
__device__ __forceinline__ void kgeo_put(__attribute__((address_space(3))) KGeo* p, const KGeo& k) {
    p->N = k.N;
    p->bpr = k.bpr;
    p->R = k.R;
    p->nbk = k.nbk;
    p->c0 = k.c0;
    p->c1 = k.c1;
}

// The layer table is read through the constant address space with a
// uniform index, so the reads are scalar loads (counted on lgkmcnt): a
// vector load would make the compiler wait on vmcnt, draining the ring.
typedef const __attribute__((address_space(4))) nb_decode_layer* layer_cptr;
__device__ __forceinline__ layer_cptr layer_at(const nb_decode_layer* layers, int l) {
    return (layer_cptr)(layers) + __builtin_amdgcn_readfirstlane(l);
}

__device__ __forceinline__ const uint8_t* packed_of(layer_cptr L, int kind) {
    return kind == kQKV ? L->qkv_packed : kind == kO ? L->o_packed
                                                     : kind == kGU ? L->gu_packed : L->down_packed;
}
__device__ __forceinline__ const float* codebook_of(layer_cptr L, int kind) {
    return kind == kQKV ? L->qkv_codebook : kind == kO ? L->o_codebook
                                                       : kind == kGU ? L->gu_codebook
                                                                     : L->down_codebook;
}

// Two-level grid barrier, called by lane 0 of the control wave.  k counts
// this workgroup's barriers.  Returns false when the wait ran past the spin
// limit or another workgroup reported an error.
__device__ bool grid_barrier(unsigned* ctl, unsigned k, int g, int G, int spin_limit) {
    const int ng = G < 8 ? G : 8;
    const int grp = g % ng;
    const unsigned gsize = (unsigned)((G - grp + ng - 1) / ng);
    if (add_agent(ctl + 64 * grp, 1u) == k * gsize - 1u) add_agent(ctl + kCtlTop, 1u);
    int n = 0;
    while (ld_agent_u(ctl + kCtlTop) < k * (unsigned)ng) {
        __builtin_amdgcn_s_sleep(2);
        if (ld_agent_u(ctl + kCtlErr) != 0u || ++n > spin_limit) {
            st_agent_u(ctl + kCtlErr, 1u);
            return false;
        }
    }
    return true;
}

// ---------------------------------------------------------------------------
// the phases' work outside the streaming loop
// ---------------------------------------------------------------------------
// The prologue helpers run out of line (noinline) and attention and head
// inline; either way the streaming loop must keep its registers: a spill
// reload there waits on vmcnt and drains the ring.  Each function reaches
// the dynamic LDS through its own extern declaration.

// LDS views of the regions (the dynamic shared array of the launch).
#define NB_SMEM extern __shared__ __align__(16) unsigned char smem[]
#define NB_ARGS reinterpret_cast<const PArgs*>(smem + kOffArgs)

// h = (x / sqrt(mean(x^2) + eps)) * w (generate_torch.py:29-38) for the
// C-wide x (agent-coherent, or the embedding row), into LDS tmp: as bf16
// (to be staged) or as the bf16-rounded value in fp32 (the head).  Every
// thread takes elements tid + kThreads j and issues all its loads before
// using any.  All threads call it (one workgroup barrier inside).
__device__ __noinline__ void norm_to_tmp(const float* src, bool coherent, const float* w,
                                         bool as_f32, int tid) {
    NB_SMEM;
    const PArgs* A = NB_ARGS;
    float* tmp = reinterpret_cast<float*>(smem + kOffTmp);
    bf16_bits* tmph = reinterpret_cast<bf16_bits*>(smem + kOffTmp);
    float* red = reinterpret_cast<float*>(smem + kOffMisc);
    const int C = A->C, lane = tid & 63, wave = tid >> 6;
    float v[kPerThreadC], wv[kPerThreadC];
#pragma unroll
    for (int j = 0; j < kPerThreadC; ++j) {
        const int i = tid + kThreads * j;
        v[j] = i < C ? (coherent ? ld_agent(src + i) : ld_g(src + i)) : 0.f;
        wv[j] = i < C ? ld_g(w + i) : 0.f;
    }
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < kPerThreadC; ++j) ss += v[j] * v[j];
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    wg_barrier();
    float t = 0.f;
    for (int w2 = 0; w2 <= kCtl; ++w2) t += red[w2];
    const float norm = sqrtf(t / (float)C + A->eps);
#pragma unroll
    for (int j = 0; j < kPerThreadC; ++j) {
        const int i = tid + kThreads * j;
        if (i < C) {
            const float h = (v[j] / norm) * wv[j];
            if (as_f32) {
                tmp[i] = round_bf16(h);
            } else {
                tmph[i] = f32_to_bf16_rne(h);
            }
        }
    }
}

// The attention output (bf16 pairs, agent-coherent) into LDS tmp.
__device__ __noinline__ void att_to_tmp(int tid) {
    NB_SMEM;
    const PArgs* A = NB_ARGS;
    uint32_t* t32 = reinterpret_cast<uint32_t*>(smem + kOffTmp);
    const int n = A->C / 2;
    const uint32_t* att = uniform_ptr(A->att);
    uint32_t v[kPerThreadC];
#pragma unroll
    for (int j = 0; j < kPerThreadC; ++j) {
        const int i = tid + kThreads * j;
        v[j] = i < n ? ld_agent_u(att + i) : 0u;
    }
#pragma unroll
    for (int j = 0; j < kPerThreadC; ++j) {
        const int i = tid + kThreads * j;
        if (i < n) t32[i] = v[j];
    }
}

// silu(gate) * up (generate_torch.py:116-117), rounded to bf16, into LDS tmp.
__device__ __noinline__ void silu_to_tmp(int tid) {
    NB_SMEM;
    const PArgs* A = NB_ARGS;
    bf16_bits* tmph = reinterpret_cast<bf16_bits*>(smem + kOffTmp);
    const int F = A->F;
    const float* gu = uniform_ptr(A->gu);
    float gv[kPerThreadF], uv[kPerThreadF];
#pragma unroll
    for (int j = 0; j < kPerThreadF; ++j) {
        const int i = tid + kThreads * j;
        gv[j] = i < F ? ld_agent(gu + i) : 0.f;
        uv[j] = i < F ? ld_agent(gu + F + i) : 0.f;
    }
#pragma unroll
    for (int j = 0; j < kPerThreadF; ++j) {
        const int i = tid + kThreads * j;
        if (i < F) {
            const float sg = gv[j] / (1.0f + expf(-gv[j]));
            tmph[i] = f32_to_bf16_rne(sg * uv[j]);
        }
    }
}

// The staged activations (selector order, nb_stream_common.h) of the
// K-wide bf16 vector in LDS tmp.
__device__ __noinline__ void stage_from_tmp(int K, int tid) {
    NB_SMEM;
    const bf16_bits* tmph = reinterpret_cast<const bf16_bits*>(smem + kOffTmp);
    unsigned char* xstage = smem + kOffX;
    const int bpr = K >> 7;
    for (int q = tid; q < bpr * 4; q += kThreads) {
        const int c = q >> 2, u = q & 3;
        const u32x4_t* p = reinterpret_cast<const u32x4_t*>(tmph + c * 128 + u * 32);
        uint32_t w[16];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const u32x4_t t = p[v];
            w[4 * v] = t.x;
            w[4 * v + 1] = t.y;
            w[4 * v + 2] = t.z;
            w[4 * v + 3] = t.w;
        }
        stage_unit(xstage + c * kXColBytes, u, w);
    }
}

// Attention for the new token at position pos (one wave per item).
// Item (head h, split s) takes kSplitLen positions [t0, t1) of 0..pos.
// Scores: lane 16 qd + p takes position t0 + p and the head dimensions of
// quarter qd, so one batch of loads brings the item's keys; the quarters
// are summed by a fixed butterfly.  Values: lane l takes dimensions 2l,
// 2l + 1 of every position.  The split holding pos rotates the new key,
// appends key and value to the caches and uses them directly.  The last
// split of a head to finish (counter) combines the splits in split order.
__device__ __forceinline__ void attention_items(int layer, int pos, int g, int G, int wave,
                                             int lane) {
    NB_SMEM;
    const PArgs* A = NB_ARGS;
    const int C = A->C, H = A->H, D = A->D, ctx = A->ctx;
    const int n = pos + 1;
    const int S = (n + kSplitLen - 1) / kSplitLen;
    const float scale = 1.0f / sqrtf((float)D);
    const int half = D >> 1;
    const int dq = D >> 2;  // dimensions per quarter
    float* qs = reinterpret_cast<float*>(smem + kOffX) + wave * (kAttScratch / 4);
    float* kn = qs + kMaxD;
    float* vn = kn + kMaxD;
    float* pw = vn + kMaxD;  // probabilities of the split, then the split weights
    const layer_cptr Ly = layer_at(A->layers, layer);
    float* kt_all = uniform_ptr(Ly->k_cache);
    float* vc_all = uniform_ptr(Ly->v_cache);
    const float* qkv = uniform_ptr(A->qkv);
    const float* cos_t = uniform_ptr(A->cos_t);
    const float* sin_t = uniform_ptr(A->sin_t);
    float* awork = uniform_ptr(A->awork);
    unsigned* ctl = uniform_ptr(A->ctl);
    uint32_t* att = uniform_ptr(A->att);
    for (int it = g + G * wave; it < H * S; it += G * kSWaves) {
        const int h = it / S, s = it - (it / S) * S;
        const int t0 = s * kSplitLen, t1 = min(n, t0 + kSplitLen);
        const bool has_new = pos >= t0 && pos < t1;
        float* kt = kt_all + (int64_t)h * D * ctx;  // [D][ctx]
        float* vc = vc_all + (int64_t)h * ctx * D;  // [ctx][D]
        if (lane < half) {
            const float cs = ld_g(cos_t + (int64_t)pos * half + lane);
            const float sn = ld_g(sin_t + (int64_t)pos * half + lane);
            const float q0 = ld_agent(qkv + h * D + 2 * lane);
            const float q1 = ld_agent(qkv + h * D + 2 * lane + 1);
            float k0 = 0.f, k1 = 0.f, v0 = 0.f, v1 = 0.f;
            if (has_new) {
                k0 = ld_agent(qkv + C + h * D + 2 * lane);
                k1 = ld_agent(qkv + C + h * D + 2 * lane + 1);
                v0 = ld_agent(qkv + 2 * C + h * D + 2 * lane);
                v1 = ld_agent(qkv + 2 * C + h * D + 2 * lane + 1);
            }
            // q * cos + rotate(q) * sin, then the reference's (q * scale)
            qs[2 * lane] = __fmul_rn(__fadd_rn(__fmul_rn(q0, cs), __fmul_rn(-q1, sn)), scale);
            qs[2 * lane + 1] = __fmul_rn(__fadd_rn(__fmul_rn(q1, cs), __fmul_rn(q0, sn)), scale);
            if (has_new) {
                const float r0 = __fadd_rn(__fmul_rn(k0, cs), __fmul_rn(-k1, sn));
                const float r1 = __fadd_rn(__fmul_rn(k1, cs), __fmul_rn(k0, sn));
                kn[2 * lane] = r0;
                kn[2 * lane + 1] = r1;
                vn[2 * lane] = v0;
                vn[2 * lane + 1] = v1;
                st_agent(kt + (int64_t)(2 * lane) * ctx + pos, r0);
                st_agent(kt + (int64_t)(2 * lane + 1) * ctx + pos, r1);
                st_agent(vc + (int64_t)pos * D + 2 * lane, v0);
                st_agent(vc + (int64_t)pos * D + 2 * lane + 1, v1);
            }
        }
        // scores
        const int qd = lane >> 4, p = lane & 15;
        const int t = t0 + p;
        const bool tin = t < t1;
        float kk[kMaxD / 4];
#pragma unroll
        for (int j = 0; j < kMaxD / 4; ++j) {
            const int d = qd * dq + j;
            kk[j] = (j < dq && tin && t != pos) ? ld_agent(kt + (int64_t)d * ctx + t) : 0.f;
        }
        float part = 0.f;
#pragma unroll
        for (int j = 0; j < kMaxD / 4; ++j) {
            if (j < dq) {
                const int d = qd * dq + j;
                part += qs[d] * (t == pos ? kn[d] : kk[j]);
            }
        }
        const float s1 = part + __shfl_xor(part, 16, 64);
        const float score = tin ? s1 + __shfl_xor(s1, 32, 64) : -INFINITY;
        const float m = wave_max(score);
        const float e = tin ? __expf(score - m) : 0.f;
        const float l = wave_sum(qd == 0 ? e : 0.f);
        if (qd == 0) pw[p] = e;
        // weighted sum of values: lane -> dimensions 2 lane, 2 lane + 1
        float acc0 = 0.f, acc1 = 0.f;
        if (lane < half) {
            float va[kSplitLen], vb[kSplitLen];
#pragma unroll
            for (int i = 0; i < kSplitLen; ++i) {
                const int tt = t0 + i;
                const bool in = tt < t1 && tt != pos;
                va[i] = in ? ld_agent(vc + (int64_t)tt * D + 2 * lane) : 0.f;
                vb[i] = in ? ld_agent(vc + (int64_t)tt * D + 2 * lane + 1) : 0.f;
            }
#pragma unroll
            for (int i = 0; i < kSplitLen; ++i) {
                const int tt = t0 + i;
                if (tt < t1) {
                    const float pv = pw[i];
                    acc0 += pv * (tt == pos ? vn[2 * lane] : va[i]);
                    acc1 += pv * (tt == pos ? vn[2 * lane + 1] : vb[i]);
                }
            }
        }
        float* wk = awork + ((int64_t)h * kMaxSplits + s) * (kMaxD + 2);
        if (lane == 0) {
            st_agent(wk, m);
            st_agent(wk + 1, l);
        }
        if (lane < half) {
            st_agent(wk + 2 + 2 * lane, acc0);
            st_agent(wk + 3 + 2 * lane, acc1);
        }
        wait_vm<0>();  // partials stored before the counter publishes them
        unsigned old = 0;
        if (lane == 0) old = add_agent(ctl + kCtlDone + h, 1u);
        old = __builtin_amdgcn_readfirstlane(old);
        if (old != (unsigned)S - 1u) continue;
        // combine: lane j < S reads split j's max and sum; the split
        // weights exp(m_j - M) go through LDS
        const float* base = awork + (int64_t)h * kMaxSplits * (kMaxD + 2);
        const float mj = lane < S ? ld_agent(base + lane * (kMaxD + 2)) : -INFINITY;
        const float lj = lane < S ? ld_agent(base + lane * (kMaxD + 2) + 1) : 0.f;
        const float M = wave_max(mj);
        const float f = (lane < S && mj != -INFINITY) ? __expf(mj - M) : 0.f;
        pw[lane] = f;
        // sum of f_j l_j in split order
        const float flj = f * lj;
        float Lsum = 0.f;
        for (int j = 0; j < S; ++j) Lsum += __shfl(flj, j, 64);
        if (lane < half) {
            float O0 = 0.f, O1 = 0.f;
            for (int j0 = 0; j0 < S; j0 += 16) {
                float oa[16], ob[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    const float* pj = base + (j0 + u) * (kMaxD + 2);
                    oa[u] = j0 + u < S ? ld_agent(pj + 2 + 2 * lane) : 0.f;
                    ob[u] = j0 + u < S ? ld_agent(pj + 3 + 2 * lane) : 0.f;
                }
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    if (j0 + u < S) {
                        O0 += pw[j0 + u] * oa[u];
                        O1 += pw[j0 + u] * ob[u];
                    }
                }
            }
            const uint32_t pr = (uint32_t)f32_to_bf16_rne(O0 / Lsum) |
                                ((uint32_t)f32_to_bf16_rne(O1 / Lsum) << 16);
            st_agent_u(att + ((h * D) >> 1) + lane, pr);
        }
        if (lane == 0) st_agent_u(ctl + kCtlDone + h, 0u);  // ready for the next layer
        wait_vm<0>();
    }
}

// Tied head rows of this wave (two in flight), soft cap 30 tanh(l / 30),
// logits out; returns the wave's largest argmax key (lane 0).  The key is
// (order-preserving bits of the capped logit) << 32 | (0xffffffff - row),
// so the largest key is the first row with the largest value -- torch's
// argmax -- whatever the order of the atomics.
__device__ __forceinline__ unsigned long long head_rows(int g, int G, int wave, int lane) {
    NB_SMEM;
    const PArgs* A = NB_ARGS;
    const float* tmp = reinterpret_cast<const float*>(smem + kOffTmp);
    const int C = A->C, V = A->V;
    const bf16_bits* emb = uniform_ptr(A->emb_bf16);
    float* logits = A->logits;
    const int NW = G * kSWaves;
    unsigned long long best = 0ull;
    auto dot = [&](const u32x4_t (&v)[kHeadPieces]) -> float {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < kHeadPieces; ++i) {
            const int c = lane * 8 + 512 * i;
            if (c < C) {
                const uint32_t wv[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc += tmp[c + 2 * j] * __uint_as_float(wv[j] << 16);
                    acc += tmp[c + 2 * j + 1] * __uint_as_float(wv[j] & 0xffff0000u);
                }
            }
        }
        return wave_sum(acc);
    };
    auto finish = [&](float acc, int r) {
        const float capped = 30.0f * tanhf(acc / 30.0f);
        if (lane == 0) {
            if (logits) *as_global_mut(logits + r) = capped;
            const unsigned long long key =
                ((unsigned long long)orderable(capped) << 32) | (0xffffffffu - (uint32_t)r);
            best = key > best ? key : best;
        }
    };
    for (int r = g * kSWaves + wave; r < V; r += 2 * NW) {
        const int r2 = r + NW;
        u32x4_t va[kHeadPieces], vb[kHeadPieces];
        const u32x4_t z = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < kHeadPieces; ++i) {
            const int c = lane * 8 + 512 * i;
            va[i] = c < C ? __builtin_nontemporal_load(
                                as_global(reinterpret_cast<const u32x4_t*>(emb + (int64_t)r * C + c)))
                          : z;
            vb[i] = (c < C && r2 < V) ? __builtin_nontemporal_load(as_global(
                                            reinterpret_cast<const u32x4_t*>(emb + (int64_t)r2 * C + c)))
                                      : z;
        }
        finish(dot(va), r);
        if (r2 < V) finish(dot(vb), r2);
    }
    return best;
}

// ---------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3, 3)))
void decode_persistent_kernel(PArgs args) {
    NB_SMEM;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = blockIdx.x, G = gridDim.x;
    // The arguments live in LDS and are read where they are used: kept in
    // scalar registers for the whole kernel they left too few for the
    // streaming loop.
    PArgs* A = reinterpret_cast<PArgs*>(smem + kOffArgs);
    if (tid == 0) *A = args;
    LDS3 float* ybuf = lds_at<float>(kOffY);
    LDS3 int* cnt = lds_at<int>(kOffCnt);
    LDS3 unsigned long long* wkey = lds_at<unsigned long long>(kOffMisc + 64);  // 16
    LDS3 int* abort_flag = lds_at<int>(kOffMisc + 192);
    LDS3 KGeo* kg = lds_at<KGeo>(kOffGeo);
    LDS3 uint8_t* lcol_t = lds_at<uint8_t>(kOffLane);  // [kind][lane] column of the lane's block
    typedef const void* gptr;
    LDS3 gptr* ptab = lds_at<gptr>(kOffPtab);

    const int L = args.L, C = args.C, F = args.F;
    const int GP = args.n_steps * 4 * L;  // GEMV phases of the whole sequence
    int pos = ld_g(&args.st->pos), tok = ld_g(&args.st->token), step = ld_g(&args.st->step);
    unsigned nbar = 0;  // grid barriers passed (control wave)
    // A token outside the embedding table never forms an address: it sets
    // bit 1 of the error word (every workgroup then leaves at its next grid
    // barrier, the launch ends normally) and row 0 is read instead.
    auto checked_token = [&](int t) -> int {
        if ((unsigned)t < (unsigned)args.V) return t;
        if (tid == 0) {
            __hip_atomic_fetch_or(as_global_mut(args.ctl + kCtlErr), 2u, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
        }
        return 0;
    };
    tok = checked_token(tok);

    // ---- set-up: geometry of the four GEMV kinds for this workgroup, lane
    // table, the stream and codebook pointers of every layer and kind, and
    // the chunk counters (LDS reads keep divisions and global loads -- whose
    // vmcnt waits would drain the ring -- out of the streaming loop)
    if (tid < 4) {
        const int kind = tid;
        KGeo k;
        k.N = kind == kQKV ? 3 * C : kind == kGU ? 2 * F : C;
        k.bpr = (kind == kDown ? F : C) >> 7;
        k.R = kChunkMax / k.bpr;
        k.nbk = k.R * k.bpr;
        const int nch = (k.N + k.R - 1) / k.R;
        k.c0 = (int)((int64_t)nch * g / G);
        k.c1 = (int)((int64_t)nch * (g + 1) / G);
        kgeo_put(kg + kind, k);
    }
    if (tid < 4 * 64) {
        const int kind = tid >> 6, l = tid & 63;
        const int bpr = (kind == kDown ? F : C) >> 7;
        lcol_t[tid] = (uint8_t)(l < (kChunkMax / bpr) * bpr ? l % bpr : 0);
    }
    for (int i = tid; i < L * 4; i += kThreads) {
        const layer_cptr Ly = (layer_cptr)(args.layers) + (i >> 2);
        ptab[2 * i] = packed_of(Ly, i & 3);
        ptab[2 * i + 1] = codebook_of(Ly, i & 3);
    }
    if (tid == 0) *abort_flag = 0;
    wg_barrier();
    if (tid < kCntWindow) cnt[tid] = kg[tid & 3].c0;
    wg_barrier();

    // ---- streaming-wave ring state -----------------------------------------
    const uint32_t ring_lds = (uint32_t)(kOffRing + wave * kDepth * kSlotBytes);
    LDS3 unsigned char* my_ring = lds_at<unsigned char>(kOffRing + wave * kDepth * kSlotBytes);
    // load cursor: GEMV phase cq (kind ck of layer cl) to take chunks from
    int cq = 0, ck = 0, cl = 0;
    bool cv = GP > 0;
    // slot meta: GEMV phase, chunk, loaded (scalars, not arrays: a runtime
    // index would put them in scratch)
    int sq0 = 0, sc0 = 0, sq1 = 0, sc1 = 0;
    bool sv0 = false, sv1 = false;
    int hs = 0;  // ring head (oldest slot)

    // next chunk of the sequence for this wave: (phase, chunk) or invalid;
    // loads it into slot s (five 1 KiB direct-to-LDS loads; lanes past the
    // chunk's bytes re-read its last 16 bytes)
    auto grab_issue = [&](int s) {
        bool valid = false;
        int q = 0, c = 0;
        while (cv) {
            int t = 0;
            if (lane == 0) {
                t = __hip_atomic_fetch_add(cnt + (cq & (kCntWindow - 1)), 1, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_WORKGROUP);
            }
            t = __builtin_amdgcn_readfirstlane(t);
            if (t < kg[ck].c1) {
                valid = true;
                q = cq;
                c = t;
                break;
            }
            ++cq;
            if (++ck == 4) {
                ck = 0;
                if (++cl == L) cl = 0;
            }
            if (cq >= GP) cv = false;
        }
        if (s) {
            sv1 = valid;
            sq1 = q;
            sc1 = c;
        } else {
            sv0 = valid;
            sq0 = q;
            sc0 = c;
        }
        if (!valid) return;
        const KGeo k = kgeo_get(kg + ck);
        const int pi = (cl * 4 + ck) * 2;
        const uint8_t* pk = static_cast<const uint8_t*>(uniform_ptr(ptab[pi]));
        const uint8_t* cb = static_cast<const uint8_t*>(uniform_ptr(ptab[pi + 1]));
        const int nbk = min(k.R, k.N - c * k.R) * k.bpr;
        const int64_t b0 = (int64_t)c * k.nbk;
        const uint8_t* ip = pk + b0 * 48;
        const uint8_t* cp = cb + b0 * 32;
        const int ilast = nbk * 48 - 16, clast = nbk * 32 - 16;
        const uint32_t dst = __builtin_amdgcn_readfirstlane(ring_lds + s * kSlotBytes);
        dma16<0>(dst, ip + min(16 * lane, ilast));
        dma16<0>(dst + 1024, ip + min(16 * lane + 1024, ilast));
        dma16<0>(dst + 2048, ip + min(16 * lane + 2048, ilast));
        dma16<0>(dst + kIdxSlot, cp + min(16 * lane, clast));
        dma16<0>(dst + kIdxSlot + 1024, cp + min(16 * lane + 1024, clast));
    };

    if (wave < kSWaves) {
        grab_issue(0);
        grab_issue(1);
    }

    // ---- one ring step: compute the head slot (a chunk of kind `kind`) ------
    auto ring_step = [&](int kind) {
        const int s = hs;
        const int c = s ? sc1 : sc0;
        const KGeo k = kgeo_get(kg + kind);
        const int rows = min(k.R, k.N - c * k.R);
        const int bpr = k.bpr;
        const bool live = lane < rows * bpr;
        const int col = lcol_t[kind * 64 + lane];
        u32x4_t xv[16];
        const LDS3 u32x4_t* xb = lds_at<u32x4_t>(kOffX + col * kXColBytes);
#pragma unroll
        for (int j = 0; j < 16; ++j) xv[j] = xb[j];
        // the other slot was loaded after this one: its loads may stay in flight
        if (s ? sv0 : sv1) {
            wait_vm<kLoadsPerChunk>();
        } else {
            wait_vm<0>();
        }
        const LDS3 unsigned char* src = my_ring + s * kSlotBytes;
        const LDS3 u32x4_t* pi = (const LDS3 u32x4_t*)(src + 48 * lane);
        const LDS3 u32x4_t* pc = (const LDS3 u32x4_t*)(src + kIdxSlot + 32 * lane);
        const u32x4_t d0 = pi[0], d1 = pi[1], d2 = pi[2], c0 = pc[0], c1 = pc[1];
        wait_lds();
        grab_issue(s);
        const float dot = diag_of(block_dot(d0, d1, d2, c0, c1, xv), lane);
        // row sums in block order through the wave's scratch, read 8 at a time
        LDS3 float* rs = lds_at<float>(kOffTmp + wave * 256);
        rs[lane] = live ? dot : 0.f;
        if (lane < rows) {
            const LDS3 float* rr = rs + lane * bpr;
            float sum = 0.f;
            for (int j = 0; j < bpr; j += 8) {
                float v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = j + u < bpr ? rr[j + u] : 0.f;
#pragma unroll
                for (int u = 0; u < 8; ++u) sum += v[u];
            }
            ybuf[(c - k.c0) * k.R + lane] = sum;
        }
        hs ^= 1;
    };

    // ---- synchronisation at the end of a phase ----------------------------
    // All waves call it.  `epi` runs in the control wave between the two
    // workgroup barriers, before its stores are waited for and the grid
    // barrier is taken.  Returns false when the launch is being abandoned.
    auto phase_end = [&](auto epi) -> bool {
        wg_barrier();
        if (wave == kCtl) {
            epi();
            wait_vm<0>();
            bool ok = true;
            ++nbar;
            if (lane == 0) ok = grid_barrier(uniform_ptr(A->ctl), nbar, g, G, A->spin_limit);
            if (lane == 0 && !ok) *abort_flag = 1;
        }
        wg_barrier();
        return *abort_flag == 0;
    };

    // ---- one GEMV phase ---------------------------------------------------
    auto gemv_phase = [&](int kind, int layer, int gq) -> bool {
        if (kind == kQKV || kind == kGU) {
            const layer_cptr Ly = layer_at(A->layers, layer);
            const bool emb = kind == kQKV && layer == 0;
            const float* src = emb ? A->emb_f32 + (int64_t)tok * C : A->xres;
            norm_to_tmp(src, !emb, kind == kQKV ? Ly->ln1 : Ly->ln2, false, tid);
            if (emb && wave == kCtl) {
                // this workgroup's share of the residual stream starts as
                // the embedding row (stored before the phase's barrier by
                // the control wave, which waits for its stores there)
                const int i0 = (int)((int64_t)C * g / G), i1 = (int)((int64_t)C * (g + 1) / G);
                float* x = uniform_ptr(A->xres);
                for (int i = i0 + lane; i < i1; i += 64) st_agent(x + i, ld_g(src + i));
            }
        } else if (kind == kO) {
            att_to_tmp(tid);
        } else {
            silu_to_tmp(tid);
        }
        wg_barrier();
        stage_from_tmp(kind == kDown ? F : C, tid);
        wg_barrier();
        if (wave < kSWaves) {
            while ((hs ? sv1 : sv0) && (hs ? sq1 : sq0) == gq) ring_step(kind);
        }
        return phase_end([&] {
            const KGeo k = kgeo_get(kg + kind);
            if (lane == 0) cnt[gq & (kCntWindow - 1)] = k.c0;  // ready for phase gq + 32
            const int r0 = k.c0 * k.R;
            const int nrows = min(k.N, k.c1 * k.R) - r0;
            float* out = uniform_ptr(kind == kQKV ? A->qkv : kind == kGU ? A->gu : A->xres);
            for (int i = lane; i < nrows; i += 64) {
                const int row = r0 + i;
                const float v = ybuf[i];
                if (kind == kQKV || kind == kGU) {
                    st_agent(out + row, v);
                } else {
                    // residual add (generate_torch.py:130-131)
                    st_agent(out + row, ld_agent(out + row) + v);
                }
            }
        });
    };

    auto attention_phase = [&](int layer) -> bool {
        if (wave < kSWaves && pos < A->ctx) attention_items(layer, pos, g, G, wave, lane);
        return phase_end([&] {
            // every workgroup read the argmax key before the QKV barrier of
            // layer 0; clear it for this token's head
            if (layer == 0 && g == 0 && lane == 0) {
                __hip_atomic_store(&as_global_mut(A->st)->key, 0ull, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
        });
    };

    auto head_phase = [&]() -> bool {
        norm_to_tmp(A->xres, true, A->ln_f, true, tid);
        wg_barrier();
        if (wave < kSWaves) {
            const unsigned long long best = head_rows(g, G, wave, lane);
            if (lane == 0) wkey[wave] = best;
        }
        return phase_end([&] {
            if (lane == 0) {
                unsigned long long b = 0ull;
                for (int w = 0; w < kSWaves; ++w) b = wkey[w] > b ? wkey[w] : b;
                __hip_atomic_fetch_max(&as_global_mut(A->st)->key, b, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
        });
    };

    // ---- the sequence -----------------------------------------------------
    bool ok = true;
    for (int t = 0; ok && t < args.n_steps; ++t) {
        // phases of a layer: QKV, ATT, O, GU, DOWN (one call site each, so
        // the GEMV phase is compiled once)
        for (int ph = 0; ok && ph < 5 * L; ++ph) {
            const int l = ph / 5, j = ph - l * 5;
            if (j == 1) {
                ok = attention_phase(l);
            } else {
                const int kind = j == 0 ? kQKV : j - 1;
                ok = gemv_phase(kind, l, (t * L + l) * 4 + kind);
            }
        }
        if (!ok || !head_phase()) {
            ok = false;
            break;
        }
        const unsigned long long key =
            __hip_atomic_load(&as_global_mut(A->st)->key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int am = (int)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
        if (g == 0 && tid == 0 && step >= 0 && step < A->tokens_cap) {
            *as_global_mut(A->tokens_out + step) = am;
        }
        tok = checked_token((step >= 0 && step < A->n_force) ? ld_g(A->force + step) : am);
        pos += 1;
        step += 1;
    }
    // every workgroup has read the last key: publish the state
    if (ok) ok = phase_end([] {});
    if (ok && g == 0 && tid == 0) {
        auto* st = as_global_mut(A->st);
        st->key = 0ull;
        st->done = 0u;
        st->pos = pos;
        st->token = tok;
        st->step = step;
    }
    wait_vm<0>();  // no ring load outlives the workgroup
}

__global__ void clear_ctl_kernel(unsigned* __restrict__ ctl, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) ctl[i] = 0u;
}

}  // namespace

int64_t decode_persistent_workspace_bytes(int C, int H, int F) {
    auto up = [](int64_t b) { return (b + 255) / 256 * 256; };
    return kCtlBytes + up((int64_t)C * 4) + up((int64_t)3 * C * 4) + up((int64_t)C * 2) +
           up((int64_t)2 * F * 4) + up((int64_t)H * kMaxSplits * (kMaxD + 2) * 4);
}

int decode_persistent_limits(int* max_c, int* max_f, int* max_d, int* max_ctx, int* max_heads,
                             int* max_layers) {
    *max_layers = kMaxLayers;
    *max_c = kMaxC;
    *max_f = kMaxF;
    *max_d = kMaxD;
    *max_ctx = kMaxSplits * kSplitLen;
    *max_heads = kMaxHeads;
    return NB_OK;
}

int launch_decode_persistent(const nb_decode_model& m, void* workspace, nb_decode_state* st,
                             float* logits, int32_t* tokens_out, int tokens_cap,
                             const int32_t* force, int n_force, int n_steps, int spin_limit,
                             hipStream_t stream) {
    // one workgroup per CU, fewer when a layer has fewer row chunks (every
    // workgroup needs a chunk of every GEMV kind); each workgroup's outputs
    // of a phase must fit the LDS result buffer
    PArgs a = {};
    a.C = m.n_embd;
    a.F = m.ffn_hidden;
    int G = device_cu_count();
    for (int kind = 0; kind < 4; ++kind) {
        const int N = kind == kQKV ? 3 * a.C : kind == kGU ? 2 * a.F : a.C;
        const int K = kind == kDown ? a.F : a.C;
        const int R = kChunkMax / (K / 128);
        G = std::min(G, (N + R - 1) / R);
    }
    for (int kind = 0; kind < 4; ++kind) {
        const int N = kind == kQKV ? 3 * a.C : kind == kGU ? 2 * a.F : a.C;
        const int K = kind == kDown ? a.F : a.C;
        const int R = kChunkMax / (K / 128);
        const int nch = (N + R - 1) / R;
        if ((int64_t)((nch + G - 1) / G) * R > kYMax) {
            return fail(NB_EUNSUPPORTED, "nb_decode_persistent: %dx%d layer: %d rows per "
                                         "workgroup exceed %d", N, K, (nch + G - 1) / G * R, kYMax);
        }
    }
    if (hipFuncSetAttribute((const void*)decode_persistent_kernel,
                            hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes) != hipSuccess) {
        return fail(NB_ELAUNCH, "nb_decode_persistent: cannot reserve %d bytes of LDS", kLdsBytes);
    }
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, decode_persistent_kernel, kThreads,
                                                     kLdsBytes) != hipSuccess || occ < 1) {
        return fail(NB_ELAUNCH, "nb_decode_persistent: kernel does not fit a CU (occupancy %d)", occ);
    }
    unsigned char* ws = static_cast<unsigned char*>(workspace);
    auto up = [](int64_t b) { return (b + 255) / 256 * 256; };
    int64_t off = kCtlBytes;
    a.ctl = reinterpret_cast<unsigned*>(ws);
    a.xres = reinterpret_cast<float*>(ws + off);
    off += up((int64_t)a.C * 4);
    a.qkv = reinterpret_cast<float*>(ws + off);
    off += up((int64_t)3 * a.C * 4);
    a.att = reinterpret_cast<uint32_t*>(ws + off);
    off += up((int64_t)a.C * 2);
    a.gu = reinterpret_cast<float*>(ws + off);
    off += up((int64_t)2 * a.F * 4);
    a.awork = reinterpret_cast<float*>(ws + off);
    a.layers = m.layers;
    a.ln_f = m.ln_f;
    a.emb_f32 = m.emb_f32;
    a.emb_bf16 = static_cast<const bf16_bits*>(m.emb_bf16);
    a.cos_t = m.rope_cos;
    a.sin_t = m.rope_sin;
    a.st = st;
    a.logits = logits;
    a.tokens_out = tokens_out;
    a.force = force;
    a.tokens_cap = tokens_cap;
    a.n_force = n_force;
    a.L = m.n_layers;
    a.H = m.n_head;
    a.D = m.head_dim;
    a.V = m.vocab;
    a.ctx = m.ctx;
    a.n_steps = n_steps;
    a.eps = m.eps;
    a.spin_limit = spin_limit;
    // barrier counters, error word and split counters start at zero (a
    // kernel, not a memset node: the call stays graph-capturable)
    hipLaunchKernelGGL(clear_ctl_kernel, dim3(1), dim3(256), 0, stream,
                       reinterpret_cast<unsigned*>(ws), kCtlBytes / 4);
    if (check_launch("nb_decode_persistent") != NB_OK) return NB_ELAUNCH;
    void* args[] = {&a};
    const hipError_t e = hipLaunchCooperativeKernel((const void*)decode_persistent_kernel, dim3(G),
                                                    dim3(kThreads), args, kLdsBytes, stream);
    if (e != hipSuccess) {
        return fail(NB_ELAUNCH, "nb_decode_persistent: cooperative launch of %d workgroups failed: %s",
                    G, hipGetErrorString(e));
    }
    return check_launch("nb_decode_persistent");
}

}  // namespace nb
