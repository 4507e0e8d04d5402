// Fused dequant + GEMV for NativeBit packed weights on gfx950.
//
//   y[m][n] = sum_k x[m][k] * W[n][k],  W.flat[i] = cb[i / BS][field i]
//
// Replaces the reference's thread-per-row CUDA kernel
// (inference/cuda_kernel.py:38-104) and the Triton compare-select kernels
// (inference/triton_kernel.py:23-196).  Two kernels:
//
// * gemv_fast_kernel: M == 1, 2/3/4-bit with 2^bits entries, BS in
//   {64,128,256}, K % 256 == 0, K <= 8192 (every 2.2B-shape layer).  The
//   workgroup's 256 lanes tile P = 256 / (K/32) rows side by side; lane t
//   owns one 32-weight "slice" (BITS consecutive dwords of the packed stream,
//   so a wave reads one contiguous run of the stream) and keeps the 32
//   activations of that slice in registers for every row it visits.  The
//   block's codebook is staged in LDS by the BS/32 lanes that share the
//   block (one coalesced load each), every weight is one field extract, one
//   LDS lookup and one fp32 FMA, and the row sum is reduced in 8-lane groups
//   then across groups through LDS.  R row-sets are in flight per iteration
//   to keep enough HBM requests outstanding.
// * gemv_generic_kernel: any shape, bits 1..8, M <= 16.  One workgroup per
//   output row, lanes stride over k and read each field from the byte
//   stream.  Used for ragged shapes and as an independent statement of the
//   arithmetic.
//
// Arithmetic for both: with fp32 x the exact fp32 codebook value, with bf16 x
// the codebook value rounded to bf16 (the reference's bf16 semantics,
// inference/eval_ppl.py:166; nb_gemv_mfma.hip computes the same), times x
// widened to fp32, fp32 FMA accumulation; y is stored as fp32 or rounded to
// bf16 (RNE).
//
// The bf16-activation 3-bit / 8-entry / block-128 case is taken by the MFMA
// kernel in nb_gemv_mfma.hip before either kernel here is considered.
#include "nb_device.h"
#include "nb_internal.h"

#include <utility>

namespace nb {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxM = 16;

__device__ __forceinline__ float load_x(const void* x, int dtype, int64_t i) {
    if (dtype == NB_BF16) return bf16_to_f32(static_cast<const bf16_bits*>(x)[i]);
    return static_cast<const float*>(x)[i];
}

__device__ __forceinline__ void store_y(void* y, int dtype, int64_t i, float v) {
    if (dtype == NB_BF16) {
        static_cast<bf16_bits*>(y)[i] = f32_to_bf16_rne(v);
    } else {
        static_cast<float*>(y)[i] = v;
    }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// ---------------------------------------------------------------------------
// generic kernel
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void gemv_generic_kernel(GemvArgs a) {
    __shared__ float red[kThreads / 64][kMaxM];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const uint32_t last = (uint32_t)(a.n_entries - 1);
    for (int n = blockIdx.x; n < a.N; n += gridDim.x) {
        float acc[kMaxM];
#pragma unroll
        for (int m = 0; m < kMaxM; ++m) acc[m] = 0.f;
        for (int k = threadIdx.x; k < a.K; k += kThreads) {
            const int64_t flat = (int64_t)n * a.K + k;
            uint32_t e = read_field(a.packed, a.packed_bytes, flat, a.bits);
            e = e < last ? e : last;
            float w = a.codebook[(flat / a.block_size) * a.n_entries + e];
            if (a.x_dtype == NB_BF16) w = round_bf16(w);
#pragma unroll
            for (int m = 0; m < kMaxM; ++m) {
                if (m < a.M) acc[m] = fmaf(w, load_x(a.x, a.x_dtype, m * a.ldx + k), acc[m]);
            }
        }
#pragma unroll
        for (int m = 0; m < kMaxM; ++m) {
            if (m < a.M) {
                const float v = wave_sum(acc[m]);
                if (lane == 0) red[wave][m] = v;
            }
        }
        __syncthreads();
        if ((int)threadIdx.x < a.M) {
            float s = 0.f;
#pragma unroll
            for (int w = 0; w < kThreads / 64; ++w) s += red[w][threadIdx.x];
            store_y(a.y, a.y_dtype, (int64_t)threadIdx.x * a.ldy + n, s);
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(kThreads) void fill_zero_kernel(void* y, int dtype,
                                                             int M, int N,
                                                             int64_t ldy) {
    const int64_t total = (int64_t)M * N;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kThreads) {
        const int64_t m = i / N, n = i - m * N;
        store_y(y, dtype, m * ldy + n, 0.f);
    }
}

// ---------------------------------------------------------------------------
// fast M == 1 kernel
// ---------------------------------------------------------------------------
template <bool kXBF16>
__device__ __forceinline__ void load_x_slice(const void* x, int s, float (&xr)[32]) {
    if (kXBF16) {
        const uint4* p = reinterpret_cast<const uint4*>(static_cast<const bf16_bits*>(x) + s * 32);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint4 u = p[v];
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                xr[v * 8 + 2 * h] = __uint_as_float(w[h] << 16);
                xr[v * 8 + 2 * h + 1] = __uint_as_float(w[h] & 0xFFFF0000u);
            }
        }
    } else {
        const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + s * 32);
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            const float4 f = p[v];
            xr[4 * v] = f.x;
            xr[4 * v + 1] = f.y;
            xr[4 * v + 2] = f.z;
            xr[4 * v + 3] = f.w;
        }
    }
}

// (a & MASK) | b in one VALU op.  Written as asm because the compiler
// rewrites the disjoint `or` into an add and then needs a separate and+add.
template <uint32_t MASK>
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t b) {
    static_assert(MASK <= 64, "mask must be an inline constant");
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "i"(MASK), "v"(b));
    return r;
}

// Byte offset of codebook entry (field j) in the lane's table, whose base
// byte offset `base` is a multiple of 4 << BITS: the field is shifted
// straight to bit 2 and merged with the base, two VALU ops per weight (the
// two fields of a 3-bit slice that straddle a dword use a funnel shift).
template <int BITS, int J>
__device__ __forceinline__ uint32_t entry_offset(const uint32_t (&d)[BITS], uint32_t base) {
    constexpr int bit = J * BITS;
    constexpr int w = bit >> 5;
    constexpr int off = bit & 31;
    constexpr uint32_t kMask = ((1u << BITS) - 1u) << 2;
    uint32_t v;
    if constexpr (off + BITS > 32) {
        v = __builtin_amdgcn_alignbit(d[w + 1], d[w], off - 2);
    } else if constexpr (off >= 2) {
        v = d[w] >> (off - 2);
    } else {
        v = d[w] << (2 - off);
    }
    return and_or<kMask>(v, base);
}

template <int BITS, int J0, int... Js>
__device__ __forceinline__ void lookup8(const uint32_t (&d)[BITS], uint32_t base,
                                        const char* tab, float (&w)[8],
                                        std::integer_sequence<int, Js...>) {
    ((w[Js] = *reinterpret_cast<const float*>(tab + entry_offset<BITS, J0 + Js>(d, base))), ...);
}

// sum_j cb[field j] * x[j] over the 32 weights of a slice.  Lookups are
// issued eight at a time into registers before the FMAs so that the LDS
// latency overlaps, and two accumulators shorten the FMA chain.
template <int BITS>
__device__ __forceinline__ float slice_dot(const uint32_t (&d)[BITS], uint32_t base,
                                           const char* tab, const float (&xr)[32]) {
    float a0 = 0.f, a1 = 0.f;
    float w[4][8];
    lookup8<BITS, 0>(d, base, tab, w[0], std::make_integer_sequence<int, 8>{});
    lookup8<BITS, 8>(d, base, tab, w[1], std::make_integer_sequence<int, 8>{});
    lookup8<BITS, 16>(d, base, tab, w[2], std::make_integer_sequence<int, 8>{});
    lookup8<BITS, 24>(d, base, tab, w[3], std::make_integer_sequence<int, 8>{});
#pragma unroll
    for (int g = 0; g < 4; ++g) {
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            a0 = fmaf(w[g][i], xr[g * 8 + i], a0);
            a1 = fmaf(w[g][i + 1], xr[g * 8 + i + 1], a1);
        }
    }
    return a0 + a1;
}

// Pipeline depth of the streaming kernel (row-sets whose loads are in flight
// per lane) and resident workgroups per CU it is launched with.
#ifndef NB_GEMV_DEPTH
#define NB_GEMV_DEPTH 2
#endif
#ifndef NB_GEMV_WG_PER_CU
#define NB_GEMV_WG_PER_CU 4
#endif

// Row-set `set` of the stream: this lane's BITS dwords and EPL codebook
// entries (loads only; nothing waits here).
template <int BITS, int BS, int EPL>
__device__ __forceinline__ void issue_set(const uint32_t* __restrict__ packed,
                                          const float* __restrict__ cb, int row,
                                          int S, int s, int bpr, int q,
                                          uint32_t (&d)[BITS], float (&cv)[EPL]) {
    constexpr int NE = 1 << BITS;
    constexpr int SPB = BS / 32;
    const uint32_t* pk = packed + ((int64_t)row * S + s) * BITS;
#pragma unroll
    for (int w = 0; w < BITS; ++w) d[w] = stream_load(pk + w);
    const float* c = cb + ((int64_t)row * bpr + s / SPB) * NE + q * EPL;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        if (q * EPL + e < NE) cv[e] = stream_load(c + e);
    }
}

// Each workgroup streams a contiguous range of row-sets.  Lane registers
// hold a ring of D row-sets: the loads of set i+D are issued right after set
// i has been consumed, so every lane keeps D sets of HBM requests in flight
// while it computes.
template <int BITS, int BS, bool kXBF16, int D>
__global__ __launch_bounds__(kThreads) void gemv_fast_kernel(
    const void* __restrict__ x, const uint32_t* __restrict__ packed,
    const float* __restrict__ cb, void* __restrict__ y, int y_dtype, int N,
    int K, int P, int n_sets) {
    constexpr int NE = 1 << BITS;
    constexpr int SPB = BS / 32;                  // slices (lanes) per block
    constexpr int NSLOT = kThreads / SPB;         // blocks per row-set
    constexpr int EPL = (NE + SPB - 1) / SPB;     // entries staged per lane
    __shared__ float s_cb[NSLOT * NE];
    __shared__ float s_red[2][kThreads / 8];

    const int t = threadIdx.x;
    const int S = K >> 5;           // slices per row
    const int row_sub = t / S;      // row inside the row-set
    const int s = t - row_sub * S;  // slice inside the row
    const bool lane_on = row_sub < P;
    const int bpr = K / BS;
    const int slot = t / SPB;
    const int q = t - slot * SPB;

    // contiguous, balanced range of row-sets for this workgroup
    const int per = n_sets / gridDim.x;
    const int rem = n_sets - per * gridDim.x;
    const int b = blockIdx.x;
    const int set_begin = b * per + (b < rem ? b : rem);
    const int count = per + (b < rem ? 1 : 0);

    // Loads are never predicated (a predicated load makes the compiler copy
    // its result right away, i.e. wait for it): lanes past the last row or
    // set load a clamped, already-cached address and their sums are dropped.
    const int last_set = set_begin + count - 1;
    auto clamp_row = [&](int set) {
        const int r = (set < last_set ? set : last_set) * P + row_sub;
        return r < N ? r : N - 1;
    };
    // The activations are requested first: a wave's loads retire in issue
    // order, so set 0 can be computed as soon as it and x are in while the
    // later sets are still arriving.
    float xr[32];
    load_x_slice<kXBF16>(x, s, xr);
    uint32_t d[D][BITS];
    float cv[D][EPL];
#pragma unroll
    for (int st = 0; st < D; ++st) {
        issue_set<BITS, BS, EPL>(packed, cb, clamp_row(set_begin + st), S, s, bpr, q,
                                 d[st], cv[st]);
    }

    for (int base = 0; base < count; base += D) {
#pragma unroll
        for (int st = 0; st < D; ++st) {
            const int i = base + st;
            if (i < count) {  // uniform over the workgroup
                const int set = set_begin + i;
                const bool valid = lane_on && set * P + row_sub < N;
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    if (q * EPL + e < NE) {
                        s_cb[slot * NE + q * EPL + e] = kXBF16 ? round_bf16(cv[st][e]) : cv[st][e];
                    }
                }
                // The SPB lanes sharing a slot are consecutive lanes of one
                // wave and a wave's LDS operations complete in issue order:
                // the table is visible below without a barrier, and the next
                // set's write comes after these reads.
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                float acc = slice_dot<BITS>(d[st], (uint32_t)(slot * NE * 4),
                                            reinterpret_cast<const char*>(s_cb), xr);
                acc = valid ? acc : 0.f;
                issue_set<BITS, BS, EPL>(packed, cb, clamp_row(set + D), S, s, bpr, q,
                                         d[st], cv[st]);
                // 8 consecutive lanes always belong to one row (S % 8 == 0).
                acc += __shfl_xor(acc, 1, 8);
                acc += __shfl_xor(acc, 2, 8);
                acc += __shfl_xor(acc, 4, 8);
                float* red = s_red[i & 1];
                if ((t & 7) == 0) red[t >> 3] = acc;
                // one barrier per set: s_red is double buffered, so the next
                // set writes the other half while this one is summed.
                __syncthreads();
                if (t < P) {
                    const int orow = set * P + t;
                    if (orow < N) {
                        const int ng = S >> 3;
                        float sum = 0.f;
                        for (int g = t * ng; g < (t + 1) * ng; ++g) sum += red[g];
                        store_y(y, y_dtype, orow, sum);
                    }
                }
            }
        }
    }
}

typedef void (*FastFn)(const void*, const uint32_t*, const float*, void*, int,
                       int, int, int, int);

template <int BITS, int BS>
FastFn pick_x(bool xb) {
    return xb ? gemv_fast_kernel<BITS, BS, true, NB_GEMV_DEPTH>
              : gemv_fast_kernel<BITS, BS, false, NB_GEMV_DEPTH>;
}

template <int BITS>
FastFn pick_bs(int bs, bool xb) {
    switch (bs) {
        case 64: return pick_x<BITS, 64>(xb);
        case 128: return pick_x<BITS, 128>(xb);
        case 256: return pick_x<BITS, 256>(xb);
    }
    return nullptr;
}

FastFn pick_fast(int bits, int bs, bool xb) {
    switch (bits) {
        case 2: return pick_bs<2>(bs, xb);
        case 3: return pick_bs<3>(bs, xb);
        case 4: return pick_bs<4>(bs, xb);
    }
    return nullptr;
}

bool fast_eligible(const GemvArgs& a) {
    if (a.M != 1) return false;
    if (a.bits < 2 || a.bits > 4 || a.n_entries != (1 << a.bits)) return false;
    if (a.block_size != 64 && a.block_size != 128 && a.block_size != 256) return false;
    if (a.K <= 0 || a.K % 256 != 0 || a.K % a.block_size != 0 || a.K / 32 > kThreads) return false;
    if (reinterpret_cast<uintptr_t>(a.packed) % 4 != 0) return false;
    if (reinterpret_cast<uintptr_t>(a.x) % 16 != 0) return false;
    return true;
}

}  // namespace

int launch_gemv(const GemvArgs& a, hipStream_t stream) {
    if (a.M == 0 || a.N == 0) return NB_OK;
    const int cus = device_cu_count();
    if (a.K == 0) {
        int64_t total = (int64_t)a.M * a.N;
        int64_t g = (total + kThreads - 1) / kThreads;
        if (g > cus * 8) g = cus * 8;
        hipLaunchKernelGGL(fill_zero_kernel, dim3((int)g), dim3(kThreads), 0, stream,
                           a.y, a.y_dtype, a.M, a.N, a.ldy);
        return check_launch("nb_gemv (K == 0)");
    }
    const int st = launch_gemv_mfma(a, stream);
    if (st != 1) return st;
    if (fast_eligible(a)) {
        const int S = a.K / 32;
        const int P = kThreads / S;
        const int n_sets = (a.N + P - 1) / P;
        int64_t grid = (int64_t)cus * NB_GEMV_WG_PER_CU;
        if (grid > n_sets) grid = n_sets;
        FastFn fn = pick_fast(a.bits, a.block_size, a.x_dtype == NB_BF16);
        hipLaunchKernelGGL(fn, dim3((int)grid), dim3(kThreads), 0, stream, a.x,
                           reinterpret_cast<const uint32_t*>(a.packed), a.codebook,
                           a.y, a.y_dtype, a.N, a.K, P, n_sets);
        return check_launch("nb_gemv (fast)");
    }
    int64_t grid = a.N;
    if (grid > (int64_t)cus * 16) grid = (int64_t)cus * 16;
    hipLaunchKernelGGL(gemv_generic_kernel, dim3((int)grid), dim3(kThreads), 0, stream, a);
    return check_launch("nb_gemv (generic)");
}

}  // namespace nb
