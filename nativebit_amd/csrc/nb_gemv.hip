// Fused dequant + GEMV for NativeBit packed weights on gfx950.
//
//   y[m][n] = sum_k x[m][k] * W[n][k],  W.flat[i] = cb[i / BS][field i]
//
// Replaces the reference's thread-per-row CUDA kernel
// (inference/cuda_kernel.py:38-104) and the Triton compare-select kernels
// (inference/triton_kernel.py:23-196).  Two kernels:
//
// * gemv_fast_kernel: M == 1, 2/3/4-bit with 2^bits entries, BS in
//   {64,128,256}, K % 256 == 0, K <= 8192 (every 2.2B-shape layer).  One
//   workgroup per CU of P * K/32 lanes (P rows side by side); lane t owns
//   one 32-weight "slice" of each of its row-sets (BITS consecutive dwords
//   of the packed stream) and keeps the slice's 32 activations in registers
//   for all of them.  The activations are staged once per workgroup; each
//   wave brings its 64 slices of a set (index bytes and their blocks'
//   codebooks, contiguous in the stream) into a ring of LDS slots by
//   direct-to-LDS loads, every set's loads issued up front where the ring
//   holds them.  Every weight is one field shift merged into an LDS address,
//   one lookup and one fp32 FMA; row sums are reduced in 8-lane groups by
//   DPP, then across groups through LDS after one barrier.
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
#include "nb_stream_common.h"

#include <algorithm>
#include <cstdint>
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
// (a & mask) | b in one VALU op, the mask in a scalar register (the disjoint
// `or` would otherwise become an add after a separate and).
__device__ __forceinline__ uint32_t and_or_s(uint32_t a, uint32_t mask, uint32_t b) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(mask), "v"(b));
    return r;
}

// LDS byte address of codebook entry (field j) in the lane's table:
// `base` | field << POS.  POS = 8 for a lane's entry-major copy (the wave's
// table holds entry e of lane l at byte 256 e + 4 l, so every lookup of a
// wave hits a bank of its own); POS = 2 for the block's own NE entries where
// they landed in LDS.  `base` has zeros in the field's bits.  The field is
// shifted straight to bit POS and merged with the base: two VALU ops a
// weight (the fields of a 3-bit slice that straddle a dword take a funnel
// shift).
template <int BITS, int J, int POS>
__device__ __forceinline__ uint32_t entry_offset(const uint32_t (&d)[BITS], uint32_t base) {
    constexpr int bit = J * BITS;
    constexpr int w = bit >> 5;
    constexpr int off = bit & 31;
    constexpr uint32_t kMask = ((1u << BITS) - 1u) << POS;
    uint32_t v;
    if constexpr (off + BITS > 32) {
        v = __builtin_amdgcn_alignbit(d[w + 1], d[w], off - POS);
    } else if constexpr (off >= POS) {
        v = d[w] >> (off - POS);
    } else {
        v = d[w] << (POS - off);
    }
    return and_or_s(v, kMask, base);
}

typedef __attribute__((address_space(3))) const float lds_f32;

template <int BITS, int POS, int J0, int... Js>
__device__ __forceinline__ void lookup8(const uint32_t (&d)[BITS], uint32_t base, float (&w)[8],
                                        std::integer_sequence<int, Js...>) {
    ((w[Js] = *(lds_f32*)(uintptr_t)entry_offset<BITS, J0 + Js, POS>(d, base)), ...);
}

// sum_j cb[field j] * x[j] over the 32 weights of a slice.  Lookups are
// issued eight at a time into registers before the FMAs so that the LDS
// latency overlaps, and two accumulators shorten the FMA chain.
template <int BITS, int POS>
__device__ __forceinline__ float slice_dot(const uint32_t (&d)[BITS], uint32_t base,
                                           const float (&xr)[32]) {
    float a0 = 0.f, a1 = 0.f;
    float w[4][8];
    lookup8<BITS, POS, 0>(d, base, w[0], std::make_integer_sequence<int, 8>{});
    lookup8<BITS, POS, 8>(d, base, w[1], std::make_integer_sequence<int, 8>{});
    lookup8<BITS, POS, 16>(d, base, w[2], std::make_integer_sequence<int, 8>{});
    lookup8<BITS, POS, 24>(d, base, w[3], std::make_integer_sequence<int, 8>{});
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

// ---- the M == 1 kernel: row-sets streamed into LDS -------------------------
//
// A workgroup owns `per` consecutive row-sets of P rows: P * S lanes (S =
// K / 32 slices a row), one 32-weight slice each, and every lane keeps its
// slice's 32 activations in registers for all of its sets.  The activations
// are staged once per workgroup.  Each wave streams the bytes of its own 64
// slices of a set -- their index bytes and their blocks' codebooks, both
// contiguous in the stream -- into a ring of `depth` LDS slots by
// direct-to-LDS loads (untracked by the compiler; every wait is a counted
// `s_waitcnt vmcnt`), and looks the codebook entries up where they landed.
// The partial sums of up to kFastRedSets sets are reduced after one barrier.

template <int BITS, int BS>
struct FastGeom {
    static constexpr int NE = 1 << BITS;
    static constexpr int SPB = BS / 32;                   // slices per block
    static constexpr int kIdxBytes = 64 * 4 * BITS;       // a wave's 64 slices
    static constexpr int kCbBytes = (64 / SPB) * NE * 4;  // their blocks' entries
    static constexpr int kSlotBytes = kIdxBytes + kCbBytes;
    // Lanes of one block look its entries up where they landed when a
    // half-wave's tables fill its 32 banks at most once (BS >= 128 at 8
    // entries: SPB lanes read one table, each entry in a bank of its own);
    // with more tables a half-wave (BS 64) each lane copies its block's
    // entries into an entry-major column of its own.
    static constexpr bool kPrivate = SPB <= 2;
    static constexpr int kLoads = (kIdxBytes + 1023) / 1024 + (kCbBytes + 1023) / 1024;
};
constexpr int kFastMaxDepth = 8;      // LDS slots per wave
constexpr int kFastRedSets = 8;       // sets reduced together
constexpr int kFastMaxThreads = 1024;
constexpr int kFastMinWaves = 8;      // (fewer leave the lookups' latency exposed)

// NBYTES contiguous bytes from src to LDS byte address `lds`, 16 bytes a
// lane: ceil(NBYTES / 1024) instructions, lanes past NBYTES masked off in
// the last; sources past `last` read `last` (those bytes are never used).
template <int NBYTES>
__device__ __forceinline__ void dma_bytes(uint32_t lds, const uint8_t* src, const uint8_t* last,
                                          int lane) {
#pragma unroll
    for (int p = 0; p < (NBYTES + 1023) / 1024; ++p) {
        const uint8_t* sp = src + p * 1024 + 16 * lane;
        sp = sp < last ? sp : last;
        const uint32_t dst = __builtin_amdgcn_readfirstlane(lds + p * 1024);
        if (p * 1024 + 1024 <= NBYTES || p * 1024 + 16 * lane < NBYTES) {
            stream::dma16<0>(dst, sp);
        }
    }
}

// Waits until at most n vector-memory operations of the wave are
// outstanding (n a multiple of STEP, at most N; n becomes the immediate).
template <int N, int STEP>
__device__ __forceinline__ void wait_vm_le(int n) {
    if constexpr (N > 0) {
        if (n >= N) {
            stream::wait_vm<N>();
            return;
        }
        wait_vm_le<N - STEP, STEP>(n);
    } else {
        stream::wait_vm<0>();
    }
}

template <int BITS, int BS, bool kXBF16>
__global__ __launch_bounds__(kFastMaxThreads) void gemv_fast_kernel(
    const void* __restrict__ x, const uint8_t* __restrict__ packed,
    const float* __restrict__ cb, void* __restrict__ y, int y_dtype, int N, int K, int P,
    int n_sets, int depth) {
    using G = FastGeom<BITS, BS>;
    extern __shared__ __align__(16) unsigned char smem[];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int nwaves = blockDim.x >> 6;
    const int S = K >> 5;
    const int xbytes = K * (kXBF16 ? 2 : 4);
    // LDS: the waves' entry-major tables if any (NE * 256 bytes each, from
    // the first multiple of that size: a lookup address is the table's
    // address OR'ed with field << 8), the staged activations, the waves'
    // rings (from a 64-byte boundary: a block's entries start at a multiple
    // of NE * 4 bytes), the reduction buffer
    constexpr uint32_t kTab = G::kPrivate ? G::NE * 256 : 64;
    const uint32_t smem_lds = stream::lds_addr(smem);
    const uint32_t tab0 = ((smem_lds + kTab - 1) & ~(kTab - 1)) - smem_lds;
    float* tabw = reinterpret_cast<float*>(smem + tab0 + wave * kTab);
    unsigned char* xsm = smem + tab0 + (G::kPrivate ? nwaves * kTab : 0);
    unsigned char* ring = xsm + xbytes + wave * depth * G::kSlotBytes;
    float* red = reinterpret_cast<float*>(xsm + xbytes + nwaves * depth * G::kSlotBytes);
    const int nred = blockDim.x >> 3;  // 8-lane groups
    // set i of this workgroup is blockIdx.x + i * gridDim.x: at any step the
    // workgroups read one contiguous stretch of the stream together
    const int G0 = gridDim.x;
    const int count = (n_sets - (int)blockIdx.x + G0 - 1) / G0;
    auto set_of = [&](int i) { return (int)blockIdx.x + i * G0; };

    // ---- the activations, 16-byte pieces to LDS: piece j of slice s at
    //      place j ^ (s & 7) (fp32) or j ^ ((s >> 1) & 3) (bf16) of the
    //      slice, so 8 consecutive lanes read 8 different bank groups
    const int npieces = xbytes >> 4;
    {
        const uint32_t xs = stream::lds_addr(xsm);
        for (int q = wave; q * 64 < npieces; q += nwaves) {
            const int p = q * 64 + lane;
            int sp;
            if (kXBF16) {
                const int s = p >> 2;
                sp = (s << 2) | ((p & 3) ^ ((s >> 1) & 3));
            } else {
                const int s = p >> 3;
                sp = (s << 3) | ((p & 7) ^ (s & 7));
            }
            sp = sp < npieces ? sp : npieces - 1;
            const uint32_t dst = __builtin_amdgcn_readfirstlane(xs + q * 1024);
            if (p < npieces) stream::dma16<0>(dst, static_cast<const uint8_t*>(x) + 16 * sp);
        }
    }

    // ---- the sets' bytes: the wave's 64 slices of set i start at slice g0
    const int64_t nslices = (int64_t)N * S;
    const uint8_t* pk_last = packed + nslices * (4 * BITS) - 16;
    const uint8_t* cbb = reinterpret_cast<const uint8_t*>(cb);
    const uint8_t* cb_last = cbb + (nslices / G::SPB) * (G::NE * 4) - 16;
    const uint32_t ring_lds = stream::lds_addr(ring);
    int slot_in = 0;
    auto issue = [&](int i) {
        const int64_t g0 = (int64_t)set_of(i) * P * S + wave * 64;
        const uint32_t dst = ring_lds + slot_in * G::kSlotBytes;
        dma_bytes<G::kIdxBytes>(dst, packed + g0 * (4 * BITS), pk_last, lane);
        dma_bytes<G::kCbBytes>(dst + G::kIdxBytes, cbb + (g0 / G::SPB) * (G::NE * 4), cb_last,
                               lane);
        slot_in = slot_in + 1 == depth ? 0 : slot_in + 1;
    };
    const int first = min(count, depth);
    for (int i = 0; i < first; ++i) issue(i);
    // the wave's activation pieces went out first: they are in once at most
    // the sets' loads remain
    wait_vm_le<kFastMaxDepth * G::kLoads, G::kLoads>(first * G::kLoads);
    __syncthreads();

    // ---- the lane's slice and its activations
    const bool lane_on = t < P * S;
    const int row_sub = t / S;
    const int s = t - row_sub * S;
    float xr[32];
    if (kXBF16) {
        const uint4* xp = reinterpret_cast<const uint4*>(xsm) + s * 4;
        const int sw = (s >> 1) & 3;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint4 u = xp[j ^ sw];
            const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                xr[j * 8 + 2 * h] = __uint_as_float(w4[h] << 16);
                xr[j * 8 + 2 * h + 1] = __uint_as_float(w4[h] & 0xFFFF0000u);
            }
        }
    } else {
        const float4* xp = reinterpret_cast<const float4*>(xsm) + s * 8;
        const int sw = s & 7;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float4 f = xp[j ^ sw];
            xr[4 * j] = f.x;
            xr[4 * j + 1] = f.y;
            xr[4 * j + 2] = f.z;
            xr[4 * j + 3] = f.w;
        }
    }

    // ---- the sets
    const uint32_t pbase = stream::lds_addr(tabw) + (uint32_t)(lane * 4);
    int slot_out = 0;
    for (int i = 0; i < count; ++i) {
        // set i's loads are in once at most the later sets' loads remain
        const int after = min(count, i + depth) - (i + 1);
        wait_vm_le<(kFastMaxDepth - 1) * G::kLoads, G::kLoads>(after * G::kLoads);
        unsigned char* slot = ring + slot_out * G::kSlotBytes;
        slot_out = slot_out + 1 == depth ? 0 : slot_out + 1;
        uint32_t d[BITS];
        const uint32_t* ip = reinterpret_cast<const uint32_t*>(slot) + lane * BITS;
#pragma unroll
        for (int w = 0; w < BITS; ++w) d[w] = ip[w];
        float* blk = reinterpret_cast<float*>(slot + G::kIdxBytes) + (lane / G::SPB) * G::NE;
        float acc;
        if constexpr (G::kPrivate) {
            // the lane's block entries into its column of the wave's
            // entry-major table (bf16 activations multiply the entries
            // rounded to bf16, the reference's bf16 path); a lane reads back
            // only what it wrote
#pragma unroll
            for (int e4 = 0; e4 < G::NE / 4; ++e4) {
                const float4 v = reinterpret_cast<const float4*>(blk)[e4];
                const float ev[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    tabw[(4 * e4 + h) * 64 + lane] = kXBF16 ? round_bf16(ev[h]) : ev[h];
                }
            }
            acc = slice_dot<BITS, 8>(d, pbase, xr);
        } else {
            if constexpr (kXBF16) {
                // the slot's entries rounded to bf16 in place, a share per
                // lane; a wave's LDS operations complete in issue order
                float* cbs = reinterpret_cast<float*>(slot + G::kIdxBytes);
#pragma unroll
                for (int e = 0; e < G::kCbBytes / 4; e += 64) {
                    if (e + lane < G::kCbBytes / 4) cbs[e + lane] = round_bf16(cbs[e + lane]);
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
            acc = slice_dot<BITS, 2>(d, stream::lds_addr(blk), xr);
        }
        stream::wait_lds();  // the slot's reads are done before it is refilled
        if (i + depth < count) issue(i + depth);
        const bool valid = lane_on && set_of(i) * P + row_sub < N;
        acc = valid ? acc : 0.f;
        // 8 consecutive lanes always belong to one row (S % 8 == 0): pair,
        // quad, then half-row sums by DPP moves (lane 0 of the 8 adds the
        // same two quad sums as a lane ^ 4 exchange would)
        acc += dpp_mov<0xB1>(acc);   // quad_perm(1, 0, 3, 2)
        acc += dpp_mov<0x4E>(acc);   // quad_perm(2, 3, 0, 1)
        acc += dpp_mov<0x141>(acc);  // row_half_mirror
        const int gi = i % kFastRedSets;
        if ((t & 7) == 0) red[gi * nred + (t >> 3)] = acc;
        if (gi == kFastRedSets - 1 || i + 1 == count) {
            __syncthreads();
            if (t < (gi + 1) * P) {
                const int il = t / P, r = t - il * P;
                const int orow = set_of(i - gi + il) * P + r;
                if (orow < N) {
                    const int ng = S >> 3;
                    const float* rr = red + il * nred + r * ng;
                    float sum = 0.f;
                    for (int g = 0; g < ng; ++g) sum += rr[g];
                    store_y(y, y_dtype, orow, sum);
                }
            }
            __syncthreads();  // red is written again by the next sets
        }
    }
    stream::wait_vm<0>();  // (nothing is in flight here; kept as a guard)
}

typedef void (*FastFn)(const void*, const uint8_t*, const float*, void*, int, int, int, int,
                       int, int);

// Launch shape of gemv_fast_kernel: P rows a set (P * S <= kFastMaxThreads
// lanes, at least kFastMinWaves waves where K allows), one workgroup per CU
// with at most `per` sets each (set i of workgroup b is b + i * grid); the
// shape with the fewest slices per SIMD (per x waves) wins, then the one
// with fewer sets per workgroup.  `depth` slots per wave fit in LDS beside
// the staged activations, the tables and the reduction buffer.
struct FastPlan {
    int P = 0, per = 0, grid = 0, threads = 0, depth = 0;
    size_t lds = 0;
};

template <int BITS, int BS>
FastPlan fast_plan_t(int N, int K, bool xb, int cus, size_t lds_max) {
    using G = FastGeom<BITS, BS>;
    const int S = K / 32;
    const int min_waves = std::min(kFastMinWaves, (kFastMaxThreads / S) * S / 64);
    FastPlan best;
    int64_t best_cost = INT64_MAX;
    for (int P = 1; P * S <= kFastMaxThreads; ++P) {
        const int waves = (P * S + 63) / 64;
        if (waves < min_waves) continue;
        const int64_t n_sets = (N + P - 1) / P;
        const int64_t per = (n_sets + cus - 1) / cus;
        const int64_t grid = (n_sets + per - 1) / per;
        const size_t tables = G::kPrivate ? (size_t)(waves + 1) * G::NE * 256 : 64;
        const size_t fixed = (size_t)K * (xb ? 2 : 4) + tables + (size_t)waves * 64 * 4;
        if (fixed >= lds_max) continue;
        const int64_t room = (int64_t)(lds_max - fixed) / ((int64_t)waves * G::kSlotBytes);
        const int depth = (int)std::min<int64_t>(std::min<int64_t>(per, kFastMaxDepth), room);
        if (depth < 1) continue;
        const int64_t cost = per * waves;
        if (cost < best_cost || (cost == best_cost && per < best.per)) {
            best_cost = cost;
            best.P = P;
            best.per = (int)per;
            best.grid = (int)grid;
            best.threads = waves * 64;
            best.depth = depth;
            best.lds = fixed + (size_t)waves * depth * G::kSlotBytes;
        }
    }
    return best;
}

template <int BITS, int BS>
FastFn pick_x(bool xb, int N, int K, int cus, size_t lds_max, FastPlan& plan) {
    plan = fast_plan_t<BITS, BS>(N, K, xb, cus, lds_max);
    return xb ? gemv_fast_kernel<BITS, BS, true> : gemv_fast_kernel<BITS, BS, false>;
}

template <int BITS>
FastFn pick_bs(int bs, bool xb, int N, int K, int cus, size_t lds_max, FastPlan& plan) {
    switch (bs) {
        case 64: return pick_x<BITS, 64>(xb, N, K, cus, lds_max, plan);
        case 128: return pick_x<BITS, 128>(xb, N, K, cus, lds_max, plan);
        case 256: return pick_x<BITS, 256>(xb, N, K, cus, lds_max, plan);
    }
    return nullptr;
}

FastFn pick_fast(int bits, int bs, bool xb, int N, int K, int cus, size_t lds_max,
                 FastPlan& plan) {
    switch (bits) {
        case 2: return pick_bs<2>(bs, xb, N, K, cus, lds_max, plan);
        case 3: return pick_bs<3>(bs, xb, N, K, cus, lds_max, plan);
        case 4: return pick_bs<4>(bs, xb, N, K, cus, lds_max, plan);
    }
    return nullptr;
}

bool fast_eligible(const GemvArgs& a) {
    if (a.M != 1) return false;
    if (a.bits < 2 || a.bits > 4 || a.n_entries != (1 << a.bits)) return false;
    if (a.block_size != 64 && a.block_size != 128 && a.block_size != 256) return false;
    if (a.K <= 0 || a.K % 256 != 0 || a.K % a.block_size != 0 || a.K / 32 > kThreads) return false;
    // 16-byte direct-to-LDS loads of the stream, the codebook and x
    if (reinterpret_cast<uintptr_t>(a.packed) % 16 != 0) return false;
    if (reinterpret_cast<uintptr_t>(a.codebook) % 16 != 0) return false;
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
        FastPlan plan;
        FastFn fn = pick_fast(a.bits, a.block_size, a.x_dtype == NB_BF16, a.N, a.K, cus,
                              (size_t)device_lds_bytes(), plan);
        if (fn == nullptr || plan.P == 0) return fail(NB_EUNSUPPORTED, "nb_gemv: no launch shape");
        const int n_sets = (a.N + plan.P - 1) / plan.P;
        hipLaunchKernelGGL(fn, dim3(plan.grid), dim3(plan.threads), plan.lds, stream, a.x,
                           a.packed, a.codebook, a.y, a.y_dtype, a.N, a.K, plan.P, n_sets,
                           plan.depth);
        return check_launch("nb_gemv (fast)");
    }
    int64_t grid = a.N;
    if (grid > (int64_t)cus * 16) grid = (int64_t)cus * 16;
    hipLaunchKernelGGL(gemv_generic_kernel, dim3((int)grid), dim3(kThreads), 0, stream, a);
    return check_launch("nb_gemv (generic)");
}

}  // namespace nb
