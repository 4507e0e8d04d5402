// Packed 3-bit GEMV / skinny GEMM with bf16 activations on gfx950:
// register codebook lookups (v_perm_b32) feeding bf16 MFMA.
//
//   y[m][n] = sum_k x[m][k] * bf16(W[n][k]),  m < M <= 16
//
// Weights are rounded to bf16 (round to nearest even) before the multiply,
// the reference's bf16 semantics (inference/eval_ppl.py:149-174:
// W.to(torch.bfloat16) then a bf16 matmul with fp32 accumulation).
//
// Work split.  One workgroup owns 16 output rows and all of K; its W waves
// split the row's 128-weight blocks into "steps" of 4 blocks.  In a step,
// lane l = q*16 + r takes row r, block 4*step + q: 48 bytes of packed
// indices (3 x 16-byte loads; the 4 lanes of a row read 192 contiguous
// bytes) and the block's 8 fp32 codebook entries.  The lane then produces
// its 128 bf16 weights as 16 MFMA A-operands (8 consecutive weights each) of
// v_mfma_f32_16x16x32_bf16, whose B operand is the matching 8 activations of
// each of the 16 MFMA columns (= the M rows of x; M == 1 leaves 15 unused).
// The accumulator stays in registers for the whole K range; the W partial
// results are summed through LDS once at the end.
//
// Codebook lookup without memory.  The block's 8 bf16 entries are split into
// byte planes (LO0/LO1 = low bytes of entries 0-3/4-7, HI0/HI1 = high bytes).
// For four indices placed one per byte of a selector S, v_perm_b32(LO1, LO0,
// S) returns their four low bytes and v_perm_b32(HI1, HI0, S) the high bytes;
// two more v_perm_b32 interleave them into two bf16x2 dwords.  A 24-bit group
// of eight 3-bit indices becomes two selectors in 9 VALU ops, so eight
// weights cost 17 VALU ops and no LDS traffic.
#include "nb_device.h"
#include "nb_internal.h"

namespace nb {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;

constexpr int kMaxWaves = 16;
constexpr int kLdsXRows = 4;   // x rows staged in LDS (more rows: read from L2)

// Waves launched per CU (spread over the 16-row groups).
#ifndef NB_MFMA_WAVES_PER_CU
#define NB_MFMA_WAVES_PER_CU 16
#endif
// Stage x in LDS when it fits (1) or always read it from global memory (0).
#ifndef NB_MFMA_X_LDS
#define NB_MFMA_X_LDS 1
#endif

// One packed bf16x2 from two floats, round to nearest even.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
    bf16x2_t v;
    v.x = (__bf16)lo;
    v.y = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
}

// 8 bf16 weights (natural order) of one 24-bit index group `g` (bits above
// 24 are ignored) from the byte planes lo0/lo1/hi0/hi1.
__device__ __forceinline__ u32x4_t lookup8(uint32_t g, uint32_t lo0, uint32_t lo1,
                                           uint32_t hi0, uint32_t hi1) {
    // halves: lo16 = indices 0-3 at bits 0,3,6,9; hi16 = indices 4-7 likewise
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

// Group j (0..15) of a 128-index block held in 12 dwords.
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

struct StepRegs {
    uint32_t d[12];   // 48 bytes of packed indices
    float c[8];       // the block's codebook
};

__device__ __forceinline__ void load_step(const uint8_t* __restrict__ packed,
                                          const float* __restrict__ cb,
                                          int64_t row, int bcol, int bpr, int64_t row_bytes,
                                          StepRegs& s) {
    const u32x4_t* p = reinterpret_cast<const u32x4_t*>(packed + row * row_bytes + (int64_t)bcol * 48);
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
__device__ __forceinline__ void mfma_groups(const StepRegs& s, uint32_t lo0, uint32_t lo1,
                                            uint32_t hi0, uint32_t hi1,
                                            const u32x4_t* __restrict__ bsrc, f32x4_t& acc) {
    if constexpr (J < 16) {
        const u32x4_t a = lookup8(group24<J>(s.d), lo0, lo1, hi0, hi1);
        const u32x4_t b = bsrc[J];
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                      __builtin_bit_cast(bf16x8_t, b), acc,
                                                      0, 0, 0);
        mfma_groups<J + 1>(s, lo0, lo1, hi0, hi1, bsrc, acc);
    }
}

// Consumes one step: byte planes of the codebook (zeroed when the lane has
// no block here, so its weights are 0) and 16 MFMAs.
__device__ __forceinline__ void compute_step(const StepRegs& s, bool live,
                                             const u32x4_t* __restrict__ bsrc,
                                             f32x4_t& acc) {
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
    mfma_groups<0>(s, lo0, lo1, hi0, hi1, bsrc, acc);
}

__device__ __forceinline__ void store_out(void* y, int dtype, int64_t i, float v) {
    if (dtype == NB_BF16) {
        static_cast<bf16_bits*>(y)[i] = f32_to_bf16_rne(v);
    } else {
        static_cast<float*>(y)[i] = v;
    }
}

// kXLds: x (M <= kLdsXRows rows) is staged in LDS and B operands are LDS
// reads, which leaves vmcnt to the weight stream, so the next step's weight
// loads are kept in flight while a step is consumed.  Otherwise B operands
// are read from global memory (L2-resident) and each step is loaded, then
// consumed (an in-order vmcnt wait for a B load would also wait for any
// prefetch issued before it).
template <bool kXLds>
__global__ __launch_bounds__(64 * kMaxWaves) void gemv_mfma3_kernel(
    const bf16_bits* __restrict__ x, int64_t ldx, const uint8_t* __restrict__ packed,
    const float* __restrict__ cb, void* __restrict__ y, int y_dtype, int64_t ldy,
    int M, int N, int K) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int nwaves = blockDim.x >> 6;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int r = lane & 15;
    const int q = lane >> 4;
    const int bpr = K >> 7;
    const int nsteps = (bpr + 3) >> 2;
    const int64_t row_bytes = (int64_t)bpr * 48;
    const int row0 = blockIdx.x * 16;
    const int row = row0 + r;
    const int64_t lrow = row < N ? row : N - 1;   // clamped: loads stay in bounds
    const bool row_ok = row < N;

    const int s_begin = (int)(((int64_t)wave * nsteps) / nwaves);
    const int s_end = (int)(((int64_t)(wave + 1) * nsteps) / nwaves);
    auto bcol_of = [&](int st) {
        const int b = st * 4 + q;
        return b < bpr ? b : bpr - 1;
    };

    // Issue the first step's loads before anything waits.
    StepRegs cur, nxt;
    load_step(packed, cb, lrow, bcol_of(s_begin), bpr, row_bytes, cur);

    bf16_bits* xs = reinterpret_cast<bf16_bits*>(smem);
    float* red = reinterpret_cast<float*>(smem + (kXLds ? (size_t)M * K * 2 : 0));
    if (kXLds) {
        const int chunks = (K >> 3);  // 16-byte chunks per row
        for (int i = t; i < M * chunks; i += blockDim.x) {
            const int m = i / chunks, c = i - m * chunks;
            reinterpret_cast<u32x4_t*>(xs + (int64_t)m * K)[c] =
                reinterpret_cast<const u32x4_t*>(x + m * ldx)[c];
        }
        __syncthreads();
    }

    const int xm = r < M ? r : M - 1;  // MFMA column r holds x row r
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    auto consume = [&](int st, const StepRegs& s) {
        const int b = st * 4 + q;
        const bool live = row_ok && b < bpr;
        const int bc = b < bpr ? b : bpr - 1;
        const u32x4_t* bsrc = kXLds
            ? reinterpret_cast<const u32x4_t*>(xs + (int64_t)xm * K + bc * 128)
            : reinterpret_cast<const u32x4_t*>(x + (int64_t)xm * ldx + bc * 128);
        compute_step(s, live, bsrc, acc);
    };
    if (kXLds) {
        // Two-stage ring: the next step's loads are always issued (clamped to
        // a valid block, so the last one is a harmless cache hit) before the
        // current step is consumed.
        for (int st = s_begin; st < s_end; st += 2) {
            load_step(packed, cb, lrow, bcol_of(st + 1 < s_end ? st + 1 : st), bpr, row_bytes,
                      nxt);
            consume(st, cur);
            if (st + 1 < s_end) {
                load_step(packed, cb, lrow, bcol_of(st + 2 < s_end ? st + 2 : st + 1), bpr,
                          row_bytes, cur);
                consume(st + 1, nxt);
            }
        }
    } else {
        for (int st = s_begin; st < s_end; ++st) {
            if (st != s_begin) load_step(packed, cb, lrow, bcol_of(st), bpr, row_bytes, cur);
            consume(st, cur);
        }
    }

    // acc lane (c = r, g = q) holds C[4g + v][c] = partial y[c][row0 + 4g + v]
    float* mine = red + wave * 256;
#pragma unroll
    for (int v = 0; v < 4; ++v) mine[(4 * q + v) * 16 + r] = acc[v];
    __syncthreads();
    if (t < M * 16) {
        const int c = t >> 4;
        const int rr = t & 15;
        if (row0 + rr < N) {
            float s = 0.f;
            for (int w = 0; w < nwaves; ++w) s += red[w * 256 + rr * 16 + c];
            store_out(y, y_dtype, (int64_t)c * ldy + row0 + rr, s);
        }
    }
}

}  // namespace

// Launches the MFMA kernel when the problem is 3-bit / 8 entries / block 128
// with bf16 activations and aligned operands; returns 1 if not eligible.
int launch_gemv_mfma(const GemvArgs& a, hipStream_t stream) {
    if (a.x_dtype != NB_BF16 || a.bits != 3 || a.n_entries != 8 || a.block_size != 128) return 1;
    if (a.M < 1 || a.M > 16 || a.K <= 0 || a.K % 128 != 0) return 1;
    if (reinterpret_cast<uintptr_t>(a.packed) % 16 != 0) return 1;
    if (reinterpret_cast<uintptr_t>(a.codebook) % 16 != 0) return 1;
    if (reinterpret_cast<uintptr_t>(a.x) % 16 != 0) return 1;
    if (a.M > 1 && a.ldx % 8 != 0) return 1;
    const int bpr = a.K / 128;
    const int nsteps = (bpr + 3) / 4;
    const int groups = (a.N + 15) / 16;
    // enough waves to cover every SIMD a few times, at most one per step
    const int cus = device_cu_count();
    int waves = (int)(((int64_t)NB_MFMA_WAVES_PER_CU * cus + groups - 1) / groups);
    if (waves > nsteps) waves = nsteps;
    if (waves > kMaxWaves) waves = kMaxWaves;
    if (waves < 1) waves = 1;
    const size_t red_bytes = (size_t)waves * 1024;
    const size_t x_bytes = (size_t)a.M * a.K * 2;
    const bool x_lds = NB_MFMA_X_LDS && a.M <= kLdsXRows &&
                       x_bytes + red_bytes <= (size_t)device_lds_bytes();
    const size_t lds = (x_lds ? x_bytes : 0) + red_bytes;
    const bf16_bits* x = static_cast<const bf16_bits*>(a.x);
    const int64_t ldx = a.M > 1 ? a.ldx : (int64_t)a.K;
    const int64_t ldy = a.M > 1 ? a.ldy : (int64_t)a.N;
    if (x_lds) {
        hipLaunchKernelGGL(gemv_mfma3_kernel<true>, dim3(groups), dim3(64 * waves), lds, stream,
                           x, ldx, a.packed, a.codebook, a.y, a.y_dtype, ldy, a.M, a.N, a.K);
    } else {
        hipLaunchKernelGGL(gemv_mfma3_kernel<false>, dim3(groups), dim3(64 * waves), lds, stream,
                           x, ldx, a.packed, a.codebook, a.y, a.y_dtype, ldy, a.M, a.N, a.K);
    }
    return check_launch("nb_gemv (mfma)");
}

}  // namespace nb
