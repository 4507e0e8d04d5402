// Prefill: dense contraction with a packed weight (gfx950).
//
//   Y[m][n] = sum_k X[m][k] * bf16(W[n][k]),   W 3-bit / 8-entry / block-128
//
// for many activation rows at once (M >= 16 or so; the decode path is the
// GEMV).  The reference computes this as unpack + gather + a dense matmul
// that materialises W on every call (inference/triton_kernel.py:258-275;
// in bf16, inference/eval_ppl.py:149-174).  Here each 128 x 128 output tile
// of a 256-thread workgroup walks K in steps of 128 -- exactly one codebook
// block per weight row per step:
//
//   * the X tile (128 rows x 128 bf16) is loaded with global_load_lds_dwordx4
//     (one contiguous KiB of four rows per instruction); lanes pick their
//     16-byte chunk so that chunk c of row r lands in LDS slot c ^ (r & 15)
//     of the row, which makes the MFMA operand reads bank-conflict free;
//   * the W tile is read packed (48 index bytes + 32 codebook bytes per row
//     per step), turned into bf16 with v_perm_b32 lookups into the block's
//     codebook byte planes, and stored in LDS with the same swizzle;
//   * four waves each own a 64 x 64 quarter of the tile, 4 x 4
//     v_mfma_f32_16x16x32_bf16 tiles, fp32 accumulation;
//   * two LDS stages: the next step's loads and dequantization overlap the
//     current step's MFMAs.
// Weights are the codebook entries rounded to bf16 (RNE), as the bf16 path.
#include <algorithm>

#include "nb_device.h"
#include "nb_internal.h"

namespace nb {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;

constexpr int kBM = 128, kBN = 128, kBK = 128;
constexpr int kThreads = 256;
constexpr int kTileBytes = kBM * kBK * 2;  // 32 KiB per operand tile
constexpr int kStageBytes = 2 * kTileBytes;

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
    bf16x2_t v;
    v.x = (__bf16)lo;
    v.y = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
}

// 8 bf16 weights (natural order) of one 24-bit index group from the byte
// planes of the block's codebook: two selectors of four 3-bit indices, four
// v_perm_b32 lookups, two interleaves per bf16 pair.
__device__ __forceinline__ u32x4_t lookup8(uint32_t g, uint32_t lo0, uint32_t lo1, uint32_t hi0,
                                           uint32_t hi1) {
    const uint32_t h = (g & 0xfffu) | ((g << 4) & 0x0fff0000u);  // i0-3 low half, i4-7 high
    const uint32_t sa = (h & 0x00070007u) | ((h << 5) & 0x07000700u);          // i0 i1 i4 i5
    const uint32_t sb = ((h >> 6) & 0x00070007u) | ((h >> 1) & 0x07000700u);   // i2 i3 i6 i7
    const uint32_t la = __builtin_amdgcn_perm(lo1, lo0, sa);
    const uint32_t ha = __builtin_amdgcn_perm(hi1, hi0, sa);
    const uint32_t lb = __builtin_amdgcn_perm(lo1, lo0, sb);
    const uint32_t hb = __builtin_amdgcn_perm(hi1, hi0, sb);
    u32x4_t w;
    w.x = __builtin_amdgcn_perm(ha, la, 0x05010400u);  // i0 i1
    w.y = __builtin_amdgcn_perm(hb, lb, 0x05010400u);  // i2 i3
    w.z = __builtin_amdgcn_perm(ha, la, 0x07030602u);  // i4 i5
    w.w = __builtin_amdgcn_perm(hb, lb, 0x07030602u);  // i6 i7
    return w;
}

// LDS byte offset of 16-byte chunk c (0..15) of tile row r.
__device__ __forceinline__ uint32_t swz(int r, int c) {
    return (uint32_t)((r * 16 + (c ^ (r & 15))) * 16);
}

__device__ __forceinline__ void dma16(uint32_t lds, const void* src) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(lds), "v"(src)
                 : "memory", "m0");
}

template <typename T>
__device__ __forceinline__ uint32_t lds_addr(T* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) T*)p;
}

struct PrefillArgs {
    const uint16_t* x;
    int64_t ldx;
    const uint8_t* packed;
    const float* codebook;
    void* y;
    int64_t ldy;
    int y_dtype;
    int M, N, K;
};

__global__ __launch_bounds__(kThreads) void prefill_kernel(PrefillArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = blockIdx.x * kBN, m0 = blockIdx.y * kBM;
    const int bpr = a.K / kBK;
    const uint32_t base = lds_addr(smem);

    // X tile loads: instruction i of wave w covers tile rows 32w + 4i .. +3;
    // lane l fills LDS slot (l & 15) of row 32w + 4i + (l >> 4)
    auto load_x = [&](int step, int stage) {
        const uint32_t sbase = base + stage * kStageBytes;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = wave * 32 + 4 * i + (lane >> 4);
            const int slot = lane & 15;
            const int c = slot ^ (r & 15);
            const int gm = min(m0 + r, a.M - 1);
            const uint16_t* src = a.x + (int64_t)gm * a.ldx + (int64_t)step * kBK + c * 8;
            dma16(__builtin_amdgcn_readfirstlane(sbase + (wave * 32 + 4 * i) * 256), src);
        }
    };
    // W tile: thread t dequantizes half h = t & 1 (64 weights) of row t >> 1
    const int wr = tid >> 1, wh = tid & 1;
    const int gn = min(n0 + wr, a.N - 1);
    auto load_w = [&](int step, uint32_t (&d)[6], u32x4_t& c0, u32x4_t& c1) {
        const int64_t blk = (int64_t)gn * bpr + step;
        const uint2* ip = reinterpret_cast<const uint2*>(a.packed + blk * 48 + wh * 24);
        const uint2 v0 = ip[0], v1 = ip[1], v2 = ip[2];
        d[0] = v0.x; d[1] = v0.y; d[2] = v1.x; d[3] = v1.y; d[4] = v2.x; d[5] = v2.y;
        const u32x4_t* cp = reinterpret_cast<const u32x4_t*>(a.codebook + blk * 8);
        c0 = cp[0];
        c1 = cp[1];
    };
    auto store_w = [&](int stage, const uint32_t (&d)[6], const u32x4_t& c0, const u32x4_t& c1) {
        const uint32_t q0 = pack_bf16x2(__uint_as_float(c0.x), __uint_as_float(c0.y));
        const uint32_t q1 = pack_bf16x2(__uint_as_float(c0.z), __uint_as_float(c0.w));
        const uint32_t q2 = pack_bf16x2(__uint_as_float(c1.x), __uint_as_float(c1.y));
        const uint32_t q3 = pack_bf16x2(__uint_as_float(c1.z), __uint_as_float(c1.w));
        const uint32_t lo0 = __builtin_amdgcn_perm(q1, q0, 0x06040200u);
        const uint32_t hi0 = __builtin_amdgcn_perm(q1, q0, 0x07050301u);
        const uint32_t lo1 = __builtin_amdgcn_perm(q3, q2, 0x06040200u);
        const uint32_t hi1 = __builtin_amdgcn_perm(q3, q2, 0x07050301u);
        unsigned char* wt = smem + stage * kStageBytes + kTileBytes;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            // group j (8 indices) of this half: 24 bits at bit 24 j of d
            const int bit = 24 * j;
            const int w = bit >> 5, off = bit & 31;
            uint32_t g;
            if (off == 0) {
                g = d[w];
            } else if (off + 24 <= 32) {
                g = d[w] >> off;
            } else {
                g = __builtin_amdgcn_alignbit(d[w + 1], d[w], off);
            }
            const u32x4_t wv = lookup8(g, lo0, lo1, hi0, hi1);
            *reinterpret_cast<u32x4_t*>(wt + swz(wr, wh * 8 + j)) = wv;
        }
    };

    // wave (wm, wn) owns rows 64 wm .. +63 and columns 64 wn .. +63
    const int wm = wave >> 1, wn = wave & 1;
    const int fr = lane & 15, fq = lane >> 4;
    f32x4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    uint32_t d[6];
    u32x4_t c0, c1;
    load_x(0, 0);
    load_w(0, d, c0, c1);
    store_w(0, d, c0, c1);
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
    __syncthreads();

    for (int step = 0; step < bpr; ++step) {
        const int cur = step & 1;
        const bool more = step + 1 < bpr;
        if (more) {
            load_x(step + 1, cur ^ 1);
            load_w(step + 1, d, c0, c1);
        }
        const unsigned char* xt = smem + cur * kStageBytes;
        const unsigned char* wt = xt + kTileBytes;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {  // 32 columns of K per MFMA
            const int c = ks * 4 + fq;
            u32x4_t av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                av[i] = *reinterpret_cast<const u32x4_t*>(xt + swz(wm * 64 + i * 16 + fr, c));
                bv[i] = *reinterpret_cast<const u32x4_t*>(wt + swz(wn * 64 + i * 16 + fr, c));
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8_t, av[i]), __builtin_bit_cast(bf16x8_t, bv[j]),
                        acc[i][j], 0, 0, 0);
        }
        if (more) store_w(cur ^ 1, d, c0, c1);
        asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
        __syncthreads();
    }

    // D fragment: lane holds rows 4 fq .. 4 fq + 3 of column fr of tile (i, j)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + wn * 64 + j * 16 + fr;
            if (n >= a.N) continue;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int m = m0 + wm * 64 + i * 16 + fq * 4 + e;
                if (m >= a.M) continue;
                const float v = acc[i][j][e];
                if (a.y_dtype == NB_BF16) {
                    static_cast<bf16_bits*>(a.y)[(int64_t)m * a.ldy + n] = f32_to_bf16_rne(v);
                } else {
                    static_cast<float*>(a.y)[(int64_t)m * a.ldy + n] = v;
                }
            }
        }
}

}  // namespace

int launch_prefill(const void* x, int64_t ldx, const uint8_t* packed, const float* codebook,
                   void* y, int y_dtype, int64_t ldy, int M, int N, int K, hipStream_t stream) {
    PrefillArgs a;
    a.x = static_cast<const uint16_t*>(x);
    a.ldx = ldx;
    a.packed = packed;
    a.codebook = codebook;
    a.y = y;
    a.ldy = ldy;
    a.y_dtype = y_dtype;
    a.M = M;
    a.N = N;
    a.K = K;
    const dim3 grid((N + kBN - 1) / kBN, (M + kBM - 1) / kBM);
    hipLaunchKernelGGL(prefill_kernel, grid, dim3(kThreads), 2 * kStageBytes, stream, a);
    return check_launch("nb_gemm_prefill");
}

}  // namespace nb
