// Prefill contraction with a packed weight, large tiles (gfx950).
//
//   Y[m][n] = sum_k X[m][k] * bf16(W[n][k]),   W 3-bit / 8-entry / block-128
//
// The reference computes this as unpack + gather + a dense matmul that
// materialises W on every call (inference/triton_kernel.py:258-275; in bf16,
// inference/eval_ppl.py:149-174).  Here a 512-thread workgroup owns a BN x
// BM tile of Y^T (BN = 256 or 128 outputs x BM = 256, 128 or 64 tokens,
// chosen per launch by grid occupancy) and walks K in steps of 64:
//
//   * the X slice (BM tokens x 64 bf16) arrives by global_load_lds_dwordx4
//     (eight rows per instruction), 16-byte chunk c of row r in LDS slot
//     c ^ (r & 7), so that eight consecutive rows read one chunk from eight
//     different bank groups;
//   * the W slice (BN rows x 64 weights: 24 index bytes per row, the codebook
//     of the row's block) is loaded into registers two steps ahead; each
//     thread turns half a row (32 indices) into bf16 with v_perm_b32 lookups
//     into the block's codebook byte planes and stores it with the same
//     swizzle;
//   * eight waves (2 x 4) each own a (BN/4) x (BM/2) sub-tile of 16 x 16
//     v_mfma_f32_16x16x32_bf16 tiles with W as the A operand and X as B, so
//     a lane's accumulator holds four consecutive outputs n of one token m
//     and the epilogue stores them as one vector;
//   * two LDS stages and one barrier per step: while a step's MFMAs run, the
//     next step's X slice is in flight and its W slice is dequantized, and
//     the two waves of each SIMD overlap one's MFMAs with the other's
//     dequantization and LDS reads;
//   * a one-dimensional grid whose workgroups (dealt to the 8 XCDs in turn)
//     take tiles XCD by XCD in contiguous runs, so an XCD's L2 holds the X
//     tiles of one or two token blocks rather than of all of them.
// Weights are the codebook entries rounded to bf16 (RNE), as the bf16 path;
// accumulation is fp32.
#include <algorithm>
#include <type_traits>

#include "nb_device.h"
#include "nb_internal.h"

namespace nb {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;

// waves per workgroup: 8 (two per SIMD) or 4 (one per SIMD, 128 x 128 per wave)
#ifndef NB_PREFILL_WAVES
#define NB_PREFILL_WAVES 8
#endif
constexpr int kBK = 64;            // K per step: half a codebook block
constexpr int kRowBytes = kBK * 2; // bf16 bytes of one row of a slice

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

// LDS byte offset of 16-byte chunk c (0..7) of slice row r.
__device__ __forceinline__ uint32_t swz(int r, int c) {
    return (uint32_t)(r * kRowBytes + ((c ^ (r & 7)) << 4));
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

struct Prefill2Args {
    const uint16_t* x;
    int64_t ldx;
    const uint8_t* packed;
    const float* codebook;
    void* y;
    int64_t ldy;
    int y_dtype;
    int M, N, K;
    int ksplit;   // K ranges per output tile (1: the whole of K)
    float* part;  // ksplit > 1: fp32 partial products [ksplit][M][N], else null
    int accumulate;  // fp32 y only: y += result instead of y = result
};

// Tile of the calling workgroup.  Workgroups are dealt to the 8 XCDs in
// turn (workgroup g to XCD g % 8), each XCD with its own L2: XCD x takes a
// contiguous run of the tiles in (token tile, output tile) order, so its
// workgroups share one or two token tiles of X in its L2 rather than all of
// them.  With a K split, virtual tile v is K range v / ntiles of output
// tile v % ntiles, so an XCD's run holds neighbouring tiles of one K range
// (which share their X slices).
struct TileOf {
    int n0, m0;       // first output and first token of the tile
    int ks;           // K range of this workgroup
    int s0, nsteps;   // its K steps: [s0, s0 + nsteps) of the K / 64
};

template <int BM, int BN>
__device__ __forceinline__ TileOf tile_of(const Prefill2Args& a) {
    const int nn = (a.N + BN - 1) / BN;
    const int ntiles = nn * ((a.M + BM - 1) / BM);
    const int T = gridDim.x, g = blockIdx.x, full = T / 8, rem = T % 8, x = g % 8;
    const int v = x * full + min(x, rem) + g / 8;
    TileOf t;
    t.ks = v / ntiles;
    const int tile = v - t.ks * ntiles;
    t.n0 = (tile % nn) * BN;
    t.m0 = (tile / nn) * BM;
    t.s0 = (int)((int64_t)t.ks * (a.K / kBK) / a.ksplit);
    t.nsteps = (int)((int64_t)(t.ks + 1) * (a.K / kBK) / a.ksplit) - t.s0;
    return t;
}

// Epilogue: D fragment (i, j) of a wave whose A sub-tiles start at output
// nb and B sub-tiles at token mb -- the lane holds outputs
// nb + 16 i + 4 fq .. + 3 for token mb + 16 j + fr.  With a K split, the
// fp32 partial products go to plane ks of `part` (row stride N), summed by
// prefill_reduce_kernel.
template <int TI, int TJ>
__device__ __forceinline__ void store_tile(const Prefill2Args& a, const f32x4_t (&acc)[TI][TJ],
                                           int nb, int mb, int fq, int fr, int ks) {
    const bool partial = a.part != nullptr;
    const int y_dtype = partial ? NB_F32 : a.y_dtype;
    void* const yb = partial ? static_cast<void*>(a.part + (int64_t)ks * a.M * a.N) : a.y;
    const int64_t ldy = partial ? a.N : a.ldy;
#pragma unroll
    for (int i = 0; i < TI; ++i) {
        const int n = nb + i * 16 + fq * 4;
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int m = mb + j * 16 + fr;
            if (m >= a.M) continue;
            const f32x4_t v = acc[i][j];
            if (y_dtype == NB_BF16) {
                bf16_bits* yp = static_cast<bf16_bits*>(yb) + (int64_t)m * ldy + n;
                // one 8-byte store where the four outputs exist and the
                // address allows it (y may be any 2-byte-aligned view)
                if (n + 3 < a.N && (reinterpret_cast<uintptr_t>(yp) & 7) == 0) {
                    u32x2_t p;
                    p.x = (uint32_t)f32_to_bf16_rne(v.x) | ((uint32_t)f32_to_bf16_rne(v.y) << 16);
                    p.y = (uint32_t)f32_to_bf16_rne(v.z) | ((uint32_t)f32_to_bf16_rne(v.w) << 16);
                    *reinterpret_cast<u32x2_t*>(yp) = p;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n + e < a.N) yp[e] = f32_to_bf16_rne(v[e]);
                }
            } else {
                float* yp = static_cast<float*>(yb) + (int64_t)m * ldy + n;
                const bool acc_y = !partial && a.accumulate;
                if (n + 3 < a.N && (reinterpret_cast<uintptr_t>(yp) & 15) == 0) {
                    *reinterpret_cast<f32x4_t*>(yp) =
                        acc_y ? *reinterpret_cast<const f32x4_t*>(yp) + v : v;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n + e < a.N) yp[e] = acc_y ? yp[e] + v[e] : v[e];
                }
            }
        }
    }
}

// One thread's share of a W slice: 12 index bytes (32 weights) per half
// row it takes (H = 1 or 2) and the codebook of the row's block.  Each
// 12-byte piece is one register tuple, so its loads land in place without
// copies.
template <int H>
struct WRegs {
    u32x4_t d[H];  // x, y, z of d[h]: the index bytes of half h
    u32x4_t c0, c1;
};

template <int BM, int BN, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void prefill2_kernel(Prefill2Args a) {
    constexpr int kThreads = 64 * WAVES;
    constexpr int WGM = WAVES >= 16 ? 4 : 2;  // waves along the tokens
    constexpr int WGN = WAVES / WGM;     // waves along the outputs
    constexpr int WN = BN / WGN;         // outputs per wave (A operand rows)
    constexpr int WM = BM / WGM;         // tokens per wave (B operand rows)
    constexpr int TI = WN / 16, TJ = WM / 16;
    constexpr int kXBytes = BM * kRowBytes, kWBytes = BN * kRowBytes;
    constexpr int kStage = kXBytes + kWBytes;
    constexpr int kXLoads = BM / (8 * WAVES);  // dma16 per wave per step (8 rows each)
    // threads per W row: 2 (half a row each) or 1; with more threads than
    // two per row, the first 2 BN threads dequantize
    constexpr int TPR = kThreads >= 2 * BN ? 2 : kThreads / BN;
    constexpr int H = 2 / TPR;           // 32-weight halves per thread
    constexpr bool kAllDeq = kThreads <= 2 * BN;
    static_assert(TPR == 1 || TPR == 2, "one or two threads per W row");
    using WR = WRegs<H>;
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const TileOf t = tile_of<BM, BN>(a);
    const int n0 = t.n0, m0 = t.m0, ks = t.ks, s0 = t.s0, nsteps = t.nsteps;
    const int bpr = a.K / 128;
    const uint32_t base = lds_addr(smem);

    // X slice: instruction i of wave w covers slice rows 8 (kXLoads w + i)
    // .. +7; lane l fills slot l & 7 of row 8 (...) + (l >> 3)
    auto load_x = [&](int step, int stage) {
#pragma unroll
        for (int i = 0; i < kXLoads; ++i) {
            const int r0 = (wave * kXLoads + i) * 8;
            const int r = r0 + (lane >> 3);
            const int c = (lane & 7) ^ (r & 7);
            const int gm = min(m0 + r, a.M - 1);
            const uint16_t* src = a.x + (int64_t)gm * a.ldx + (int64_t)(s0 + step) * kBK + c * 8;
            dma16(__builtin_amdgcn_readfirstlane(base + stage * kStage + r0 * kRowBytes), src);
        }
    };
    // W slice: thread t takes halves h0 .. h0 + H - 1 of row t / TPR
    const int wr = (tid / TPR) % BN, h0 = (tid % TPR) * H;
    const int gn = min(n0 + wr, a.N - 1);
    const bool deq = kAllDeq || tid < 2 * BN;
    auto load_w = [&](int step, WR& w) {
        if (!deq) return;
        const int64_t blk = (int64_t)gn * bpr + ((s0 + step) >> 1);
#pragma unroll
        for (int h = 0; h < H; ++h) {
            const uint32_t* ip = reinterpret_cast<const uint32_t*>(
                a.packed + blk * 48 + ((s0 + step) & 1) * 24 + (h0 + h) * 12);
            w.d[h].x = ip[0];
            w.d[h].y = ip[1];
            w.d[h].z = ip[2];
        }
        const u32x4_t* cp = reinterpret_cast<const u32x4_t*>(a.codebook + blk * 8);
        w.c0 = cp[0];
        w.c1 = cp[1];
    };
    auto store_w = [&](int stage, const WR& w) {
        if (!deq) return;
        const uint32_t q0 = pack_bf16x2(__uint_as_float(w.c0.x), __uint_as_float(w.c0.y));
        const uint32_t q1 = pack_bf16x2(__uint_as_float(w.c0.z), __uint_as_float(w.c0.w));
        const uint32_t q2 = pack_bf16x2(__uint_as_float(w.c1.x), __uint_as_float(w.c1.y));
        const uint32_t q3 = pack_bf16x2(__uint_as_float(w.c1.z), __uint_as_float(w.c1.w));
        const uint32_t lo0 = __builtin_amdgcn_perm(q1, q0, 0x06040200u);
        const uint32_t hi0 = __builtin_amdgcn_perm(q1, q0, 0x07050301u);
        const uint32_t lo1 = __builtin_amdgcn_perm(q3, q2, 0x06040200u);
        const uint32_t hi1 = __builtin_amdgcn_perm(q3, q2, 0x07050301u);
        unsigned char* wt = smem + stage * kStage + kXBytes;
#pragma unroll
        for (int h = 0; h < H; ++h) {
            // the four 24-bit groups of the half's 96 index bits
            const u32x4_t d = w.d[h];
            const uint32_t g[4] = {d.x & 0xffffffu, __builtin_amdgcn_alignbit(d.y, d.x, 24),
                                   __builtin_amdgcn_alignbit(d.z, d.y, 16), d.z >> 8};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                *reinterpret_cast<u32x4_t*>(wt + swz(wr, (h0 + h) * 4 + j)) =
                    lookup8(g[j], lo0, lo1, hi0, hi1);
            }
        }
    };

    const int wm = wave / WGN, wn = wave % WGN;
    const int fr = lane & 15, fq = lane >> 4;
    f32x4_t acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    WR wq0, wq1;  // W slices of even / odd steps (named, so they stay in registers)
    load_x(0, 0);
    load_w(0, wq0);
    if (nsteps > 1) load_w(1, wq1);
    store_w(0, wq0);
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
    __syncthreads();

    // One step on LDS stage CUR (= step & 1): the W slice of step + 2 goes
    // into the registers this step's came from (already in LDS) and the next
    // X slice is requested, the MFMAs run, then the next step's W slice
    // (loaded one step ago) is dequantized into the other stage.
    auto run_step = [&](int step, auto cur_c, WR& mine, WR& next) {
        constexpr int cur = decltype(cur_c)::value;
        // The next step's W slice was loaded a step ago and the previous
        // step ended with vmcnt(0): passing its registers through an empty
        // asm statement here puts the compiler's wait for them at this point
        // (where it costs nothing), so the dequantization below may sit
        // among the MFMAs without a wait that would also drain the X slice
        // requested next (the compiler cannot see that load).
#pragma unroll
        for (int h = 0; h < H; ++h) asm volatile("" : "+v"(next.d[h]));
        asm volatile("" : "+v"(next.c0), "+v"(next.c1));
        if (step + 2 < nsteps) load_w(step + 2, mine);
        if (step + 1 < nsteps) load_x(step + 1, cur ^ 1);
        const unsigned char* xt = smem + cur * kStage;
        const unsigned char* wt = xt + kXBytes;
        auto mfma_k32 = [&](int ks) {  // 32 of the step's 64 K
            const int c = ks * 4 + fq;
            u32x4_t av[TI], bv[TJ];
#pragma unroll
            for (int i = 0; i < TI; ++i)
                av[i] = *reinterpret_cast<const u32x4_t*>(wt + swz(wn * WN + i * 16 + fr, c));
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                bv[j] = *reinterpret_cast<const u32x4_t*>(xt + swz(wm * WM + j * 16 + fr, c));
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8_t, av[i]), __builtin_bit_cast(bf16x8_t, bv[j]),
                        acc[i][j], 0, 0, 0);
        };
        mfma_k32(0);
        if (step + 1 < nsteps) store_w(cur ^ 1, next);
        mfma_k32(1);
        // the next X slice (direct-to-LDS, not tracked by the compiler) must
        // be in LDS before the barrier; the W loads of step + 2, issued
        // before it, have had the whole step to arrive
        asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
        __syncthreads();
    };
    for (int step = 0; step < nsteps; step += 2) {
        run_step(step, std::integral_constant<int, 0>{}, wq0, wq1);
        if (step + 1 < nsteps) run_step(step + 1, std::integral_constant<int, 1>{}, wq1, wq0);
    }

    store_tile<TI, TJ>(a, acc, n0 + wn * WN, m0 + wm * WM, fq, fr, ks);
}

// y[m][n] = sum over k ranges s = 0, 1, ... of part[s][m][n] (in that
// order, so the result does not depend on which workgroup finished first),
// converted to y's dtype (added to fp32 y with accumulate).  Four
// consecutive outputs per thread where the rows allow it.
__global__ __launch_bounds__(256) void prefill_reduce_kernel(const float* __restrict__ part,
                                                             int S, int M, int N, void* y,
                                                             int y_dtype, int64_t ldy,
                                                             int accumulate) {
    const int64_t plane = (int64_t)M * N;
    // four outputs a thread where every row starts on a 4-output boundary
    // of both part and y (rows of 4k outputs, bases aligned for the vector
    // width: 16 bytes for part and fp32 y, 8 for bf16 y)
    const uintptr_t y_align = y_dtype == NB_BF16 ? 7 : 15;
    const bool vec = ((N | ldy) & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & y_align) == 0 &&
                     (reinterpret_cast<uintptr_t>(part) & 15) == 0;
    const int64_t total = vec ? plane / 4 : plane;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * 256) {
        if (vec) {
            const int64_t e = 4 * i, m = e / N, n = e - m * N;
            f32x4_t v = *reinterpret_cast<const f32x4_t*>(part + e);
            for (int k = 1; k < S; ++k) v += *reinterpret_cast<const f32x4_t*>(part + k * plane + e);
            if (y_dtype == NB_BF16) {
                u32x2_t p;
                p.x = (uint32_t)f32_to_bf16_rne(v.x) | ((uint32_t)f32_to_bf16_rne(v.y) << 16);
                p.y = (uint32_t)f32_to_bf16_rne(v.z) | ((uint32_t)f32_to_bf16_rne(v.w) << 16);
                *reinterpret_cast<u32x2_t*>(static_cast<bf16_bits*>(y) + m * ldy + n) = p;
            } else {
                f32x4_t* yp = reinterpret_cast<f32x4_t*>(static_cast<float*>(y) + m * ldy + n);
                *yp = accumulate ? *yp + v : v;
            }
        } else {
            const int64_t m = i / N, n = i - m * N;
            float v = part[i];
            for (int k = 1; k < S; ++k) v += part[k * plane + i];
            if (y_dtype == NB_BF16) {
                static_cast<bf16_bits*>(y)[m * ldy + n] = f32_to_bf16_rne(v);
            } else {
                float* yp = static_cast<float*>(y) + m * ldy + n;
                *yp = accumulate ? *yp + v : v;
            }
        }
    }
}

struct PrefillPlan {
    int BM, BN, S;
};

// The tile (BM tokens x BN outputs) and the number of K ranges per tile.
// One launch over all of K: the largest tile (fewest workgroups, least
// redundant traffic) whose grid still gives about 0.6 workgroups per CU.
// Where only the smallest tile (64 x 128) is left -- few tokens or a narrow
// layer, where every workgroup walks all of K with little work per step --
// and a split is allowed, the largest tile that reaches that grid when
// repeated over S <= 8 K ranges of at least 8 steps each, preferring fp32
// partial products (written, then read once by the reduction) of at most
// twice the packed weight's bytes, else four times.  Measured on MI355X
// over the four 2.2B layer shapes: M = 128 layer 140 -> 86 us, M = 512
// 191 -> 156-162 us (down 75 -> 44-45 us); splitting tiles that already
// fill the grid was slower.  A tile that reaches 0.6 per CU but leaves more
// than a tenth of the CUs idle gives way to 256 x 256 over S K ranges when
// K is long (below).
PrefillPlan prefill_plan(int M, int N, int K, bool allow_split) {
    const int64_t cus = device_cu_count();
    const int64_t want = cus * 3 / 5;
    const int nsteps = K / kBK;
    const int64_t wbytes = (int64_t)N * K / 128 * 80;
    auto groups = [&](int bm, int bn) {
        return (int64_t)((N + bn - 1) / bn) * ((M + bm - 1) / bm);
    };
    const int tiles[4][2] = {{256, 256}, {256, 128}, {128, 128}, {64, 128}};
    for (int t = 0; t < 3; ++t) {
        const int64_t g = groups(tiles[t][0], tiles[t][1]);
        if (g < want) continue;
        // A long K on a grid that still leaves a tenth of the CUs idle: the
        // 256 x 256 tile over S K ranges of at least 32 steps, where that
        // gives more workgroups (down at M = 2048: 160 tiles of 256 x 128
        // 126-135 us, 3 x 80 of 256 x 256 92-98 us; o, whose K ranges would
        // be 13 steps, stays at 51-54 us unsplit).
        if (allow_split && M >= 256 && g * 10 < cus * 9) {
            const int64_t g2 = groups(256, 256);
            const int S = (int)std::min<int64_t>(cus / g2, nsteps / 32);
            if (S >= 2 && g2 * S > g) return {256, 256, S};
        }
        return {tiles[t][0], tiles[t][1], 1};
    }
    if (allow_split) {
        for (int64_t mult = 2; mult <= 4; mult += 2) {
            for (int t = 0; t < 4; ++t) {
                const int bm = tiles[t][0], bn = tiles[t][1];
                if (bm > std::max(64, M)) continue;   // mostly empty token rows
                const int64_t g = groups(bm, bn);
                int S = (int)std::min<int64_t>({cus / g, 8, nsteps / 8});
                while (S > 1 && (int64_t)S * M * N * 4 > mult * wbytes) --S;
                if (S > 1 && g * S >= want) return {bm, bn, S};
            }
        }
    }
    return {64, 128, 1};
}

// x (M rows, stride ldx, fp32) -> hi = bf16(x), lo = bf16(x - hi), rows of
// K (contiguous).  x - hi is exact in fp32, so hi + lo is x to 2^-18.
__global__ __launch_bounds__(256) void split_bf16_kernel(const float* __restrict__ x, int64_t ldx,
                                                         bf16_bits* __restrict__ hi,
                                                         bf16_bits* __restrict__ lo, int M, int K) {
    const int64_t total = (int64_t)M * K;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * 256) {
        const int64_t m = i / K, k = i - m * K;
        const float v = x[m * ldx + k];
        const bf16_bits h = f32_to_bf16_rne(v);
        hi[i] = h;
        lo[i] = f32_to_bf16_rne(v - bf16_to_f32(h));
    }
}

// The residual codebook: cb_lo = cb - bf16(cb) (exact in fp32).
__global__ __launch_bounds__(256) void cb_residual_kernel(const float* __restrict__ cb,
                                                          float* __restrict__ cb_lo, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * 256) {
        const float v = cb[i];
        cb_lo[i] = v - bf16_to_f32(f32_to_bf16_rne(v));
    }
}

inline int64_t align256(int64_t v) { return (v + 255) & ~(int64_t)255; }

}  // namespace

int64_t prefill_f32_bytes(int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0 || K % 128) return 0;
    const int64_t xb = align256((int64_t)M * K * 2);
    const int64_t cb = align256((int64_t)N * (K / 128) * 8 * 4);
    return 2 * xb + cb + prefill_split_bytes(M, N, K);
}

int launch_prefill_f32(const float* x, int64_t ldx, const uint8_t* packed, const float* codebook,
                       float* y, int64_t ldy, int M, int N, int K, void* workspace,
                       int64_t ws_bytes, hipStream_t stream) {
    unsigned char* w = static_cast<unsigned char*>(workspace);
    const int64_t xb = align256((int64_t)M * K * 2);
    const int64_t nent = (int64_t)N * (K / 128) * 8;
    bf16_bits* hi = reinterpret_cast<bf16_bits*>(w);
    bf16_bits* lo = reinterpret_cast<bf16_bits*>(w + xb);
    float* cb_lo = reinterpret_cast<float*>(w + 2 * xb);
    unsigned char* split = w + 2 * xb + align256(nent * 4);
    const int64_t split_bytes = ws_bytes - (split - w);
    const unsigned g1 = (unsigned)std::min<int64_t>(((int64_t)M * K + 255) / 256, 8192);
    hipLaunchKernelGGL(split_bf16_kernel, dim3(g1), dim3(256), 0, stream, x, ldx, hi, lo, M, K);
    const unsigned g2 = (unsigned)std::min<int64_t>((nent + 255) / 256, 4096);
    hipLaunchKernelGGL(cb_residual_kernel, dim3(g2), dim3(256), 0, stream, codebook, cb_lo, nent);
    int st = check_launch("nb_gemm_prefill_f32");
    if (st) return st;
    void* sw = split_bytes > 0 ? static_cast<void*>(split) : nullptr;
    // x.W ~= hi.bf16(cb) + hi.bf16(cb_lo) + lo.bf16(cb), each pass in fp32,
    // added to y in that order
    st = launch_prefill2(hi, K, packed, codebook, y, NB_F32, ldy, M, N, K, sw, split_bytes, stream,
                         false);
    if (st) return st;
    st = launch_prefill2(hi, K, packed, cb_lo, y, NB_F32, ldy, M, N, K, sw, split_bytes, stream,
                         true);
    if (st) return st;
    return launch_prefill2(lo, K, packed, codebook, y, NB_F32, ldy, M, N, K, sw, split_bytes,
                           stream, true);
}

int64_t prefill_split_bytes(int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0 || K % 128) return 0;
    const PrefillPlan p = prefill_plan(M, N, K, true);
    return p.S > 1 ? (int64_t)p.S * M * N * 4 : 0;
}

int launch_prefill2(const void* x, int64_t ldx, const uint8_t* packed, const float* codebook,
                    void* y, int y_dtype, int64_t ldy, int M, int N, int K, void* workspace,
                    int64_t ws_bytes, hipStream_t stream, bool accumulate) {
    Prefill2Args a;
    a.accumulate = accumulate ? 1 : 0;
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
    PrefillPlan p = prefill_plan(M, N, K, workspace != nullptr);
    if (p.S > 1 && ws_bytes < (int64_t)p.S * M * N * 4) p = prefill_plan(M, N, K, false);
    a.ksplit = p.S;
    a.part = p.S > 1 ? static_cast<float*>(workspace) : nullptr;
    constexpr int W = NB_PREFILL_WAVES;
    const unsigned grid = (unsigned)(((N + p.BN - 1) / p.BN) * ((M + p.BM - 1) / p.BM) * p.S);
#define NB_PREFILL2_LAUNCH(BMv, BNv)                                                          \
    hipLaunchKernelGGL((prefill2_kernel<BMv, BNv, W>), dim3(grid), dim3(64 * W),             \
                       (size_t)2 * (BMv + BNv) * kRowBytes, stream, a)
    if (p.BM == 256 && p.BN == 256) {
        NB_PREFILL2_LAUNCH(256, 256);
    } else if (p.BM == 256) {
        NB_PREFILL2_LAUNCH(256, 128);
    } else if (p.BM == 128) {
        NB_PREFILL2_LAUNCH(128, 128);
    } else {
        NB_PREFILL2_LAUNCH(64, 128);
    }
#undef NB_PREFILL2_LAUNCH
    if (p.S > 1) {
        const int st = check_launch("nb_gemm_prefill");
        if (st) return st;
        const int64_t items = ((N | ldy) & 3) == 0 ? (int64_t)M * N / 4 : (int64_t)M * N;
        const unsigned rg = (unsigned)std::min<int64_t>((items + 255) / 256, 4096);
        hipLaunchKernelGGL(prefill_reduce_kernel, dim3(rg), dim3(256), 0, stream, a.part, p.S,
                           M, N, y, y_dtype, ldy, a.accumulate);
    }
    return check_launch("nb_gemm_prefill");
}

}  // namespace nb
