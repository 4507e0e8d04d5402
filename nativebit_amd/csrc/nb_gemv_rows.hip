// Single-problem streaming GEMV for the launches of a decode step (gfx950).
//
//   r[n] = sum_k a[k] * bf16(W[n][k])        (M = 1, 3-bit, 8 entries, BS 128)
//
// with a = x (bf16), RMSNorm(x) or silu(gate) * up (fp32 inputs, rounded to
// bf16 once), as the batched kernel's x_mode forms, and y = r, y += r, or --
// for a gate|up layer whose rows alternate gate, up -- y[i] =
// bf16(silu(r[2i]) * r[2i+1]), the SwiGLU product the down projection reads
// (NB_Y_SILU_PAIRS).  A decode step's GEMVs are 2-18 MB each, so a launch
// lasts a few microseconds and its cost is latency, not bandwidth.  This
// kernel is shaped for that:
//
// * Chunks are whole rows: R = floor(64 / bpr) rows (R * bpr <= 64 blocks,
//   one block per lane), so a lane's column block is the same in every
//   chunk and its 16 units of staged activations stay in registers for the
//   whole launch; every CU gets a share of even the smallest layer (a 2560 x
//   2560 o projection is 853 chunks).
// * One workgroup per CU, 12 waves; a workgroup owns a contiguous run of
//   chunks (whole gate|up pairs), dealt to its waves one by one, and each
//   wave requests up to SLOTS of its chunks (direct-to-LDS, five 1 KiB loads
//   each) at once.
// * The activation inputs also arrive by direct-to-LDS loads, issued before
//   the weight loads: vmcnt counts in issue order, so the wait for them
//   leaves the weight loads in flight, and no compiler-tracked load sits
//   among the ring loads (the compiler cannot see the ring loads and would
//   otherwise wait for all of them).  The norm's sum of squares, the bf16
//   rounding and the staging into the selector layout overlap the weights'
//   arrival.
// * A chunk's work is its 64 block dot products, one LDS store each; the
//   row sums (in block order, deterministic, independent of the grid) and
//   the y epilogue run once per workgroup after its last chunk.
//
// Weights are the codebook entries rounded to bf16 (RNE), as the reference's
// bf16 path (inference/eval_ppl.py:149-174); accumulation is fp32.
#include <algorithm>

#include "nb_device.h"
#include "nb_internal.h"
#include "nb_stream_common.h"

namespace nb {
namespace {

using namespace stream;

constexpr int kWaves = 12;                        // 3 per SIMD (8: 0.7 % fewer tokens/s)
constexpr int kThreads = 64 * kWaves;
constexpr int kSlotIdx = 64 * 48;                 // 3 KiB of index stream
constexpr int kSlotBytes = kSlotIdx + 64 * 32;    // + 2 KiB of codebook
constexpr int kLoads = 5;                         // dma16 per chunk
constexpr int kMaxK = 8192;

struct RowsArgs {
    const uint8_t* packed;
    const float* codebook;
    const void* x;
    const float* norm_w;
    void* y;
    int N, K, bpr, R, nchunks;
    int unit;           // chunks per scheduling unit (2 keeps gate|up pairs in one workgroup)
    int wg_chunks;      // LDS dot-product rows (64 floats) per workgroup: its largest share
    int raw_bytes;      // LDS bytes of the raw activation inputs (multiple of 1 KiB)
    int y_mode, y_dtype;
    float eps;
};

__device__ __forceinline__ float wsum(float v) { return wave64_sum(v); }

// Halfword position of element e (0..7) of 8-element group g (0..15) of a
// column block in the staged layout of nb_stream_common.h (stage_unit).
__device__ __forceinline__ int staged_half(int g, int e) {
    const int s = e == 0 ? 0 : e == 1 ? 1 : e == 2 ? 6 : e == 3 ? 2 : e == 4 ? 3 : e == 5 ? 7
                : e == 6 ? 4 : 5;
    return (4 * (g >> 2) + (s >> 1)) * 8 + (s & 1) * 4 + (g & 3);
}

// Waits until at most n loads are outstanding (n a multiple of kLoads, at
// most N), with n as the instruction's immediate.
template <int N>
__device__ __forceinline__ void wait_vm_n(int n) {
    if constexpr (N > 0) {
        if (n >= N) {
            wait_vm<N>();
            return;
        }
        wait_vm_n<N - kLoads>(n);
    } else {
        wait_vm<0>();
    }
}

// One 1 KiB piece of a contiguous byte range [base, base + nbytes) to LDS:
// lane i copies bytes 16 i .. 16 i + 15 of piece p (past the end it re-reads
// the range's last 16 bytes; those LDS bytes are never used).
__device__ __forceinline__ void dma_piece(uint32_t lds, const uint8_t* base, int nbytes, int p,
                                          int lane) {
    const uint8_t* last = base + nbytes - 16;
    const uint8_t* src = base + p * 1024 + 16 * lane;
    dma16<0>(__builtin_amdgcn_readfirstlane(lds + p * 1024), src < last ? src : last);
}

// kSel: the index stream is in the selector-ordered unit layout
// (nb_stream_layout); the products are the same.
template <int XMODE, int SLOTS, bool kSel>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3, 3)))
void gemv_rows_kernel(RowsArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int K = a.K, bpr = a.bpr, R = a.R;
    unsigned char* xs = smem;                                   // staged bf16 activations
    unsigned char* raw = xs + bpr * kXColBytes;                 // raw activation inputs
    unsigned char* ring = raw + a.raw_bytes;                    // kWaves x SLOTS slots
    float* dots = reinterpret_cast<float*>(ring + kWaves * SLOTS * kSlotBytes);  // 64 per chunk
    float* red = dots + a.wg_chunks * 64;                       // kWaves floats

    // ---- 1. the activation inputs, this wave's share of 1 KiB pieces ------
    const uint32_t raw_lds = lds_addr(raw);
    if constexpr (XMODE == NB_X_BF16) {
        const int nb = 2 * K;
        for (int p = wave; p * 1024 < nb; p += kWaves)
            dma_piece(raw_lds, static_cast<const uint8_t*>(a.x), nb, p, lane);
    } else {
        // x (fp32) at raw[0, 4K); the norm weights, or up (the second half
        // of gate | up), at raw[sofs, sofs + 4K), sofs = 4K rounded up to
        // whole pieces so that x's last piece cannot overwrite them
        const int nb = 4 * K;
        const uint8_t* xb = static_cast<const uint8_t*>(a.x);
        const uint8_t* sb = XMODE == NB_X_RMSNORM ? reinterpret_cast<const uint8_t*>(a.norm_w)
                                                  : xb + nb;
        for (int p = wave; p * 1024 < nb; p += kWaves) {
            dma_piece(raw_lds, xb, nb, p, lane);
            dma_piece(raw_lds + a.raw_bytes / 2, sb, nb, p, lane);
        }
    }

    // ---- 2. the workgroup's chunks and this wave's first loads --------------
    // The workgroup owns chunks [c0, c1) (whole units); wave w takes chunks
    // c0 + w, c0 + w + kWaves, ...
    const int nunits = (a.nchunks + a.unit - 1) / a.unit;
    const int u0 = (int)((int64_t)blockIdx.x * nunits / gridDim.x);
    const int u1 = (int)((int64_t)(blockIdx.x + 1) * nunits / gridDim.x);
    const int c0 = u0 * a.unit, c1 = min(a.nchunks, u1 * a.unit);
    const int n = c1 - c0 > wave ? (c1 - c0 - wave + kWaves - 1) / kWaves : 0;
    unsigned char* my_ring = ring + wave * SLOTS * kSlotBytes;
    const uint32_t ring_lds = lds_addr(my_ring);
    const int64_t total_blocks = (int64_t)a.N * bpr;
    const uint8_t* ilast = a.packed + total_blocks * 48 - 16;
    const uint8_t* clast = reinterpret_cast<const uint8_t*>(a.codebook) + total_blocks * 32 - 16;
    auto issue = [&](int c, int slot) {
        const int64_t b0 = (int64_t)c * R * bpr;
        const uint8_t* ip = a.packed + b0 * 48 + 16 * lane;
        const uint8_t* cp = reinterpret_cast<const uint8_t*>(a.codebook) + b0 * 32 + 16 * lane;
        const uint32_t dst = __builtin_amdgcn_readfirstlane(ring_lds + slot * kSlotBytes);
        dma16<0>(dst, min(ip, ilast));
        dma16<0>(dst + 1024, min(ip + 1024, ilast));
        dma16<0>(dst + 2048, min(ip + 2048, ilast));
        dma16<0>(dst + kSlotIdx, min(cp, clast));
        dma16<0>(dst + kSlotIdx + 1024, min(cp + 1024, clast));
    };
    // One chunk's loads go out behind the activation pieces, the other slots'
    // once the activations are staged: the pieces (which every workgroup
    // needs before it can compute) then do not queue behind the whole weight
    // burst, and no load issue stalls a wave between the barriers below.
    const int first = min(n, SLOTS);
    const int early = min(first, 1);
    for (int i = 0; i < early; ++i) issue(c0 + wave + i * kWaves, i);

    // ---- 3. activations: wait for their pieces (the weights stay in flight),
    //         form them in fp32, round to bf16, stage in the selector layout
    wait_vm_n<SLOTS * kLoads>(early * kLoads);
    typedef __attribute__((ext_vector_type(4))) float f4;
    if constexpr (XMODE == NB_X_RMSNORM) {
        // the norm's sum of squares over this wave's own pieces of x (in LDS
        // now), so that one barrier publishes both the pieces and the sums
        const f4* xr4 = reinterpret_cast<const f4*>(raw);
        float ssw = 0.f;
        for (int p = wave; p * 1024 < 4 * K; p += kWaves) {
            const int e0 = p * 256 + 4 * lane;   // K % 4 == 0: a lane's 4 are all in or out
            const f4 v = xr4[e0 >> 2];
            if (e0 < K) ssw += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
        ssw = wsum(ssw);
        if (lane == 0) red[wave] = ssw;
    }
    __syncthreads();  // every wave's pieces (and partial sums) are in LDS
    uint16_t* xh = reinterpret_cast<uint16_t*>(xs);
    if constexpr (XMODE == NB_X_BF16) {
        // one thread per 32-element unit: its 64 bytes in four 16-byte
        // reads, the staged unit's four 16-byte pieces in four writes (one
        // LDS round trip; element by element, each write would wait for its
        // read)
        for (int u = tid; u < (K >> 5); u += kThreads) {
            const u32x4_t* src = reinterpret_cast<const u32x4_t*>(raw + 64 * u);
            const u32x4_t r0 = src[0], r1 = src[1], r2 = src[2], r3 = src[3];
            const uint32_t w[16] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w,
                                    r2.x, r2.y, r2.z, r2.w, r3.x, r3.y, r3.z, r3.w};
            stage_unit(xs + (u >> 2) * kXColBytes, u & 3, w);
        }
    } else {
        // quarter groups of 4 inputs per thread (each thread's divisions
        // are its critical path), read into registers before any is used
        const int nq = K >> 2;
        constexpr int kMaxQ = (kMaxK / 4 + kThreads - 1) / kThreads;
        const f4* xf4 = reinterpret_cast<const f4*>(raw);
        const f4* sf4 = reinterpret_cast<const f4*>(raw + a.raw_bytes / 2);
        f4 xr[kMaxQ], sr[kMaxQ];
#pragma unroll
        for (int j = 0; j < kMaxQ; ++j) {
            const int q = tid + j * kThreads;
            const int qq = q < nq ? q : 0;
            xr[j] = xf4[qq];
            sr[j] = sf4[qq];
        }
        float norm = 1.f;
        if constexpr (XMODE == NB_X_RMSNORM) {
            // the waves' partial sums, added in wave order in every thread
            const f4 r0 = reinterpret_cast<const f4*>(red)[0];
            const f4 r1 = reinterpret_cast<const f4*>(red)[1];
            const f4 r2 = reinterpret_cast<const f4*>(red)[2];
            static_assert(kWaves == 12, "three vectors of partial sums");
            const float rw[12] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y,
                                  r1.z, r1.w, r2.x, r2.y, r2.z, r2.w};
            float t = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) t += rw[w];
            norm = sqrtf(t / (float)K + a.eps);
        }
        // x / norm for a divisor shared by every element: rn = RN(1 / norm)
        // by one IEEE division, then q0 = RN(x rn), the exact remainder
        // x - q0 norm (one fma) and q0 + remainder * rn (one fma), which is
        // RN(x / norm) (Markstein's correction; values here are far from
        // overflow and underflow)
        const float rn = 1.0f / norm;
#pragma unroll
        for (int j = 0; j < kMaxQ; ++j) {
            const int q = tid + j * kThreads;
            if (q < nq) {
                const int g = q >> 1, e0 = 4 * (q & 1);
                uint16_t* col = xh + (g >> 4) * (kXColBytes / 2);
                const float xv[4] = {xr[j].x, xr[j].y, xr[j].z, xr[j].w};
                const float sv[4] = {sr[j].x, sr[j].y, sr[j].z, sr[j].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    // RMSNorm.forward's (x / norm) * w, generate_torch.py:37; silu(g) * u,
                    // 116-117 (exp(-g) by v_exp_f32, a few ulp, below the bf16 rounding)
                    float r;
                    if constexpr (XMODE == NB_X_RMSNORM) {
                        const float q0 = xv[e] * rn;
                        r = fmaf(fmaf(-q0, norm, xv[e]), rn, q0) * sv[e];
                    } else {
                        r = (xv[e] / (1.0f + __expf(-xv[e]))) * sv[e];
                    }
                    col[staged_half(g & 15, e0 + e)] = f32_to_bf16_rne(r);
                }
            }
        }
    }
    __syncthreads();
    // the wave's other first chunks go out now: issued before the staging,
    // their loads stall behind the memory system's queue and hold up the
    // barriers above
    for (int i = early; i < first; ++i) issue(c0 + wave + i * kWaves, i);

    // ---- 4. the wave's chunks: wait, read the slot, refill it, compute ------
    // Lane l takes column block l % bpr of row l / bpr of every chunk (lanes
    // past R * bpr compute a block nobody reads), so its activation units
    // are loaded once, with the first chunk.
    u32x4_t xv[16];
    const unsigned char* xb = xs + (lane % bpr) * kXColBytes;
    for (int i = 0; i < n; ++i) {
        const int slot = i % SLOTS;
        const int issued = min(n, i + SLOTS);
        wait_vm_n<(SLOTS - 1) * kLoads>((issued - i - 1) * kLoads);
        const unsigned char* src = my_ring + slot * kSlotBytes;
        const u32x4_t* pi = reinterpret_cast<const u32x4_t*>(src + 48 * lane);
        const u32x4_t* pc = reinterpret_cast<const u32x4_t*>(src + kSlotIdx + 32 * lane);
        const u32x4_t d0 = pi[0], d1 = pi[1], d2 = pi[2], e0 = pc[0], e1 = pc[1];
        if (i == 0) {
            // The activation units go out behind the slot's five reads (the
            // empty asm keeps the compiler from reordering them). LDS
            // operations complete in order, so waiting until at most 15 of
            // the 16 unit reads are outstanding (15: the counter's largest
            // value) means the slot has been read and may be refilled, while
            // the dequantization below overlaps the unit reads (the compiler
            // waits for those before the MFMAs). This holds while no scalar
            // memory load is in flight between the slot reads and the wait
            // (those return out of order on the same counter): the code
            // between them issues none.
            asm volatile("" : : : "memory");
#pragma unroll
            for (int j = 0; j < 16; ++j) xv[j] = *reinterpret_cast<const u32x4_t*>(xb + 16 * j);
            asm volatile("s_waitcnt lgkmcnt(15)" : : : "memory");
        } else {
            wait_lds();
        }
        if (i + SLOTS < n) issue(c0 + wave + (i + SLOTS) * kWaves, slot);
        const f32x4_t acc = block_dot<kSel>(d0, d1, d2, e0, e1, xv);
        dots[(wave + i * kWaves) * 64 + lane] = diag_of(acc, lane);
    }
    __syncthreads();

    // ---- 5. row sums and y, once per workgroup ------------------------------
    // Row r0 + j is row j % R of local chunk j / R; its bpr dot products are
    // added in block order into 16 partial sums, then a fixed tree.
    const int r0 = c0 * R;
    const int nrows = min(a.N, c1 * R) - r0;
    auto row_sum = [&](int j) -> float {
        const float* p = dots + (j / R) * 64 + (j % R) * bpr;
        float acc[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[q] = 0.f;
        for (int j0 = 0; j0 < bpr; j0 += 16) {
            float v[16];
#pragma unroll
            for (int q = 0; q < 16; ++q) v[q] = p[min(j0 + q, bpr - 1)];
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[q] += j0 + q < bpr ? v[q] : 0.f;
        }
#pragma unroll
        for (int h = 8; h > 0; h >>= 1) {
#pragma unroll
            for (int q = 0; q < h; ++q) acc[q] += acc[q + h];
        }
        return acc[0];
    };
    if (a.y_mode == NB_Y_SILU_PAIRS) {
        // rows 2i, 2i+1 are gate row i and up row i (r0 and nrows are even)
        bf16_bits* act = static_cast<bf16_bits*>(a.y) + r0 / 2;
        for (int q = tid; q < nrows / 2; q += kThreads) {
            const float g = row_sum(2 * q), u = row_sum(2 * q + 1);
            act[q] = f32_to_bf16_rne((g / (1.0f + __expf(-g))) * u);
        }
    } else {
        for (int j = tid; j < nrows; j += kThreads) {
            const float v = row_sum(j);
            const int row = r0 + j;
            if (a.y_dtype == NB_BF16) {
                *as_global_mut(static_cast<bf16_bits*>(a.y) + row) = f32_to_bf16_rne(v);
            } else if (a.y_mode == NB_Y_ADD) {
                float* yp = static_cast<float*>(a.y) + row;
                *as_global_mut(yp) = *as_global(yp) + v;   // the row is this workgroup's alone
            } else {
                *as_global_mut(static_cast<float*>(a.y) + row) = v;
            }
        }
    }
}

struct RowsShape {
    int R, nchunks, unit, G, wg_chunks, raw_bytes, slots;
    size_t lds;
};

RowsShape rows_shape(const StreamProblem& p) {
    RowsShape s;
    const int bpr = p.K / 128;
    s.R = 64 / bpr;
    s.nchunks = (p.N + s.R - 1) / s.R;
    // gate|up pairs must not be split between workgroups: with R odd, two
    // chunks (an even number of rows) are the unit of the split
    s.unit = (p.y_mode == NB_Y_SILU_PAIRS && (s.R & 1)) ? 2 : 1;
    const int nunits = (s.nchunks + s.unit - 1) / s.unit;
    s.G = std::max(1, std::min(device_cu_count(), nunits));
    s.wg_chunks = (nunits + s.G - 1) / s.G * s.unit;   // the largest workgroup share
    // bf16 x; or fp32 x and a second fp32 input, each from a whole piece
    s.raw_bytes = p.x_mode == NB_X_BF16 ? (2 * p.K + 1023) / 1024 * 1024
                                        : 2 * ((4 * p.K + 1023) / 1024 * 1024);
    const size_t fixed = (size_t)bpr * kXColBytes + s.raw_bytes + (size_t)s.wg_chunks * 64 * 4 +
                         (size_t)kWaves * 4;
    s.slots = fixed + (size_t)kWaves * 3 * kSlotBytes <= (size_t)device_lds_bytes() ? 3 : 2;
    s.lds = fixed + (size_t)kWaves * s.slots * kSlotBytes;
    return s;
}

template <int XMODE, bool kSel>
void launch_mode(const RowsShape& s, const RowsArgs& a, hipStream_t stream) {
    if (s.slots == 3) {
        hipLaunchKernelGGL((gemv_rows_kernel<XMODE, 3, kSel>), dim3(s.G), dim3(kThreads), s.lds,
                           stream, a);
    } else {
        hipLaunchKernelGGL((gemv_rows_kernel<XMODE, 2, kSel>), dim3(s.G), dim3(kThreads), s.lds,
                           stream, a);
    }
}

template <bool kSel>
void launch_modes(int x_mode, const RowsShape& s, const RowsArgs& a, hipStream_t stream) {
    switch (x_mode) {
        case NB_X_BF16: launch_mode<NB_X_BF16, kSel>(s, a, stream); break;
        case NB_X_RMSNORM: launch_mode<NB_X_RMSNORM, kSel>(s, a, stream); break;
        default: launch_mode<NB_X_SILU_MUL, kSel>(s, a, stream); break;
    }
}

}  // namespace

bool gemv_rows_fits(const StreamProblem& p) {
    if (p.K % 128 || p.K < 128 || p.K > kMaxK || p.N < 1) return false;
    return rows_shape(p).lds <= (size_t)device_lds_bytes();
}

int launch_gemv_rows(const StreamProblem& p, int y_dtype, bool sel, hipStream_t stream) {
    const RowsShape s = rows_shape(p);
    RowsArgs a;
    a.packed = p.packed;
    a.codebook = p.codebook;
    a.x = p.x;
    a.norm_w = p.norm_w;
    a.y = p.y;
    a.N = p.N;
    a.K = p.K;
    a.bpr = p.K / 128;
    a.R = s.R;
    a.nchunks = s.nchunks;
    a.unit = s.unit;
    a.wg_chunks = s.wg_chunks;
    a.raw_bytes = s.raw_bytes;
    a.y_mode = p.y_mode;
    a.y_dtype = y_dtype;
    a.eps = p.eps;
    if (sel) {
        launch_modes<true>(p.x_mode, s, a, stream);
    } else {
        launch_modes<false>(p.x_mode, s, a, stream);
    }
    return check_launch("nb_gemv_batched");
}

}  // namespace nb
