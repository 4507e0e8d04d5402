// extern "C" boundary of libnativebit_amd.so: argument validation, error
// reporting and dispatch to the gfx950 kernels.  Every check here runs on
// the host before any launch, so the whole validation surface can be tested
// without a GPU.  Unlike the reference operator, which checks nothing and
// hides every failure behind a bare `except Exception` fallback
// (inference/triton_kernel.py:244-257), each failure returns a distinct
// status with a message and nothing is launched.
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <cmath>
#include <mutex>
#include <vector>

#include "nb_internal.h"

namespace nb {
namespace {

thread_local char g_last_error[512] = "";

constexpr int kMaxDevices = 64;
int g_cu_count[kMaxDevices];
int g_lds_bytes[kMaxDevices];
int g_device_ok[kMaxDevices];  // 0 unknown, 1 gfx950, -1 unusable
std::mutex g_dev_mutex;

bool aligned(const void* p, size_t a) {
    return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

size_t dtype_size(int dt) {
    switch (dt) {
        case NB_F32: return 4;
        case NB_BF16: return 2;
        case NB_U8: return 1;
    }
    return 0;
}

// Confirms the current device is a gfx950 and caches its CU count.
int ensure_device() {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        return fail(NB_ENODEV, "hipGetDevice failed: %s", hipGetErrorString(e));
    }
    if (dev < 0 || dev >= kMaxDevices) return fail(NB_ENODEV, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_dev_mutex);
    if (g_device_ok[dev] == 0) {
        hipDeviceProp_t prop;
        e = hipGetDeviceProperties(&prop, dev);
        if (e != hipSuccess) {
            return fail(NB_ENODEV, "hipGetDeviceProperties failed: %s", hipGetErrorString(e));
        }
        if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
            g_device_ok[dev] = -1;
        } else {
            g_device_ok[dev] = 1;
            g_cu_count[dev] = prop.multiProcessorCount;
            g_lds_bytes[dev] = (int)prop.sharedMemPerBlock;
        }
    }
    if (g_device_ok[dev] != 1) {
        return fail(NB_ENODEV, "device %d is not a gfx950 (MI355X); this library "
                               "carries gfx950 code only", dev);
    }
    return NB_OK;
}

int check_format(int bits, int n_entries, int block_size, const char* fn) {
    if (bits < 1 || bits > 8) return fail(NB_EUNSUPPORTED, "%s: bits=%d outside 1..8", fn, bits);
    if (n_entries < 1 || n_entries > (1 << bits)) {
        return fail(NB_EINVAL, "%s: n_entries=%d does not fit in %d bits", fn, n_entries, bits);
    }
    if (block_size < 1) return fail(NB_EINVAL, "%s: block_size=%d < 1", fn, block_size);
    return NB_OK;
}

}  // namespace

int fail(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return status;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(NB_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
    return NB_OK;
}

int device_cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    std::lock_guard<std::mutex> lock(g_dev_mutex);
    return g_cu_count[dev] > 0 ? g_cu_count[dev] : 256;
}

int device_lds_bytes() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 64 * 1024;
    std::lock_guard<std::mutex> lock(g_dev_mutex);
    return g_lds_bytes[dev] > 0 ? g_lds_bytes[dev] : 64 * 1024;
}

}  // namespace nb

using namespace nb;

extern "C" {

int nb_abi_version(void) { return NB_ABI_VERSION; }

const char* nb_last_error(void) { return g_last_error; }

int64_t nb_packed_nbytes(int64_t count, int bits) { return packed_nbytes(count, bits); }

int nb_gemv(const void* x, int x_dtype, int64_t ldx, const uint8_t* packed,
            const float* codebook, void* y, int y_dtype, int64_t ldy, int M,
            int N, int K, int bits, int n_entries, int block_size, void* stream) {
    const char* fn = "nb_gemv";
    if (M < 1 || M > 16) return fail(NB_EUNSUPPORTED, "%s: M=%d outside 1..16", fn, M);
    if (N < 0 || K < 0) return fail(NB_EINVAL, "%s: negative shape N=%d K=%d", fn, N, K);
    int st = check_format(bits, n_entries, block_size, fn);
    if (st) return st;
    if (x_dtype != NB_F32 && x_dtype != NB_BF16) return fail(NB_EINVAL, "%s: x_dtype=%d is not F32/BF16", fn, x_dtype);
    if (y_dtype != NB_F32 && y_dtype != NB_BF16) return fail(NB_EINVAL, "%s: y_dtype=%d is not F32/BF16", fn, y_dtype);
    if (M > 1 && ldx < K) return fail(NB_EINVAL, "%s: ldx=%lld < K=%d", fn, (long long)ldx, K);
    if (M > 1 && ldy < N) return fail(NB_EINVAL, "%s: ldy=%lld < N=%d", fn, (long long)ldy, N);
    if (N == 0) return NB_OK;
    if (!y) return fail(NB_EINVAL, "%s: y is NULL", fn);
    if (K > 0 && (!x || !packed || !codebook)) return fail(NB_EINVAL, "%s: NULL input pointer", fn);
    if (!aligned(y, dtype_size(y_dtype))) return fail(NB_EALIGN, "%s: y not aligned to its dtype", fn);
    if (K > 0 && !aligned(x, dtype_size(x_dtype))) return fail(NB_EALIGN, "%s: x not aligned to its dtype", fn);
    if (K > 0 && !aligned(codebook, 4)) return fail(NB_EALIGN, "%s: codebook not 4-byte aligned", fn);
    st = ensure_device();
    if (st) return st;
    GemvArgs a;
    a.x = x;
    a.x_dtype = x_dtype;
    a.ldx = M > 1 ? ldx : K;
    a.packed = packed;
    a.packed_bytes = packed_nbytes((int64_t)N * K, bits);
    a.codebook = codebook;
    a.y = y;
    a.y_dtype = y_dtype;
    a.ldy = M > 1 ? ldy : N;
    a.M = M;
    a.N = N;
    a.K = K;
    a.bits = bits;
    a.n_entries = n_entries;
    a.block_size = block_size;
    return launch_gemv(a, static_cast<hipStream_t>(stream));
}

int nb_unpack(const uint8_t* packed, uint8_t* idx_out, int64_t count, int bits, void* stream) {
    const char* fn = "nb_unpack";
    if (bits < 1 || bits > 8) return fail(NB_EUNSUPPORTED, "%s: bits=%d outside 1..8", fn, bits);
    if (count < 0) return fail(NB_EINVAL, "%s: count=%lld < 0", fn, (long long)count);
    if (count == 0) return NB_OK;
    if (!packed || !idx_out) return fail(NB_EINVAL, "%s: NULL pointer", fn);
    int st = ensure_device();
    if (st) return st;
    return launch_unpack(packed, idx_out, count, bits, static_cast<hipStream_t>(stream));
}

int nb_pack(const uint8_t* idx, uint8_t* packed_out, int64_t count, int bits, void* stream) {
    const char* fn = "nb_pack";
    if (bits < 1 || bits > 8) return fail(NB_EUNSUPPORTED, "%s: bits=%d outside 1..8", fn, bits);
    if (count < 0) return fail(NB_EINVAL, "%s: count=%lld < 0", fn, (long long)count);
    if (count == 0) return NB_OK;
    if (!idx || !packed_out) return fail(NB_EINVAL, "%s: NULL pointer", fn);
    int st = ensure_device();
    if (st) return st;
    return launch_pack(idx, packed_out, count, bits, static_cast<hipStream_t>(stream));
}

// torch.linspace(0, 1, n) in fp32 as torch's kernel forms it: step =
// 1 / (n - 1); the first half counts up from 0, the second half down from
// 1, each value one fused multiply-add (single rounding).
static void linspace01(int n, float* q) {
    if (n == 1) {
        q[0] = 0.f;
        return;
    }
    const float step = 1.0f / (float)(n - 1);
    const int halfway = n / 2;
    for (int i = 0; i < n; ++i) {
        q[i] = i < halfway ? std::fma(step, (float)i, 0.0f)
                           : std::fma(-step, (float)(n - i - 1), 1.0f);
    }
}

int nb_block_codebooks(const float* w, int64_t total, int block_size, int n_entries,
                       float* codebook_out, void* stream) {
    const char* fn = "nb_block_codebooks";
    if (block_size < 1 || block_size > 1024) {
        return fail(NB_EUNSUPPORTED, "%s: block_size=%d outside 1..1024", fn, block_size);
    }
    if (n_entries < 1 || n_entries > 256) {
        return fail(NB_EUNSUPPORTED, "%s: n_entries=%d outside 1..256", fn, n_entries);
    }
    if (total < 0) return fail(NB_EINVAL, "%s: total=%lld < 0", fn, (long long)total);
    if (total == 0) return NB_OK;
    if (!w || !codebook_out) return fail(NB_EINVAL, "%s: NULL pointer", fn);
    if (!aligned(w, 4) || !aligned(codebook_out, 4)) {
        return fail(NB_EALIGN, "%s: w/codebook not 4-byte aligned", fn);
    }
    int st = ensure_device();
    if (st) return st;
    float q[256];
    linspace01(n_entries, q);
    const int64_t num_blocks = (total + block_size - 1) / block_size;
    return launch_block_codebooks(w, total, num_blocks, block_size, n_entries, q, codebook_out,
                                  static_cast<hipStream_t>(stream));
}

int nb_linspace01(int n, float* out) {
    if (n < 1 || n > 256 || !out) return fail(NB_EINVAL, "nb_linspace01: n=%d", n);
    linspace01(n, out);
    return NB_OK;
}

int nb_quantize_pack(const float* w, int64_t total, const float* codebook, int64_t num_blocks,
                     int n_entries, int block_size, int bits, uint8_t* packed_out, void* stream) {
    const char* fn = "nb_quantize_pack";
    if (bits < 1 || bits > 8) return fail(NB_EUNSUPPORTED, "%s: bits=%d outside 1..8", fn, bits);
    if (n_entries < 1 || n_entries > (1 << bits)) {
        return fail(NB_EINVAL, "%s: n_entries=%d outside 1..2^bits", fn, n_entries);
    }
    if (block_size < 1) return fail(NB_EINVAL, "%s: block_size=%d < 1", fn, block_size);
    if (total < 0 || num_blocks < 0) return fail(NB_EINVAL, "%s: negative size", fn);
    if (num_blocks > (INT64_MAX / 2) / block_size) return fail(NB_EINVAL, "%s: size overflow", fn);
    // the layout of quantize_weight: block_size = ceil(total / num_blocks)
    if (num_blocks * block_size < total || (total > 0 && (num_blocks - 1) * block_size >= total)) {
        return fail(NB_EINVAL, "%s: %lld blocks of %d do not tile %lld weights", fn,
                    (long long)num_blocks, block_size, (long long)total);
    }
    if (total == 0) return NB_OK;
    if (!w || !codebook || !packed_out) return fail(NB_EINVAL, "%s: NULL pointer", fn);
    if (!aligned(w, 4) || !aligned(codebook, 4)) return fail(NB_EALIGN, "%s: w/codebook not 4-byte aligned", fn);
    int st = ensure_device();
    if (st) return st;
    return launch_quantize_pack(w, total, codebook, num_blocks, n_entries, block_size, bits,
                                packed_out, static_cast<hipStream_t>(stream));
}

int nb_dequant(const uint8_t* packed, const float* codebook, void* w_out, int w_dtype,
               int64_t total, int64_t num_blocks, int bits, int n_entries,
               int block_size, void* stream) {
    const char* fn = "nb_dequant";
    int st = check_format(bits, n_entries, block_size, fn);
    if (st) return st;
    if (w_dtype != NB_F32 && w_dtype != NB_BF16) return fail(NB_EINVAL, "%s: w_dtype=%d is not F32/BF16", fn, w_dtype);
    if (total < 0 || num_blocks < 0) return fail(NB_EINVAL, "%s: negative size", fn);
    if (num_blocks > INT64_MAX / block_size || num_blocks * block_size < total) {
        return fail(NB_EINVAL, "%s: num_blocks*block_size < total (%lld blocks of %d for %lld weights)",
                    fn, (long long)num_blocks, block_size, (long long)total);
    }
    if (total == 0) return NB_OK;
    if (!packed || !codebook || !w_out) return fail(NB_EINVAL, "%s: NULL pointer", fn);
    if (!aligned(codebook, 4)) return fail(NB_EALIGN, "%s: codebook not 4-byte aligned", fn);
    if (!aligned(w_out, dtype_size(w_dtype))) return fail(NB_EALIGN, "%s: w_out not aligned to its dtype", fn);
    st = ensure_device();
    if (st) return st;
    return launch_dequant(packed, codebook, w_out, w_dtype, total, num_blocks, bits, n_entries,
                          block_size, static_cast<hipStream_t>(stream));
}

int64_t nb_gemv_batch_table_bytes(int count) {
    return count > 0 ? (int64_t)count * (int64_t)sizeof(StreamProblem) : 0;
}

}  // extern "C"

int nb::build_stream_table(const nb_batch_item* items, int count, StreamProblem* out) {
    int32_t chunk_begin = 0;
    int n = 0;
    for (int i = 0; i < count; ++i) {
        const nb_batch_item& it = items[i];
        if (it.N == 0) continue;
        StreamProblem p;
        memset(&p, 0, sizeof(p));
        p.x = it.x;
        p.packed = it.packed;
        p.codebook = it.codebook;
        p.y = it.y;
        p.norm_w = it.x_mode == NB_X_RMSNORM ? it.norm_w : nullptr;
        p.N = it.N;
        p.K = it.K;
        p.x_mode = it.x_mode;
        p.y_mode = it.y_mode;
        p.eps = it.eps;
        p.bpr = it.K / 128;
        p.nchunks = (int32_t)(((int64_t)it.N * p.bpr + 63) / 64);
        p.chunk_begin = chunk_begin;
        chunk_begin += p.nchunks;
        out[n++] = p;
    }
    return n;
}

namespace {

// Shared validation of batch items; fills the total chunk count and the
// largest K.
int check_batch(const nb_batch_item* items, int count, const char* fn, int64_t* total_chunks,
                int* max_k) {
    if (count < 0) return fail(NB_EINVAL, "%s: count=%d < 0", fn, count);
    if (count > 0 && !items) return fail(NB_EINVAL, "%s: items is NULL", fn);
    int64_t chunks = 0;
    int mk = 0;
    for (int i = 0; i < count; ++i) {
        const nb_batch_item& it = items[i];
        if (it.N < 0 || it.K < 0) return fail(NB_EINVAL, "%s: item %d has a negative shape", fn, i);
        if (it.N == 0) continue;
        if (it.K == 0 || it.K % 128 != 0 || it.K > 8192) {
            return fail(NB_EUNSUPPORTED, "%s: item %d K=%d (needs K %% 128 == 0, 0 < K <= 8192)",
                        fn, i, it.K);
        }
        // block numbers are exact in fp32 below 2^24 (the kernel's row split)
        if ((int64_t)it.N * (it.K / 128) >= (1LL << 24)) {
            return fail(NB_EUNSUPPORTED, "%s: item %d has %lld blocks (limit 2^24)", fn, i,
                        (long long)it.N * (it.K / 128));
        }
        if (!it.x || !it.packed || !it.codebook || !it.y) {
            return fail(NB_EINVAL, "%s: item %d has a NULL pointer", fn, i);
        }
        if (!aligned(it.x, 16) || !aligned(it.packed, 16) || !aligned(it.codebook, 16)) {
            return fail(NB_EALIGN, "%s: item %d x/packed/codebook not 16-byte aligned", fn, i);
        }
        if (!aligned(it.y, 2)) return fail(NB_EALIGN, "%s: item %d y not 2-byte aligned", fn, i);
        if (it.x_mode < NB_X_BF16 || it.x_mode > NB_X_SILU_MUL) {
            return fail(NB_EINVAL, "%s: item %d x_mode=%d", fn, i, it.x_mode);
        }
        if (it.y_mode != NB_Y_STORE && it.y_mode != NB_Y_ADD && it.y_mode != NB_Y_SILU_PAIRS) {
            return fail(NB_EINVAL, "%s: item %d y_mode=%d", fn, i, it.y_mode);
        }
        if (it.y_mode == NB_Y_SILU_PAIRS) {
            if (count != 1) {
                return fail(NB_EUNSUPPORTED, "%s: item %d NB_Y_SILU_PAIRS must be alone in its "
                            "batch (count=%d)", fn, i, count);
            }
            if (it.N % 2) {
                return fail(NB_EINVAL, "%s: item %d NB_Y_SILU_PAIRS with odd N=%d", fn, i, it.N);
            }
        }
        if (it.reserved != 0) return fail(NB_EINVAL, "%s: item %d reserved field not zero", fn, i);
        if (it.x_mode == NB_X_RMSNORM) {
            if (!it.norm_w) return fail(NB_EINVAL, "%s: item %d NB_X_RMSNORM without norm_w", fn, i);
            if (!aligned(it.norm_w, 16)) {
                return fail(NB_EALIGN, "%s: item %d norm_w not 16-byte aligned", fn, i);
            }
            if (!(it.eps >= 0.f) || !std::isfinite(it.eps)) {
                return fail(NB_EINVAL, "%s: item %d eps=%g", fn, i, (double)it.eps);
            }
        }
        chunks += ((int64_t)it.N * (it.K / 128) + 63) / 64;
        if (it.K > mk) mk = it.K;
    }
    if (chunks > INT32_MAX) return fail(NB_EUNSUPPORTED, "%s: %lld chunks exceed int32", fn, (long long)chunks);
    *total_chunks = chunks;
    *max_k = mk;
    return NB_OK;
}

// nb_gemv_batched and nb_gemv_batched_sel: the same checks and kernels; sel
// says the index streams are in the selector-ordered unit layout.
int gemv_batched(const char* fn, const nb_batch_item* items, const void* table_dev, int count,
                 int y_dtype, bool sel, void* stream) {
    int64_t chunks = 0;
    int mk = 0;
    int st = check_batch(items, count, fn, &chunks, &mk);
    if (st) return st;
    if (y_dtype != NB_F32 && y_dtype != NB_BF16) return fail(NB_EINVAL, "%s: y_dtype=%d", fn, y_dtype);
    if (chunks == 0) return NB_OK;
    if (!table_dev) return fail(NB_EINVAL, "%s: table_dev is NULL", fn);
    if (!aligned(table_dev, 8)) return fail(NB_EALIGN, "%s: table_dev not 8-byte aligned", fn);
    int nprob = 0;
    for (int i = 0; i < count; ++i) {
        if (items[i].N == 0) continue;
        ++nprob;
        if (y_dtype == NB_F32 && !aligned(items[i].y, 4)) {
            return fail(NB_EALIGN, "%s: item %d y not 4-byte aligned", fn, i);
        }
        if (items[i].y_mode == NB_Y_ADD && y_dtype != NB_F32) {
            return fail(NB_EUNSUPPORTED, "%s: item %d NB_Y_ADD needs fp32 outputs", fn, i);
        }
        if (items[i].y_mode == NB_Y_SILU_PAIRS && y_dtype != NB_BF16) {
            return fail(NB_EUNSUPPORTED, "%s: item %d NB_Y_SILU_PAIRS needs bf16 outputs", fn, i);
        }
    }
    st = ensure_device();
    if (st) return st;
    // host copy of the table the caller uploaded (same items, same order)
    std::vector<StreamProblem> host((size_t)nprob);
    build_stream_table(items, count, host.data());
    if (host[0].y_mode == NB_Y_SILU_PAIRS && !gemv_rows_fits(host[0])) {
        return fail(NB_EUNSUPPORTED, "%s: NB_Y_SILU_PAIRS item does not fit the single-problem "
                    "kernel's LDS", fn);
    }
    return launch_gemv_stream(static_cast<const StreamProblem*>(table_dev), host.data(), nprob,
                              y_dtype, sel, static_cast<hipStream_t>(stream));
}

}  // namespace

extern "C" {

int nb_gemv_batch_plan(const nb_batch_item* items, int count, void* table_host,
                       int64_t table_bytes) {
    const char* fn = "nb_gemv_batch_plan";
    int64_t chunks = 0;
    int mk = 0;
    int st = check_batch(items, count, fn, &chunks, &mk);
    if (st) return st;
    if (table_bytes < nb_gemv_batch_table_bytes(count)) {
        return fail(NB_EINVAL, "%s: table of %lld bytes, %lld needed", fn, (long long)table_bytes,
                    (long long)nb_gemv_batch_table_bytes(count));
    }
    if (count > 0 && !table_host) return fail(NB_EINVAL, "%s: table_host is NULL", fn);
    // Items with N == 0 are left out; the table holds the others in order and
    // the unused tail of the table is zeroed.
    memset(table_host, 0, (size_t)nb_gemv_batch_table_bytes(count));
    build_stream_table(items, count, static_cast<StreamProblem*>(table_host));
    return NB_OK;
}

int nb_gemv_batched(const nb_batch_item* items, const void* table_dev, int count, int y_dtype,
                    void* stream) {
    return gemv_batched("nb_gemv_batched", items, table_dev, count, y_dtype, false, stream);
}

int nb_gemv_batched_sel(const nb_batch_item* items, const void* table_dev, int count,
                        int y_dtype, void* stream) {
    return gemv_batched("nb_gemv_batched_sel", items, table_dev, count, y_dtype, true, stream);
}

int nb_stream_layout(const uint8_t* packed, uint8_t* out, int N, int K, void* stream) {
    const char* fn = "nb_stream_layout";
    if (N < 0) return fail(NB_EINVAL, "%s: N=%d", fn, N);
    if (K <= 0 || K % 128) return fail(NB_EINVAL, "%s: K=%d must be a positive multiple of 128", fn, K);
    if (N == 0) return NB_OK;
    if (!packed || !out) return fail(NB_EINVAL, "%s: NULL pointer", fn);
    if (!aligned(packed, 4) || !aligned(out, 4)) {
        return fail(NB_EALIGN, "%s: packed/out not 4-byte aligned", fn);
    }
    const int st = ensure_device();
    if (st) return st;
    return launch_stream_layout(packed, out, (int64_t)N * (K / 32),
                                static_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace {

enum SkinnyLayout { kLayoutRows, kLayoutQuad, kLayoutTile };

// nb_gemm_skinny_batched and its row-quad and tile forms: shared
// validation, then the kernel the layout calls for.
int skinny_batched(const nb_batch_item* items, const void* table_dev, int count, int M,
                   int y_dtype, void* stream, SkinnyLayout layout) {
    const bool quad = layout == kLayoutQuad;
    const char* fn = quad                  ? "nb_gemm_skinny_quad_batched"
                     : layout == kLayoutTile ? "nb_gemm_skinny_tile_batched"
                                            : "nb_gemm_skinny_batched";
    int64_t chunks = 0;
    int mk = 0;
    int st = check_batch(items, count, fn, &chunks, &mk);
    if (st) return st;
    const int max_m = quad ? 4 : 16;
    if (M < 1 || M > max_m) return fail(NB_EINVAL, "%s: M=%d outside 1..%d", fn, M, max_m);
    if (y_dtype != NB_F32 && y_dtype != NB_BF16) return fail(NB_EINVAL, "%s: y_dtype=%d", fn, y_dtype);
    if (chunks == 0) return NB_OK;
    if (!table_dev) return fail(NB_EINVAL, "%s: table_dev is NULL", fn);
    if (!aligned(table_dev, 8)) return fail(NB_EALIGN, "%s: table_dev not 8-byte aligned", fn);
    int nprob = 0;
    for (int i = 0; i < count; ++i) {
        if (items[i].N == 0) continue;
        ++nprob;
        if (items[i].x_mode != NB_X_BF16) {
            return fail(NB_EUNSUPPORTED, "%s: item %d: only NB_X_BF16 activations", fn, i);
        }
        if (items[i].y_mode == NB_Y_SILU_PAIRS) {
            return fail(NB_EUNSUPPORTED, "%s: item %d: NB_Y_SILU_PAIRS is for M = 1", fn, i);
        }
        if (y_dtype == NB_F32 && !aligned(items[i].y, 4)) {
            return fail(NB_EALIGN, "%s: item %d y not 4-byte aligned", fn, i);
        }
        if (items[i].y_mode == NB_Y_ADD && y_dtype != NB_F32) {
            return fail(NB_EUNSUPPORTED, "%s: item %d NB_Y_ADD needs fp32 outputs", fn, i);
        }
        if (quad && items[i].K < 2048) {
            return fail(NB_EUNSUPPORTED, "%s: item %d K=%d (the row-quad kernel needs K >= 2048)",
                        fn, i, items[i].K);
        }
    }
    st = ensure_device();
    if (st) return st;
    std::vector<StreamProblem> host((size_t)nprob);
    build_stream_table(items, count, host.data());
    if (quad) {
        return launch_gemv_quad(static_cast<const StreamProblem*>(table_dev), host.data(), nprob,
                                M, y_dtype, static_cast<hipStream_t>(stream));
    }
    return launch_gemv_skinny(static_cast<const StreamProblem*>(table_dev), host.data(), nprob, M,
                              y_dtype, layout == kLayoutTile, static_cast<hipStream_t>(stream));
}

}  // namespace

extern "C" {

int nb_gemm_skinny_batched(const nb_batch_item* items, const void* table_dev, int count, int M,
                           int y_dtype, void* stream) {
    return skinny_batched(items, table_dev, count, M, y_dtype, stream, kLayoutRows);
}

int nb_gemm_skinny_quad_batched(const nb_batch_item* items, const void* table_dev, int count,
                                int M, int y_dtype, void* stream) {
    return skinny_batched(items, table_dev, count, M, y_dtype, stream, kLayoutQuad);
}

int nb_gemm_skinny_tile_batched(const nb_batch_item* items, const void* table_dev, int count,
                                int M, int y_dtype, void* stream) {
    return skinny_batched(items, table_dev, count, M, y_dtype, stream, kLayoutTile);
}

int64_t nb_quad_layout_bytes(int N, int K) {
    if (N < 0 || K < 0 || K % 128) return 0;
    return (int64_t)((N + 3) / 4) * 4 * (K / 128) * 48;
}

int nb_quad_layout(const uint8_t* packed, const float* codebook, int N, int K, uint8_t* qpacked,
                   float* qcodebook, void* stream) {
    const char* fn = "nb_quad_layout";
    if (N < 0 || K <= 0 || K % 128 || K > 8192) {
        return fail(NB_EINVAL, "%s: N=%d K=%d (needs K %% 128 == 0, 0 < K <= 8192)", fn, N, K);
    }
    if (N == 0) return NB_OK;
    if (!packed || !codebook || !qpacked || !qcodebook) {
        return fail(NB_EINVAL, "%s: NULL pointer", fn);
    }
    if (!aligned(packed, 16) || !aligned(codebook, 16) || !aligned(qpacked, 16) ||
        !aligned(qcodebook, 16)) {
        return fail(NB_EALIGN, "%s: packed/codebook/qpacked/qcodebook not 16-byte aligned", fn);
    }
    const int st = ensure_device();
    if (st) return st;
    return launch_quad_layout(packed, codebook, N, K, qpacked, qcodebook,
                              static_cast<hipStream_t>(stream));
}

int64_t nb_tile_layout_bytes(int N, int K) {
    if (N < 0 || K < 0 || K % 128) return 0;
    return tile_layout_tiles(N, K) * 3072;
}

int nb_tile_layout(const uint8_t* packed, const float* codebook, int N, int K, uint8_t* tpacked,
                   float* tcodebook, void* stream) {
    const char* fn = "nb_tile_layout";
    if (N < 0 || K <= 0 || K % 128) {
        return fail(NB_EINVAL, "%s: N=%d K=%d (needs N >= 0, K > 0, K %% 128 == 0)", fn, N, K);
    }
    if (N == 0) return NB_OK;
    if (!packed || !codebook || !tpacked || !tcodebook) {
        return fail(NB_EINVAL, "%s: NULL pointer", fn);
    }
    if (!aligned(packed, 16) || !aligned(codebook, 16) || !aligned(tpacked, 16) ||
        !aligned(tcodebook, 16)) {
        return fail(NB_EALIGN, "%s: packed/codebook/tpacked/tcodebook not 16-byte aligned", fn);
    }
    const int st = ensure_device();
    if (st) return st;
    return launch_tile_layout(packed, codebook, N, K, tpacked, tcodebook,
                              static_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace {
// Shared checks of the head entry points (h: the bf16 input, or the fp32
// residual when the norm is fused in).
int check_head(const char* fn, const void* h, const void* emb, float* logits,
               nb_decode_state* state, int32_t* tokens_out, int tokens_cap,
               const int32_t* force, int n_force, int V, int C, int h_align) {
    if (V < 1 || C < 8 || C % 8 || C > lm_head_max_c()) {
        return fail(NB_EUNSUPPORTED, "%s: V=%d C=%d (C %% 8 == 0, 8 <= C <= %d)", fn, V, C,
                    lm_head_max_c());
    }
    if (!h || !emb || !state) return fail(NB_EINVAL, "%s: NULL pointer", fn);
    if (n_force < 0 || (n_force > 0 && !force)) return fail(NB_EINVAL, "%s: n_force=%d without force", fn, n_force);
    if (tokens_cap < 0 || (tokens_cap > 0 && !tokens_out)) {
        return fail(NB_EINVAL, "%s: tokens_cap=%d without tokens_out", fn, tokens_cap);
    }
    if (!aligned(h, h_align) || !aligned(emb, 16) || (logits && !aligned(logits, 4)) ||
        !aligned(state, 8) || (tokens_out && !aligned(tokens_out, 4))) {
        return fail(NB_EALIGN, "%s: misaligned pointer", fn);
    }
    return NB_OK;
}
}  // namespace

extern "C" {

int nb_add_rmsnorm(float* x, const float* y, const float* emb, const nb_decode_state* state,
                   const float* w, void* h, int h_dtype, int n, float eps, void* stream) {
    const char* fn = "nb_add_rmsnorm";
    if (n < 1) return fail(NB_EINVAL, "%s: n=%d < 1", fn, n);
    if (!x || !w || !h) return fail(NB_EINVAL, "%s: NULL x/w/h", fn);
    if (emb && !state) return fail(NB_EINVAL, "%s: emb given without a state", fn);
    if (h_dtype != NB_F32 && h_dtype != NB_BF16) return fail(NB_EINVAL, "%s: h_dtype=%d", fn, h_dtype);
    if (!(eps >= 0.f)) return fail(NB_EINVAL, "%s: eps must be >= 0", fn);
    if (!aligned(x, 4) || !aligned(w, 4) || (y && !aligned(y, 4)) || (emb && !aligned(emb, 4)) ||
        !aligned(h, dtype_size(h_dtype))) {
        return fail(NB_EALIGN, "%s: misaligned pointer", fn);
    }
    int st = ensure_device();
    if (st) return st;
    return launch_add_rmsnorm(x, y, emb, state, w, h, h_dtype, n, eps, static_cast<hipStream_t>(stream));
}

int nb_attention_work_floats(int n_head) { return n_head > 0 ? attention_work_floats(n_head) : 0; }

int nb_attention_step(const float* qkv, float* k_cache, float* v_cache, const float* cos_t,
                      const float* sin_t, const nb_decode_state* state, float* work,
                      uint32_t* done, void* out, int out_dtype, int n_head, int head_dim,
                      int ctx, void* stream) {
    const char* fn = "nb_attention_step";
    if (n_head < 1 || ctx < 1) return fail(NB_EINVAL, "%s: n_head=%d ctx=%d", fn, n_head, ctx);
    if (ctx > attention_max_ctx()) {
        return fail(NB_EUNSUPPORTED, "%s: ctx=%d > %d", fn, ctx, attention_max_ctx());
    }
    if (head_dim < 2 || head_dim % 2 || head_dim > attention_max_head_dim()) {
        return fail(NB_EUNSUPPORTED, "%s: head_dim=%d (even, <= %d)", fn, head_dim,
                    attention_max_head_dim());
    }
    if (!qkv || !k_cache || !v_cache || !cos_t || !sin_t || !state || !work || !done || !out) {
        return fail(NB_EINVAL, "%s: NULL pointer", fn);
    }
    if (out_dtype != NB_F32 && out_dtype != NB_BF16) return fail(NB_EINVAL, "%s: out_dtype=%d", fn, out_dtype);
    if (!aligned(qkv, 4) || !aligned(k_cache, 4) || !aligned(v_cache, 4) || !aligned(work, 4) ||
        !aligned(done, 4) || !aligned(out, dtype_size(out_dtype))) {
        return fail(NB_EALIGN, "%s: misaligned pointer", fn);
    }
    int st = ensure_device();
    if (st) return st;
    return launch_attention_step(qkv, k_cache, v_cache, cos_t, sin_t, state, work, done, out,
                                 out_dtype, n_head, head_dim, ctx, static_cast<hipStream_t>(stream));
}

int nb_attention_step_static(const float* qkv, float* k_cache, float* v_cache, const float* cos_t,
                             const float* sin_t, const nb_decode_state* state, void* out,
                             int out_dtype, int n_head, int head_dim, int ctx, void* stream) {
    const char* fn = "nb_attention_step_static";
    if (n_head < 1 || ctx < 1) return fail(NB_EINVAL, "%s: n_head=%d ctx=%d", fn, n_head, ctx);
    if (n_head > static_attention_max_heads()) {
        return fail(NB_EUNSUPPORTED, "%s: n_head=%d > %d (the library's static scratch holds "
                    "%d heads; use nb_attention_step with a workspace)", fn, n_head,
                    static_attention_max_heads(), static_attention_max_heads());
    }
    if (ctx > attention_max_ctx()) {
        return fail(NB_EUNSUPPORTED, "%s: ctx=%d > %d", fn, ctx, attention_max_ctx());
    }
    if (head_dim < 2 || head_dim % 2 || head_dim > attention_max_head_dim()) {
        return fail(NB_EUNSUPPORTED, "%s: head_dim=%d (even, <= %d)", fn, head_dim,
                    attention_max_head_dim());
    }
    if (!qkv || !k_cache || !v_cache || !cos_t || !sin_t || !state || !out) {
        return fail(NB_EINVAL, "%s: NULL pointer", fn);
    }
    if (out_dtype != NB_F32 && out_dtype != NB_BF16) return fail(NB_EINVAL, "%s: out_dtype=%d", fn, out_dtype);
    if (!aligned(qkv, 4) || !aligned(k_cache, 4) || !aligned(v_cache, 4) ||
        !aligned(out, dtype_size(out_dtype))) {
        return fail(NB_EALIGN, "%s: misaligned pointer", fn);
    }
    int st = ensure_device();
    if (st) return st;
    float* work = nullptr;
    unsigned* done = nullptr;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    st = static_attention_scratch(s, &work, &done);
    if (st) return st;
    return launch_attention_step(qkv, k_cache, v_cache, cos_t, sin_t, state, work, done, out,
                                 out_dtype, n_head, head_dim, ctx, s);
}

int64_t nb_attention_static_scratch_bytes(void) { return static_attention_scratch_bytes(); }

int nb_rmsnorm_rows(float* x, const float* add, const float* emb, const int32_t* tokens,
                    int vocab, const float* w, void* h, int h_dtype, int T, int C, float eps,
                    void* stream) {
    const char* fn = "nb_rmsnorm_rows";
    if (T < 0 || C < 1) return fail(NB_EINVAL, "%s: T=%d C=%d", fn, T, C);
    if (!(eps >= 0.f) || !std::isfinite(eps)) return fail(NB_EINVAL, "%s: eps=%g", fn, (double)eps);
    if (h_dtype != NB_F32 && h_dtype != NB_BF16) return fail(NB_EINVAL, "%s: h_dtype=%d", fn, h_dtype);
    if (!x || !w || !h) return fail(NB_EINVAL, "%s: NULL x, w or h", fn);
    if ((emb == nullptr) != (tokens == nullptr)) {
        return fail(NB_EINVAL, "%s: emb and tokens go together", fn);
    }
    if (emb && add) return fail(NB_EINVAL, "%s: an embedding lookup takes no add", fn);
    if (emb && vocab < 1) return fail(NB_EINVAL, "%s: vocab=%d rows in the embedding", fn, vocab);
    if (!aligned(x, 4) || !aligned(w, 4) || (add && !aligned(add, 4)) || (emb && !aligned(emb, 4)) ||
        (tokens && !aligned(tokens, 4)) || !aligned(h, dtype_size(h_dtype))) {
        return fail(NB_EALIGN, "%s: misaligned pointer", fn);
    }
    if (T == 0) return NB_OK;
    int st = ensure_device();
    if (st) return st;
    return launch_rmsnorm_rows(x, add, emb, tokens, vocab, w, h, h_dtype, T, C, eps,
                               static_cast<hipStream_t>(stream));
}

int nb_silu_pairs_rows(const float* gu, void* act, int act_dtype, int T, int F, void* stream) {
    const char* fn = "nb_silu_pairs_rows";
    if (T < 0 || F < 1) return fail(NB_EINVAL, "%s: T=%d F=%d", fn, T, F);
    if (act_dtype != NB_F32 && act_dtype != NB_BF16) return fail(NB_EINVAL, "%s: act_dtype=%d", fn, act_dtype);
    if (!gu || !act) return fail(NB_EINVAL, "%s: NULL pointer", fn);
    if (!aligned(gu, 4) || !aligned(act, dtype_size(act_dtype))) {
        return fail(NB_EALIGN, "%s: misaligned pointer", fn);
    }
    if (T == 0) return NB_OK;
    int st = ensure_device();
    if (st) return st;
    return launch_silu_pairs_rows(gu, act, act_dtype, T, F, static_cast<hipStream_t>(stream));
}

namespace {
int check_rows_attention(const char* fn, int pos0, int T, int n_head, int head_dim, int ctx) {
    if (T < 0 || n_head < 1 || ctx < 1 || pos0 < 0) {
        return fail(NB_EINVAL, "%s: T=%d n_head=%d ctx=%d pos0=%d", fn, T, n_head, ctx, pos0);
    }
    if ((int64_t)pos0 + T > ctx) {
        return fail(NB_EINVAL, "%s: positions %d..%d beyond the cache (ctx=%d)", fn, pos0,
                    pos0 + T - 1, ctx);
    }
    if (head_dim < 2 || head_dim % 2 || head_dim > attention_rows_max_head_dim()) {
        return fail(NB_EUNSUPPORTED, "%s: head_dim=%d (even, <= %d)", fn, head_dim,
                    attention_rows_max_head_dim());
    }
    return NB_OK;
}
}  // namespace

int nb_rope_kv_rows(const float* qkv, float* k_cache, float* v_cache, const float* cos_t,
                    const float* sin_t, int pos0, int T, float* q_out, int n_head, int head_dim,
                    int ctx, void* stream) {
    const char* fn = "nb_rope_kv_rows";
    int st = check_rows_attention(fn, pos0, T, n_head, head_dim, ctx);
    if (st) return st;
    if (!qkv || !k_cache || !v_cache || !cos_t || !sin_t || !q_out) {
        return fail(NB_EINVAL, "%s: NULL pointer", fn);
    }
    if (!aligned(qkv, 4) || !aligned(k_cache, 4) || !aligned(v_cache, 4) || !aligned(cos_t, 4) ||
        !aligned(sin_t, 4) || !aligned(q_out, 4)) {
        return fail(NB_EALIGN, "%s: misaligned pointer", fn);
    }
    if (T == 0) return NB_OK;
    st = ensure_device();
    if (st) return st;
    return launch_rope_kv_rows(qkv, k_cache, v_cache, cos_t, sin_t, pos0, T, q_out, n_head,
                               head_dim, ctx, static_cast<hipStream_t>(stream));
}

int nb_attention_rows(const float* q, const float* k_cache, const float* v_cache, int pos0, int T,
                      void* out, int out_dtype, int n_head, int head_dim, int ctx, void* stream) {
    const char* fn = "nb_attention_rows";
    int st = check_rows_attention(fn, pos0, T, n_head, head_dim, ctx);
    if (st) return st;
    if (out_dtype != NB_F32 && out_dtype != NB_BF16) return fail(NB_EINVAL, "%s: out_dtype=%d", fn, out_dtype);
    if (!q || !k_cache || !v_cache || !out) return fail(NB_EINVAL, "%s: NULL pointer", fn);
    if (!aligned(q, 4) || !aligned(k_cache, 4) || !aligned(v_cache, 4) ||
        !aligned(out, dtype_size(out_dtype))) {
        return fail(NB_EALIGN, "%s: misaligned pointer", fn);
    }
    if (T == 0) return NB_OK;
    st = ensure_device();
    if (st) return st;
    return launch_attention_rows(q, k_cache, v_cache, pos0, T, out, out_dtype, n_head, head_dim,
                                 ctx, static_cast<hipStream_t>(stream));
}

int nb_silu_mul(const float* gu, void* act, int act_dtype, int n, void* stream) {
    const char* fn = "nb_silu_mul";
    if (n < 1) return fail(NB_EINVAL, "%s: n=%d < 1", fn, n);
    if (!gu || !act) return fail(NB_EINVAL, "%s: NULL pointer", fn);
    if (act_dtype != NB_F32 && act_dtype != NB_BF16) return fail(NB_EINVAL, "%s: act_dtype=%d", fn, act_dtype);
    if (!aligned(gu, 4) || !aligned(act, dtype_size(act_dtype))) return fail(NB_EALIGN, "%s: misaligned pointer", fn);
    int st = ensure_device();
    if (st) return st;
    return launch_silu_mul(gu, act, act_dtype, n, static_cast<hipStream_t>(stream));
}

int nb_rmsnorm_lm_head_argmax(const float* x, const float* norm_w, float eps, const void* emb,
                              float* logits, nb_decode_state* state, int32_t* tokens_out,
                              int tokens_cap, const int32_t* force, int n_force, int V, int C,
                              void* stream) {
    const char* fn = "nb_rmsnorm_lm_head_argmax";
    int st = check_head(fn, x, emb, logits, state, tokens_out, tokens_cap, force, n_force, V, C, 4);
    if (st) return st;
    if (!norm_w) return fail(NB_EINVAL, "%s: norm_w is NULL", fn);
    if (!aligned(norm_w, 4)) return fail(NB_EALIGN, "%s: norm_w not 4-byte aligned", fn);
    if (!(eps >= 0.f) || !std::isfinite(eps)) return fail(NB_EINVAL, "%s: eps=%g", fn, (double)eps);
    st = ensure_device();
    if (st) return st;
    return launch_lm_head_argmax(nullptr, x, norm_w, eps, emb, logits, state, tokens_out,
                                 tokens_cap, force, n_force, V, C, static_cast<hipStream_t>(stream));
}

int nb_lm_head_argmax(const void* h, const void* emb, float* logits, nb_decode_state* state,
                      int32_t* tokens_out, int tokens_cap, const int32_t* force, int n_force,
                      int V, int C, void* stream) {
    const char* fn = "nb_lm_head_argmax";
    int st = check_head(fn, h, emb, logits, state, tokens_out, tokens_cap, force, n_force, V, C, 2);
    if (st) return st;
    st = ensure_device();
    if (st) return st;
    return launch_lm_head_argmax(h, nullptr, nullptr, 0.f, emb, logits, state, tokens_out,
                                 tokens_cap, force, n_force, V, C, static_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace {
// Argument checks shared by the fused prefill entry points; NB_OK (then
// M, N > 0) or a status, with *done set for an empty product.
int check_prefill(const char* fn, const void* x, int64_t ldx, const uint8_t* packed,
                  const float* codebook, const void* y, int y_dtype, int64_t ldy, int M, int N,
                  int K, bool* done) {
    *done = false;
    if (M < 0 || N < 0 || K < 0) return fail(NB_EINVAL, "%s: negative shape", fn);
    if (K % 128 != 0) return fail(NB_EUNSUPPORTED, "%s: K=%d not a multiple of 128", fn, K);
    if ((int64_t)N * (K / 128) >= (1LL << 31)) return fail(NB_EUNSUPPORTED, "%s: too many blocks", fn);
    if (y_dtype != NB_F32 && y_dtype != NB_BF16) return fail(NB_EINVAL, "%s: y_dtype=%d", fn, y_dtype);
    if (M == 0 || N == 0) {
        *done = true;
        return NB_OK;
    }
    if (K == 0) return fail(NB_EUNSUPPORTED, "%s: K == 0 (use nb_gemv)", fn);
    if (ldx < K || ldy < N) return fail(NB_EINVAL, "%s: ldx=%lld < K or ldy=%lld < N", fn,
                                        (long long)ldx, (long long)ldy);
    if (!x || !packed || !codebook || !y) return fail(NB_EINVAL, "%s: NULL pointer", fn);
    if (!aligned(x, 16) || ldx % 8 != 0) return fail(NB_EALIGN, "%s: x must be 16-byte aligned with ldx %% 8 == 0", fn);
    if (!aligned(packed, 8) || !aligned(codebook, 16)) return fail(NB_EALIGN, "%s: packed 8- / codebook 16-byte alignment", fn);
    if (!aligned(y, dtype_size(y_dtype))) return fail(NB_EALIGN, "%s: y not aligned to its dtype", fn);
    return NB_OK;
}
}  // namespace

extern "C" int nb_gemm_prefill(const void* x, int64_t ldx, const uint8_t* packed,
                               const float* codebook, void* y, int y_dtype, int64_t ldy, int M,
                               int N, int K, void* stream) {
    bool done;
    int st = check_prefill("nb_gemm_prefill", x, ldx, packed, codebook, y, y_dtype, ldy, M, N, K,
                           &done);
    if (st || done) return st;
    st = ensure_device();
    if (st) return st;
    return launch_prefill2(x, ldx, packed, codebook, y, y_dtype, ldy, M, N, K, nullptr, 0,
                           static_cast<hipStream_t>(stream));
}

extern "C" int64_t nb_gemm_prefill_split_ws_bytes(int M, int N, int K) {
    // without a usable device the plan assumes 256 CUs (and no error is left)
    if (ensure_device() != NB_OK) g_last_error[0] = '\0';
    return prefill_split_bytes(M, N, K);
}

extern "C" int nb_gemm_prefill_split(const void* x, int64_t ldx, const uint8_t* packed,
                                     const float* codebook, void* y, int y_dtype, int64_t ldy,
                                     int M, int N, int K, void* workspace, int64_t ws_bytes,
                                     void* stream) {
    const char* fn = "nb_gemm_prefill_split";
    bool done;
    int st = check_prefill(fn, x, ldx, packed, codebook, y, y_dtype, ldy, M, N, K, &done);
    if (st || done) return st;
    if (ws_bytes < 0) return fail(NB_EINVAL, "%s: ws_bytes=%lld", fn, (long long)ws_bytes);
    if (!aligned(workspace, 256)) return fail(NB_EALIGN, "%s: workspace not 256-byte aligned", fn);
    // the size check comes before the device's status, so that it holds (for
    // 256 CUs) where there is no device
    const int dev_st = ensure_device();
    const int64_t need = prefill_split_bytes(M, N, K);
    if (ws_bytes < need || (need > 0 && !workspace)) {
        return fail(NB_EINVAL, "%s: workspace of %lld bytes < %lld", fn, (long long)ws_bytes,
                    (long long)need);
    }
    if (dev_st) return dev_st;
    return launch_prefill2(x, ldx, packed, codebook, y, y_dtype, ldy, M, N, K,
                           need > 0 ? workspace : nullptr, ws_bytes,
                           static_cast<hipStream_t>(stream));
}

extern "C" int64_t nb_gemm_prefill_f32_ws_bytes(int M, int N, int K) {
    return prefill_f32_bytes(M, N, K);
}

extern "C" int nb_gemm_prefill_f32(const float* x, int64_t ldx, const uint8_t* packed,
                                   const float* codebook, float* y, int64_t ldy, int M, int N,
                                   int K, void* workspace, int64_t ws_bytes, void* stream) {
    const char* fn = "nb_gemm_prefill_f32";
    if (M < 0 || N < 0 || K < 0) return fail(NB_EINVAL, "%s: negative shape", fn);
    if (K % 128 != 0) return fail(NB_EUNSUPPORTED, "%s: K=%d not a multiple of 128", fn, K);
    if ((int64_t)N * (K / 128) >= (1LL << 31) || (int64_t)M * K >= (1LL << 40)) {
        return fail(NB_EUNSUPPORTED, "%s: shape too large", fn);
    }
    if (M == 0 || N == 0) return NB_OK;
    if (K == 0) return fail(NB_EUNSUPPORTED, "%s: K == 0 (use nb_gemv)", fn);
    if (ldx < K || ldy < N) return fail(NB_EINVAL, "%s: ldx=%lld < K or ldy=%lld < N", fn,
                                        (long long)ldx, (long long)ldy);
    if (!x || !packed || !codebook || !y || !workspace) return fail(NB_EINVAL, "%s: NULL pointer", fn);
    if (!aligned(x, 4) || !aligned(y, 4)) return fail(NB_EALIGN, "%s: x or y not 4-byte aligned", fn);
    if (!aligned(packed, 8) || !aligned(codebook, 16)) return fail(NB_EALIGN, "%s: packed 8- / codebook 16-byte alignment", fn);
    if (!aligned(workspace, 256)) return fail(NB_EALIGN, "%s: workspace not 256-byte aligned", fn);
    const int dev_st = ensure_device();
    const int64_t need = prefill_f32_bytes(M, N, K);
    if (ws_bytes < need) {
        return fail(NB_EINVAL, "%s: workspace of %lld bytes < %lld", fn, (long long)ws_bytes,
                    (long long)need);
    }
    if (dev_st) return dev_st;
    return launch_prefill_f32(x, ldx, packed, codebook, y, ldy, M, N, K, workspace, ws_bytes,
                              static_cast<hipStream_t>(stream));
}

namespace {
// Shapes and pointers of a persistent-decode model; NB_OK or a status.
int check_decode_model(const nb_decode_model* m, const char* fn) {
    if (!m) return fail(NB_EINVAL, "%s: NULL model", fn);
    int max_c, max_f, max_d, max_ctx, max_heads, max_layers;
    decode_persistent_limits(&max_c, &max_f, &max_d, &max_ctx, &max_heads, &max_layers);
    if (m->n_layers < 1 || m->n_embd < 1 || m->n_head < 1 || m->head_dim < 1 ||
        m->ffn_hidden < 1 || m->vocab < 1 || m->ctx < 1) {
        return fail(NB_EINVAL, "%s: non-positive model dimension", fn);
    }
    if (m->n_layers > max_layers) {
        return fail(NB_EUNSUPPORTED, "%s: n_layers=%d > %d", fn, m->n_layers, max_layers);
    }
    if (m->n_embd % 128 || m->ffn_hidden % 128 || m->n_embd > max_c || m->ffn_hidden > max_f) {
        return fail(NB_EUNSUPPORTED, "%s: n_embd=%d / ffn_hidden=%d (multiples of 128, <= %d / %d)",
                    fn, m->n_embd, m->ffn_hidden, max_c, max_f);
    }
    if (m->head_dim % 2 || m->head_dim > max_d || (int64_t)m->n_head * m->head_dim != m->n_embd ||
        m->n_head > max_heads) {
        return fail(NB_EUNSUPPORTED, "%s: n_head=%d head_dim=%d (even head_dim <= %d, "
                    "n_head * head_dim == n_embd, n_head <= %d)", fn, m->n_head, m->head_dim,
                    max_d, max_heads);
    }
    if (m->ctx > max_ctx) return fail(NB_EUNSUPPORTED, "%s: ctx=%d > %d", fn, m->ctx, max_ctx);
    if (!(m->eps >= 0.f)) return fail(NB_EINVAL, "%s: eps must be >= 0", fn);
    if (!m->layers || !m->ln_f || !m->emb_f32 || !m->emb_bf16 || !m->rope_cos || !m->rope_sin) {
        return fail(NB_EINVAL, "%s: NULL model pointer", fn);
    }
    if (!aligned(m->layers, 8) || !aligned(m->ln_f, 4) || !aligned(m->emb_f32, 4) ||
        !aligned(m->emb_bf16, 16) || !aligned(m->rope_cos, 4) || !aligned(m->rope_sin, 4)) {
        return fail(NB_EALIGN, "%s: misaligned model pointer", fn);
    }
    return NB_OK;
}
}  // namespace

extern "C" int64_t nb_decode_workspace_bytes(const nb_decode_model* model) {
    if (check_decode_model(model, "nb_decode_workspace_bytes")) return 0;
    return decode_persistent_workspace_bytes(model->n_embd, model->n_head, model->ffn_hidden);
}

extern "C" int nb_decode_persistent(const nb_decode_model* model, void* workspace,
                                    int64_t workspace_bytes, nb_decode_state* state, float* logits,
                                    int32_t* tokens_out, int tokens_cap, const int32_t* force,
                                    int n_force, int n_steps, int spin_limit, void* stream) {
    const char* fn = "nb_decode_persistent";
    int st = check_decode_model(model, fn);
    if (st) return st;
    if (n_steps < 0) return fail(NB_EINVAL, "%s: n_steps=%d < 0", fn, n_steps);
    if (!workspace || !state) return fail(NB_EINVAL, "%s: NULL workspace or state", fn);
    const int64_t need = decode_persistent_workspace_bytes(model->n_embd, model->n_head,
                                                           model->ffn_hidden);
    if (workspace_bytes < need) {
        return fail(NB_EINVAL, "%s: workspace of %lld bytes, %lld needed", fn,
                    (long long)workspace_bytes, (long long)need);
    }
    if (n_force < 0 || (n_force > 0 && !force)) return fail(NB_EINVAL, "%s: n_force=%d without force", fn, n_force);
    if (tokens_cap < 0 || (tokens_cap > 0 && !tokens_out)) {
        return fail(NB_EINVAL, "%s: tokens_cap=%d without tokens_out", fn, tokens_cap);
    }
    if (!aligned(workspace, 256) || !aligned(state, 8) || (logits && !aligned(logits, 4)) ||
        (tokens_out && !aligned(tokens_out, 4)) || (force && !aligned(force, 4))) {
        return fail(NB_EALIGN, "%s: misaligned pointer (workspace needs 256 bytes)", fn);
    }
    if (n_steps == 0) return NB_OK;
    st = ensure_device();
    if (st) return st;
    // The kernel made an illegal memory access on a 26-layer model in a
    // 128-step launch and the cause has not been shown: it is not launched.
    (void)logits;
    (void)spin_limit;
    (void)stream;
    return fail(NB_EUNSUPPORTED,
                "%s: switched off (an illegal memory access on a 26-layer model is not yet "
                "explained); use the per-launch decode step", fn);
}
