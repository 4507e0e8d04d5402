// extern "C" boundary of libnativebit_amd.so: argument validation, error
// reporting and dispatch to the gfx950 kernels.  Every check here runs on
// the host before any launch, so the whole validation surface can be tested
// without a GPU.  Unlike the reference operator, which checks nothing and
// hides every failure behind a bare `except Exception` fallback
// (inference/triton_kernel.py:244-257), each failure returns a distinct
// status with a message and nothing is launched.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "nb_internal.h"

namespace nb {
namespace {

thread_local char g_last_error[512] = "";

constexpr int kMaxDevices = 64;
int g_cu_count[kMaxDevices];
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

}  // extern "C"
