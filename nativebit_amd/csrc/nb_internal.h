// Internal declarations shared by the C-ABI layer (nb_abi.cpp) and the
// kernel translation units (*.hip).  Not installed; the public interface is
// include/nativebit_amd.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nativebit_amd.h"

namespace nb {

// Records a thread-local error message and returns `status`.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Checks the HIP error state after a launch; NB_OK or NB_ELAUNCH.
int check_launch(const char* what);

// Multiprocessor count of the current device (cached per device).
int device_cu_count();

// Packed stream length, mirroring nb_packed_nbytes.
inline int64_t packed_nbytes(int64_t count, int bits) {
    if (bits < 1 || bits > 8 || count < 0) return 0;
    if (bits == 3) return ((count + 7) / 8) * 3;
    return (count * bits + 7) / 8;
}

struct GemvArgs {
    const void* x;
    int x_dtype;
    int64_t ldx;
    const uint8_t* packed;
    int64_t packed_bytes;   // readable length of the stream
    const float* codebook;
    void* y;
    int y_dtype;
    int64_t ldy;
    int M, N, K, bits, n_entries, block_size;
};

// Kernel launchers (arguments already validated by nb_abi.cpp).
int launch_gemv(const GemvArgs& a, hipStream_t stream);
int launch_unpack(const uint8_t* packed, uint8_t* out, int64_t count, int bits,
                  hipStream_t stream);
int launch_pack(const uint8_t* idx, uint8_t* out, int64_t count, int bits,
                hipStream_t stream);
int launch_dequant(const uint8_t* packed, const float* codebook, void* w,
                   int w_dtype, int64_t total, int64_t num_blocks, int bits,
                   int n_entries, int block_size, hipStream_t stream);

}  // namespace nb
