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
// Shared memory (LDS) bytes one workgroup may use on the current device.
int device_lds_bytes();

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

// One GEMV of a batch as the streaming kernel reads it (device table entry,
// written on the host by nb_gemv_batch_plan).
struct StreamProblem {
    const void* x;            // activations in the form x_mode names
    const uint8_t* packed;    // 3-bit stream
    const float* codebook;    // (N*K/128) x 8
    void* y;                  // N outputs
    const float* norm_w;      // NB_X_RMSNORM weights
    int32_t N, K;
    int32_t bpr;              // 128-weight blocks per row
    int32_t nchunks;          // 64-block chunks: ceil(N * bpr / 64)
    int32_t chunk_begin;      // chunks of all earlier problems
    int32_t x_mode;           // nb_x_mode
    int32_t y_mode;           // nb_y_mode
    float eps;                // NB_X_RMSNORM epsilon
};
static_assert(sizeof(StreamProblem) == 72, "StreamProblem layout");

// Chunk ranges of one streaming launch (kernel argument, by value):
// workgroup g owns chunks [chunk0[g], chunk0[g+1]) of problems prob0[g] ..
// prob1[g]; every range starts and ends on a row boundary.
constexpr int kStreamMaxGroups = 256;
struct StreamRanges {
    int32_t chunk0[kStreamMaxGroups + 1];
    int32_t prob0[kStreamMaxGroups];
    int32_t prob1[kStreamMaxGroups];
};

// Workgroup tasks of one skinny-GEMM launch (kernel argument, by value):
// problems prob0 .. prob0 + nprob - 1 of the table; problem prob0 + i owns
// tasks task_begin[i] .. (128 rows each).
constexpr int kSkinnyMaxProbs = 512;
struct SkinnyTasks {
    int32_t task_begin[kSkinnyMaxProbs];
    int32_t prob0;
    int32_t nprob;
};

// Fills `out` (nprob entries) from the batch items with N > 0, in order;
// returns nprob.
int build_stream_table(const nb_batch_item* items, int count, StreamProblem* out);

// Launches the streaming kernel over the problem table (device copy for the
// kernel, host copy to plan the workgroup ranges).
// One problem per launch, whole-row chunks (nb_gemv_rows.hip): the launches
// of a decode step.  gemv_rows_fits says whether its LDS holds the problem.
bool gemv_rows_fits(const StreamProblem& p);
// sel: the index streams are in the selector-ordered unit layout
// (launch_stream_layout).
int launch_gemv_rows(const StreamProblem& p, int y_dtype, bool sel, hipStream_t stream);
int launch_gemv_stream(const StreamProblem* dev_probs, const StreamProblem* host_probs,
                       int nprob, int y_dtype, bool sel, hipStream_t stream);
// Rewrites `units` 12-byte units of a 3-bit stream into the selector-ordered
// unit layout (in place allowed).
int launch_stream_layout(const uint8_t* in, uint8_t* out, int64_t units, hipStream_t stream);

// Launches the batched skinny GEMM (M <= 16 activation rows) over the
// problem table.
// tile: items are in the tile layout (nb_tile_layout).
int launch_gemv_skinny(const StreamProblem* dev_probs, const StreamProblem* host_probs,
                       int nprob, int M, int y_dtype, bool tile, hipStream_t stream);
// Tiles (16 rows x 4 column blocks) of an N x K layer's tile layout, and
// the launch that writes it (3072 index bytes and 512 floats per tile).
int64_t tile_layout_tiles(int N, int K);
int launch_tile_layout(const uint8_t* packed, const float* codebook, int N, int K,
                       uint8_t* tpacked, float* tcodebook, hipStream_t stream);

// The batched skinny GEMM for M <= 4 on the row-quad layout
// (nb_gemv_quad.hip); gemv_quad_supported says whether the batch is in its
// domain (M, K >= 2048, bf16 x, LDS).
bool gemv_quad_supported(const StreamProblem* host_probs, int nprob, int M);
int launch_gemv_quad(const StreamProblem* dev_probs, const StreamProblem* host_probs,
                     int nprob, int M, int y_dtype, hipStream_t stream);
// Writes the row-quad layout of an N x K layer.
int launch_quad_layout(const uint8_t* packed, const float* codebook, int N, int K,
                       uint8_t* qpacked, float* qcodebook, hipStream_t stream);

// Kernel launchers (arguments already validated by nb_abi.cpp).
int launch_gemv(const GemvArgs& a, hipStream_t stream);
// The bf16-activation MFMA GEMV; returns 1 (launching nothing) when the
// problem is outside its 3-bit / 8-entry / block-128 / aligned domain.
int launch_gemv_mfma(const GemvArgs& a, hipStream_t stream);
int launch_unpack(const uint8_t* packed, uint8_t* out, int64_t count, int bits,
                  hipStream_t stream);
int launch_pack(const uint8_t* idx, uint8_t* out, int64_t count, int bits,
                hipStream_t stream);
int launch_block_codebooks(const float* w, int64_t total, int64_t num_blocks, int block_size,
                           int n_entries, const float* q, float* cb, hipStream_t stream);
int launch_quantize_pack(const float* w, int64_t total, const float* codebook,
                         int64_t num_blocks, int n_entries, int block_size, int bits,
                         uint8_t* out, hipStream_t stream);
int launch_dequant(const uint8_t* packed, const float* codebook, void* w,
                   int w_dtype, int64_t total, int64_t num_blocks, int bits,
                   int n_entries, int block_size, hipStream_t stream);


// Prefill GEMM with a packed weight (nb_prefill2.hip): the packed weight
// dequantized into LDS tiles, bf16 MFMAs; arguments validated.  With a
// workspace of at least prefill_split_bytes(M, N, K) bytes, a layer whose
// tile grid leaves CUs idle is split over K ranges (fp32 partial products in
// the workspace, then one reduction launch); otherwise (workspace null) one
// launch over all of K.
int launch_prefill2(const void* x, int64_t ldx, const uint8_t* packed, const float* codebook,
                    void* y, int y_dtype, int64_t ldy, int M, int N, int K, void* workspace,
                    int64_t ws_bytes, hipStream_t stream, bool accumulate = false);
int64_t prefill_split_bytes(int M, int N, int K);
// fp32 activations: x split into bf16 hi + lo, the residual codebook cb -
// bf16(cb), three prefill passes accumulated in fp32 (workspace of
// prefill_f32_bytes(M, N, K) bytes, 256-byte aligned).
int64_t prefill_f32_bytes(int M, int N, int K);
int launch_prefill_f32(const float* x, int64_t ldx, const uint8_t* packed, const float* codebook,
                       float* y, int64_t ldy, int M, int N, int K, void* workspace,
                       int64_t ws_bytes, hipStream_t stream);

// Decode-step kernels (nb_decode.hip).
int launch_add_rmsnorm(float* x, const float* y, const float* emb, const nb_decode_state* st,
                       const float* w, void* h, int h_dtype, int n, float eps, hipStream_t stream);
int launch_attention_step(const float* qkv, float* k_cache, float* v_cache, const float* cos_t,
                          const float* sin_t, const nb_decode_state* st, float* work,
                          unsigned* done, void* out, int out_dtype, int n_head, int head_dim,
                          int ctx, hipStream_t stream);
int launch_silu_mul(const float* gu, void* act, int dtype, int n, hipStream_t stream);
// x != NULL: the head's input is RMSNorm(x) * norm_w (fp32 x), else bf16 h.
int launch_lm_head_argmax(const void* h, const float* x, const float* norm_w, float eps,
                          const void* emb, float* logits, nb_decode_state* st,
                          int32_t* tokens_out, int tokens_cap, const int32_t* force, int n_force,
                          int V, int C, hipStream_t stream);
int attention_work_floats(int n_head);
// The allocation-free attention's scratch on the current device (its
// address from hipGetSymbolAddress, set up once per device).
int static_attention_scratch(hipStream_t stream, float** work, unsigned** done);
int static_attention_max_heads();
int64_t static_attention_scratch_bytes();

// Batched-pass kernels (nb_rows.hip); arguments validated.
int launch_rmsnorm_rows(float* x, const float* add, const float* emb, const int32_t* tokens,
                        int vocab, const float* w, void* h, int h_dtype, int T, int C, float eps,
                        hipStream_t stream);
int launch_silu_pairs_rows(const float* gu, void* act, int act_dtype, int T, int F,
                           hipStream_t stream);
int launch_rope_kv_rows(const float* qkv, float* k_cache, float* v_cache, const float* cos_t,
                        const float* sin_t, int pos0, int T, float* q_out, int n_head, int D,
                        int ctx, hipStream_t stream);
int launch_attention_rows(const float* q, const float* k_cache, const float* v_cache, int pos0,
                          int T, void* out, int out_dtype, int n_head, int D, int ctx,
                          hipStream_t stream);
int attention_rows_max_head_dim();

// Persistent decode (nb_decode_persistent.hip); arguments validated.
int64_t decode_persistent_workspace_bytes(int C, int H, int F);
int decode_persistent_limits(int* max_c, int* max_f, int* max_d, int* max_ctx, int* max_heads,
                             int* max_layers);
int launch_decode_persistent(const nb_decode_model& m, void* workspace, nb_decode_state* st,
                             float* logits, int32_t* tokens_out, int tokens_cap,
                             const int32_t* force, int n_force, int n_steps, int spin_limit,
                             hipStream_t stream);
int attention_max_head_dim();
int attention_max_ctx();
int lm_head_max_c();

}  // namespace nb
