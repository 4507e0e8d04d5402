/*
 * nativebit_amd.h -- C ABI of libnativebit_amd.so, the MI355X (gfx950)
 * packed-weight decode path for NativeBit codebook-quantized layers.
 *
 * Data format (identical to the reference, byte for byte):
 *   - weights W (N x K, row major) are split into flat blocks of
 *     `block_size` consecutive weights: block j covers flat elements
 *     [j*block_size, (j+1)*block_size) of W.reshape(-1); the last block is
 *     zero padded.  num_blocks = ceil(N*K / block_size).
 *     (nativebit/layers.py:43-50)
 *   - codebook: float32 [num_blocks][n_entries], row major.
 *   - packed indices: one index per (padded) weight, bits = ceil(log2
 *     n_entries), written LSB first into a little-endian bit stream: index i
 *     occupies stream bits [i*bits, (i+1)*bits).  3-bit streams are padded
 *     to whole 24-bit groups (3 bytes per 8 indices), others to whole bytes.
 *     (nativebit/pack.py:21-138, inference/pack.py:38-57,
 *      inference/triton_kernel.py:199-220)
 *   - dequantized weight: W.flat[i] = codebook[i / block_size][index i].
 *     (nativebit/pack.py:145-169, inference/triton_kernel.py:268-273)
 *
 * Conventions:
 *   - Every function returns 0 (NB_OK) or a negative nb_status.  Argument
 *     checks run on the host before anything is launched, so they can be
 *     exercised without a GPU; nb_last_error() gives a thread-local message.
 *   - Device pointers are caller-owned; the library never allocates device
 *     memory and never synchronizes.  Work is enqueued on `stream` (a
 *     hipStream_t; NULL = the default stream) and is graph-capturable.
 *   - Element types are passed as nb_dtype codes; activations x and outputs
 *     y may be NB_F32 or NB_BF16.  Arithmetic: with NB_F32 activations the
 *     weights are the exact fp32 codebook values; with NB_BF16 activations
 *     they are the codebook values rounded to bf16 (round to nearest even),
 *     the reference's bf16 path (inference/eval_ppl.py:149-174).  Products
 *     are exact in fp32 and sums are fp32.
 */
#ifndef NATIVEBIT_AMD_H
#define NATIVEBIT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NB_ABI_VERSION 2

enum nb_status {
    NB_OK = 0,
    NB_EINVAL = -1,        /* bad argument: null pointer, negative size, ... */
    NB_EUNSUPPORTED = -2,  /* valid format the library has no kernel for      */
    NB_EALIGN = -3,        /* pointer not aligned to its element type         */
    NB_ELAUNCH = -4,       /* the HIP runtime refused the launch              */
    NB_ENODEV = -5         /* no usable gfx950 device                         */
};

enum nb_dtype {
    NB_F32 = 0,
    NB_BF16 = 1,
    NB_U8 = 2
};

/* Version of this ABI (NB_ABI_VERSION of the build). */
int nb_abi_version(void);

/* Message for the last non-zero status returned on this thread. */
const char* nb_last_error(void);

/* Bytes of a packed stream of `count` indices of `bits` bits (0 if bits is
 * out of 1..8).  Mirrors the padding of nativebit/pack.py:29-32 (3-bit) and
 * 105-107 (others). */
int64_t nb_packed_nbytes(int64_t count, int bits);

/*
 * Fused dequant + matvec / skinny GEMM:
 *     y[m][n] = sum_k x[m][k] * W[n][k],   0 <= m < M, 0 <= n < N.
 * x: M rows of K elements, row stride ldx (elements); y: M rows of N
 * elements, row stride ldy.  M in 1..16.  bits in 1..8 with
 * n_entries <= 2^bits; any N, K >= 0 and block_size >= 1.  Indices >=
 * n_entries (never produced by the packers) read the last entry.
 *
 * Replaces: dequant_matvec_3bit(x, packed, codebook, N, K)
 *           (inference/cuda_kernel.py:84-104, 133-136),
 *           dequant_matvec_3bit(x, packed_indices, codebook, N, K)
 *           (inference/triton_kernel.py:186-196),
 *           dequant_matvec(x, indices, codebook, N, K) with bits = 8
 *           (inference/triton_kernel.py:119-140),
 *           and PackedLinear.forward for x_flat.shape[0] <= 16
 *           (inference/triton_kernel.py:240-275).
 */
int nb_gemv(const void* x, int x_dtype, int64_t ldx,
            const uint8_t* packed, const float* codebook,
            void* y, int y_dtype, int64_t ldy,
            int M, int N, int K, int bits, int n_entries, int block_size,
            void* stream);

/*
 * Prefill / batched contraction with a packed weight:
 *     y[m][n] = sum_k x[m][k] * bf16(W[n][k]),  0 <= m < M, 0 <= n < N,
 * W a 3-bit stream with 8-entry fp32 codebooks per block of 128 (entries
 * rounded to bf16 as the reference's bf16 path), x bf16 with row stride ldx
 * (ldx % 8 == 0, x 16-byte aligned), y NB_BF16 or NB_F32 with row stride
 * ldy, fp32 accumulation.  Any M, N >= 1; K % 128 == 0.
 * Replaces: the batched branch of PackedLinear.forward (unpack + gather +
 *           x @ W.T, inference/triton_kernel.py:258-275) in its bf16 form
 *           (inference/eval_ppl.py:149-174, compare.py:265-288), and the
 *           TPU prefill kernel (nativebit_jax/packed_kernel.py:108-178).
 */
int nb_gemm_prefill(const void* x, int64_t ldx, const uint8_t* packed, const float* codebook,
                    void* y, int y_dtype, int64_t ldy, int M, int N, int K, void* stream);

/*
 * nb_gemm_prefill with a caller workspace for a K split: where the tile
 * grid of one launch would leave CUs idle (few tokens or a narrow layer:
 * every workgroup would walk all of K with little work per step), the
 * kernel runs over up to 8 K ranges per tile and writes fp32 partial
 * products [S][M][N] to the workspace, and a second launch adds them in
 * range order and writes y.  The workspace needs
 * nb_gemm_prefill_split_ws_bytes(M, N, K) bytes (0 where the shape is not
 * split; then `workspace` may be NULL), 256-byte aligned, contents
 * clobbered; a smaller ws_bytes is NB_EINVAL.  Same operands and result
 * contract as nb_gemm_prefill; results are deterministic and differ from
 * nb_gemm_prefill's only by fp32 summation order where a split is used.
 * Replaces: the same batched branch of PackedLinear.forward in its bf16
 *           form (inference/triton_kernel.py:258-275, inference/eval_ppl.py:
 *           149-174); the workspace follows the caller-allocates convention
 *           of the rest of this interface.
 */
int64_t nb_gemm_prefill_split_ws_bytes(int M, int N, int K);
int nb_gemm_prefill_split(const void* x, int64_t ldx, const uint8_t* packed,
                          const float* codebook, void* y, int y_dtype, int64_t ldy, int M, int N,
                          int K, void* workspace, int64_t ws_bytes, void* stream);

/*
 * The same contraction for fp32 activations against the exact fp32 codebook
 * values, y[m][n] = sum_k x[m][k] * W[n][k] (x fp32 row stride ldx, y fp32
 * row stride ldy, any alignment of their element type; K % 128 == 0), on
 * the bf16 MFMA kernel in three passes: x = hi + lo and W = W_hi + W_lo
 * split into bf16 parts (hi = bf16(v), lo = bf16(v - hi); W_lo through the
 * residual codebook cb - bf16(cb) over the same indices), y = hi.W_hi +
 * hi.W_lo + lo.W_hi accumulated in fp32 in that order.  Each product is x.W
 * to within 2^-16 of its size (the dropped lo.W_lo and the bf16 roundings
 * of the lo parts), against 2^-24 for an fp32 product; W is never
 * materialised.  The workspace needs nb_gemm_prefill_f32_ws_bytes(M, N, K)
 * bytes, 256-byte aligned (the bf16 parts of x, the residual codebook, the
 * K-split partial products), contents clobbered.  Deterministic.
 * Replaces: the batched branch of PackedLinear.forward for fp32 x
 *           (unpack + gather + x @ W.T, inference/triton_kernel.py:258-275;
 *           nativebit/inference.py:42-46), without the per-call W.
 */
int64_t nb_gemm_prefill_f32_ws_bytes(int M, int N, int K);
int nb_gemm_prefill_f32(const float* x, int64_t ldx, const uint8_t* packed,
                        const float* codebook, float* y, int64_t ldy, int M, int N, int K,
                        void* workspace, int64_t ws_bytes, void* stream);

/*
 * Unpack `count` indices of `bits` bits to one byte each.
 * Replaces: unpack_3bit / unpack_4bit / unpack_nbits
 *           (nativebit/pack.py:44-68, 85-90, 119-138) and
 *           unpack_indices_3bit (inference/generate_torch.py:165-173).
 */
int nb_unpack(const uint8_t* packed, uint8_t* idx_out, int64_t count, int bits,
              void* stream);

/*
 * Pack `count` one-byte indices (low `bits` bits used) into the stream,
 * writing exactly nb_packed_nbytes(count, bits) bytes (padding zero).
 * Replaces: pack_indices_to_3bit (inference/triton_kernel.py:199-220),
 *           pack_3bit / pack_4bit / pack_nbits (nativebit/pack.py:21-116),
 *           pack_indices_3bit (inference/pack.py:38-57).
 */
int nb_pack(const uint8_t* idx, uint8_t* packed_out, int64_t count, int bits,
            void* stream);

/* Per-block quantile codebooks (the codebook init of a packed layer):
 * codebook_out[b][e] = quantile(w[b*block_size .. min((b+1)*block_size,
 * total)), q_e), q = linspace(0, 1, n_entries), linear interpolation -- as
 * torch.quantile in init_codebook_percentile (nativebit/codebook_utils.py:
 * 6-22), called per block by NativeBitLinear (nativebit/layers.py:76); the
 * last block takes only the weights that exist.  ceil(total / block_size)
 * x n_entries fp32 outputs; block_size <= 1024, n_entries <= 256; inputs
 * finite. */
int nb_block_codebooks(const float* w, int64_t total, int block_size, int n_entries,
                       float* codebook_out, void* stream);

/* The n (1..256) fractions nb_block_codebooks uses: torch.linspace(0, 1, n)
 * in fp32 (host only, for callers and tests). */
int nb_linspace01(int n, float* out);

/* Quantize-at-pack: the nearest codebook entry of each of the `total`
 * flat fp32 weights w, by squared distance in fp32 with the first entry on
 * ties, written straight into the LSB-first stream at `bits` per index
 * (nb_packed_nbytes(num_blocks * block_size, bits) bytes, as nb_pack).
 * codebook is num_blocks x n_entries fp32; the last block's padding
 * (weights total .. num_blocks * block_size - 1) counts as 0.0, and
 * block_size must be ceil(total / num_blocks).  Replaces quantize_weight
 * (inference/pack.py:21-35) + pack_indices_3bit (38-57) without the
 * reference's (blocks x block_size x entries) distance tensor.  Inputs are
 * finite. */
int nb_quantize_pack(const float* w, int64_t total, const float* codebook, int64_t num_blocks,
                     int n_entries, int block_size, int bits, uint8_t* packed_out, void* stream);

/*
 * Dequantize the first `total` weights: w[i] = codebook[i / block_size][index
 * i], written as float32 (exact copy) or bfloat16 (round to nearest even, as
 * torch's .to(torch.bfloat16)).  num_blocks * block_size must be >= total.
 * Replaces: reconstruct_weight (nativebit/pack.py:145-169) and the gather of
 *           PackedLinear's batched branch (inference/triton_kernel.py:260-273),
 *           NativeBitInferenceLinear.forward (nativebit/inference.py:42-46).
 */
int nb_dequant(const uint8_t* packed, const float* codebook, void* w_out,
               int w_dtype, int64_t total, int64_t num_blocks, int bits,
               int n_entries, int block_size, void* stream);

/*
 * Batched GEMV: many independent 3-bit / 8-entry / block-128 GEMVs
 * (bf16 x of one row, M = 1) streamed by one persistent launch.
 *
 * No counterpart in the reference, whose operator runs one layer per call
 * (inference/triton_kernel.py:240-257).  It serves callers that hold several
 * packed layers with their activations ready at once -- the projections of
 * one decode step that share no dependency, or a sweep over all layers -- so
 * that the per-launch cost (about 1.6 us on MI355X) and the ramp of each
 * small launch are paid once.  Each item is exactly nb_gemv(x, NB_BF16, ...,
 * M = 1) of that item.
 *
 * Usage: nb_gemv_batch_plan() validates the items and writes a device-ready
 * table into caller host memory; the caller copies that table to device
 * memory once and passes it to nb_gemv_batched() (with the same items) on
 * every call.  x, packed and codebook of every item must be 16-byte aligned
 * and K % 128 == 0, K <= 8192.
 *
 * Fused activation and output forms (for the layers of a decode step, so
 * that the norm, the SwiGLU product and the residual add need no launches
 * of their own).  x_mode says how the item's K bf16 activations a[k] are
 * formed from x; every workgroup forms them itself, in fp32, rounded to
 * bf16 (nearest even) once:
 *   NB_X_BF16      a = x, K bf16 values (the plain batched GEMV);
 *   NB_X_RMSNORM   x is K fp32 values, a[k] = (x[k] / sqrt(mean(x^2) + eps))
 *                  * norm_w[k]  (RMSNorm.forward, inference/generate_torch.py:
 *                  29-38, whose output feeds q|k|v and gate|up, 126-131);
 *   NB_X_SILU_MUL  x is 2K fp32 values gate | up, a[k] = silu(x[k]) * x[K+k]
 *                  (SwiGLU, inference/generate_torch.py:116-117).
 * y_mode: NB_Y_STORE writes y = result; NB_Y_ADD updates y[n] += result in
 * fp32 (y_dtype NB_F32 only; the residual adds of TransformerBlock.forward,
 * inference/generate_torch.py:128-132); NB_Y_SILU_PAIRS takes the rows as
 * (gate, up) pairs -- row 2i a gate row, row 2i+1 the up row of the same
 * output -- and writes N/2 bf16 values y[i] = silu(r[2i]) * r[2i+1] from
 * the fp32 row results r (SwiGLU's product, generate_torch.py:116-117, fed
 * to the down projection; y_dtype NB_BF16, N even, the item alone in its
 * batch).  The y of an NB_Y_ADD item must not overlap any x or norm_w of
 * the same batch.  Zero-filled new fields select the plain GEMV.
 */
enum nb_x_mode { NB_X_BF16 = 0, NB_X_RMSNORM = 1, NB_X_SILU_MUL = 2 };
enum nb_y_mode { NB_Y_STORE = 0, NB_Y_ADD = 1, NB_Y_SILU_PAIRS = 2 };
typedef struct nb_batch_item {
    const void* x;          /* activations, see x_mode                     */
    const uint8_t* packed;  /* 3-bit stream of N*K indices                 */
    const float* codebook;  /* (N*K/128) x 8 fp32                          */
    void* y;                /* N outputs of y_dtype                        */
    int32_t N;
    int32_t K;
    int32_t x_mode;         /* nb_x_mode                                   */
    int32_t y_mode;         /* nb_y_mode                                   */
    const float* norm_w;    /* NB_X_RMSNORM: K fp32 weights (else unused)  */
    float eps;              /* NB_X_RMSNORM: epsilon                       */
    int32_t reserved;       /* zero                                        */
} nb_batch_item;

/* Bytes of the device table for `count` items. */
int64_t nb_gemv_batch_table_bytes(int count);

/* Validates items and writes the table (nb_gemv_batch_table_bytes(count)
 * bytes) into table_host. */
int nb_gemv_batch_plan(const nb_batch_item* items, int count, void* table_host,
                       int64_t table_bytes);

/* Runs the batch: table_dev is the device copy of nb_gemv_batch_plan's
 * output for the same items. */
int nb_gemv_batched(const nb_batch_item* items, const void* table_dev, int count,
                    int y_dtype, void* stream);

/* The selector-ordered unit layout of a 3-bit stream: the same bytes, each
 * 12-byte unit of 32 indices rewritten so that the batched kernels take
 * its eight four-index selectors with one shift and one mask each (17 VALU
 * ops per 32 indices instead of 25).  With o = (0, 1, 3, 4, 6, 7, 2, 5),
 * byte k (0..3) of the unit's dword 0 holds index o(0)+8k in bits 0-2,
 * o(1)+8k in bits 3-5 and the low two bits of o(6)+8k in bits 6-7;
 * dword 1 likewise o(2)+8k, o(3)+8k and the low bits of o(7)+8k; dword 2
 * o(4)+8k, o(5)+8k, the high bit of o(6)+8k (bit 6) and of o(7)+8k
 * (bit 7).  Writes the N*K*3/8 bytes of `out` (out == packed allowed);
 * K a multiple of 128, both pointers 4-byte aligned.  The codebook is
 * unchanged.
 * No counterpart in the reference: a one-time re-ordering of a layer's
 * stream (for instance at model load) for nb_gemv_batched_sel. */
int nb_stream_layout(const uint8_t* packed, uint8_t* out, int N, int K, void* stream);

/* nb_gemv_batched on streams in the selector-ordered unit layout: every
 * item's packed is nb_stream_layout's output for that item's N x K, all
 * else as for nb_gemv_batched (same table, same fused forms).  The same
 * products, bit for bit, with less dequantization work per weight.
 * Replaces the same reference paths as nb_gemv_batched
 * (inference/cuda_kernel.py:38-104, inference/triton_kernel.py:143-196,
 * bf16 form of inference/eval_ppl.py:149-174) for layers converted once. */
int nb_gemv_batched_sel(const nb_batch_item* items, const void* table_dev, int count,
                        int y_dtype, void* stream);

/* Batched skinny GEMM: the same batch with M (1..16) activation rows per
 * item -- the batched branch of PackedLinear.forward (inference/
 * triton_kernel.py:258-275) in its bf16 form (inference/eval_ppl.py:149-174)
 * for every packed layer of a small-batch decode step, in one launch:
 *   y[m][n] = sum_k x[m][k] * bf16(W[n][k])   (fp32 accumulation)
 * with x an M x K bf16 row-major matrix (row stride K) and y M x N
 * row-major (row stride N) of y_dtype.  Items are x_mode NB_X_BF16 with
 * y_mode NB_Y_STORE or NB_Y_ADD (fp32); table_dev as for nb_gemv_batched. */
int nb_gemm_skinny_batched(const nb_batch_item* items, const void* table_dev, int count,
                           int M, int y_dtype, void* stream);

/* Row-quad layout of a 3-bit / 8-entry / block-128 N x K layer: the same
 * 128-weight blocks (48 index bytes, 8 fp32 codebook entries each) with the
 * rows taken four at a time (N rounded up to a multiple of 4 with zero
 * blocks) and the four rows' blocks of one column block side by side:
 *     block 4 (q * K/128 + kb) + i  =  row 4q + i, column block kb,
 * each 12-byte unit of a block's indices in the selector-ordered unit
 * layout of nb_stream_layout.  qpacked holds nb_quad_layout_bytes(N, K) bytes, qcodebook
 * nb_quad_layout_bytes(N, K) * 2 / 3 bytes (ceil(N/4) * 4 * K/128 * 8
 * floats); both 16-byte aligned, as packed and codebook.
 * No counterpart in the reference: a one-time re-ordering of a layer's
 * packed bytes (for instance at model load) for nb_gemm_skinny_quad_batched.
 */
int64_t nb_quad_layout_bytes(int N, int K);
int nb_quad_layout(const uint8_t* packed, const float* codebook, int N, int K,
                   uint8_t* qpacked, float* qcodebook, void* stream);

/* nb_gemm_skinny_batched for M = 1..4 on layers in the row-quad layout:
 * every item's packed / codebook are nb_quad_layout's output for that
 * item's N x K (N the layer's own row count); x, y, y_mode and table_dev as
 * for nb_gemm_skinny_batched, K >= 2048.  Replaces the same reference
 * branch (inference/triton_kernel.py:258-275, bf16 form of inference/
 * eval_ppl.py:149-174) for the two to four token rows of a small-batch
 * decode step: one v_mfma_f32_4x4x4_16b_bf16 serves four rows and four
 * tokens, so the per-weight work is that of M = 1. */
int nb_gemm_skinny_quad_batched(const nb_batch_item* items, const void* table_dev, int count,
                                int M, int y_dtype, void* stream);

/* Tile layout of a 3-bit / 8-entry / block-128 N x K layer for the skinny
 * kernel: tiles of 16 rows x 4 column blocks (tile g * ceil(K/512) + s =
 * rows 16g .. 16g + 15, column blocks 4s .. 4s + 3; rows past N and blocks
 * past K/128 zero), each stored as 3072 index bytes in tpacked and 512
 * fp32 codebook entries in tcodebook, in the order the kernel's LDS slot
 * holds them: row r's 48-byte blocks b at block place
 * (b + ((r >> 1) & 3) + (r >> 3)) & 3 of its 192 bytes, its codebook
 * 16-byte pieces p at place (p + ((r & 6) | ((r ^ (r >> 3)) & 1))) & 7 of
 * its 128 bytes, and every 12-byte unit of 32 indices in the
 * selector-ordered unit layout of nb_stream_layout with selector s (s =
 * 0..7) holding indices 4s .. 4s + 3 (byte t: index 4s + t).  tpacked holds nb_tile_layout_bytes(N, K)
 * bytes, tcodebook nb_tile_layout_bytes(N, K) * 2 / 3 bytes; all four
 * pointers 16-byte aligned.
 * No counterpart in the reference: a one-time re-ordering of a layer (for
 * instance at model load) for nb_gemm_skinny_tile_batched. */
int64_t nb_tile_layout_bytes(int N, int K);
int nb_tile_layout(const uint8_t* packed, const float* codebook, int N, int K, uint8_t* tpacked,
                   float* tcodebook, void* stream);

/* nb_gemm_skinny_batched (M = 1..16) on layers in the tile layout: every
 * item's packed / codebook are nb_tile_layout's output for that item's
 * N x K; x, y, y_mode and table_dev as for nb_gemm_skinny_batched.  The
 * same products, bit for bit, with each wave's slice read by five
 * contiguous 1 KiB loads and less dequantization work per weight.
 * Replaces the same reference branch (inference/triton_kernel.py:258-275,
 * bf16 form of inference/eval_ppl.py:149-174) for the five to sixteen
 * token rows of a small-batch decode step. */
int nb_gemm_skinny_tile_batched(const nb_batch_item* items, const void* table_dev, int count,
                                int M, int y_dtype, void* stream);


/* ------------------------------------------------------------------------
 * Decode step (one token, batch 1) -- the non-GEMV kernels of the packed
 * decoder of inference/generate_torch.py, for callers that run the whole
 * step on the device (for instance captured once in a HIP graph).  The
 * current position and token live in device memory (nb_decode_state), so no
 * step needs a host round trip.  All functions enqueue on `stream`.
 * ------------------------------------------------------------------------ */
typedef struct nb_decode_state {
    uint64_t key;    /* argmax key of the step in progress (0 between steps) */
    int32_t pos;     /* position of the token being fed                     */
    int32_t token;   /* token being fed                                     */
    int32_t step;    /* index of the next entry of tokens_out               */
    uint32_t done;   /* workgroup counter of nb_lm_head_argmax (0 between)  */
} nb_decode_state;

/*
 * x (+)= y, then h = (x / sqrt(mean(x^2) + eps)) * w  (n elements; x, y, w
 * fp32, h NB_F32 or NB_BF16).  With emb != NULL the row emb[state->token]
 * (fp32, n wide) replaces x first (the embedding lookup); with y != NULL
 * (and emb == NULL) y is added to x first (the residual).  x is updated in
 * place.
 * Replaces: RMSNorm.forward (inference/generate_torch.py:29-38) with the
 *           residual adds of TransformerBlock.forward (128-132) and the
 *           embedding lookup of PackedGPT.forward (150).
 */
int nb_add_rmsnorm(float* x, const float* y, const float* emb, const nb_decode_state* state,
                   const float* w, void* h, int h_dtype, int n, float eps, void* stream);

/*
 * One token of causal self-attention for all heads at position state->pos:
 * RoPE of the query and key (pairs (2i, 2i+1), angle pos * theta^(-2i/D),
 * tables cos/sin of [ctx][D/2] fp32), append of the rotated key and the
 * value to the caches (fp32; keys transposed, [n_head][D][ctx], values
 * [n_head][ctx][D]), softmax(q k^T / sqrt(D)) over positions 0..pos,
 * output [n_head * D] (NB_F32 or NB_BF16).  ctx <= 1024, D <= 256.  A
 * position outside 0..ctx-1 leaves caches and output untouched.
 * qkv: [3 * n_head * D] fp32, q | k | v.  work: nb_attention_work_floats()
 * floats; done: n_head uint32 counters, zero before the first call (each
 * call leaves them zero).
 * Replaces: CausalAttention.forward for one token with a KV cache, minus
 *           the two projections (inference/generate_torch.py:48-60, 72-106).
 */
int nb_attention_step(const float* qkv, float* k_cache, float* v_cache, const float* cos_t,
                      const float* sin_t, const nb_decode_state* state, float* work,
                      uint32_t* done, void* out, int out_dtype, int n_head, int head_dim,
                      int ctx, void* stream);
int nb_attention_work_floats(int n_head);

/*
 * nb_attention_step without the workspace: the same kernel and the same
 * results, with the split partials and head counters in a static device
 * array of the library (nb_attention_static_scratch_bytes() bytes, about
 * 1 MiB, one copy on each GPU it runs on, held until the process ends) --
 * the call allocates nothing (no hipMalloc, no library allocation).
 * n_head <= 64; otherwise as nb_attention_step.  All calls on one GPU share
 * that GPU's array: calls that overlap in time on one GPU (several streams
 * or threads) race, and must be ordered by the caller.  The head counters
 * start at zero (cleared once per device by a small kernel on the first
 * call's stream) and every completed call leaves them at zero.
 * No counterpart in the reference (whose attention is torch code,
 * inference/generate_torch.py:72-106).  It is for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation.
 */
int nb_attention_step_static(const float* qkv, float* k_cache, float* v_cache,
                             const float* cos_t, const float* sin_t,
                             const nb_decode_state* state, void* out, int out_dtype,
                             int n_head, int head_dim, int ctx, void* stream);
int64_t nb_attention_static_scratch_bytes(void);

/*
 * act[i] = silu(gu[i]) * gu[n + i]  (gu fp32 gate | up, act NB_F32/NB_BF16).
 * Replaces: F.silu(gate(x)) * up(x) (inference/generate_torch.py:116-117).
 */
int nb_silu_mul(const float* gu, void* act, int act_dtype, int n, void* stream);

/*
 * Tied LM head with soft cap and greedy choice: l[v] = 30 tanh((h . emb[v])
 * / 30) for v < V (h bf16 [C], emb bf16 [V][C], C % 8 == 0); logits (if not
 * NULL) receives l; the first v with the largest l is written to
 * tokens_out[state->step] (when state->step < tokens_cap) and becomes
 * state->token -- unless
 * state->step < n_force, in which case force[state->step] becomes the next
 * token (teacher forcing, to feed a prompt) -- and state->pos and
 * state->step advance by one.  state->key and state->done must be zero
 * before the call (every call leaves them zero).
 * Replaces: the head and argmax of PackedGPT.forward / benchmark
 *           (inference/generate_torch.py:157-159, 311).
 */
int nb_lm_head_argmax(const void* h, const void* emb, float* logits, nb_decode_state* state,
                      int32_t* tokens_out, int tokens_cap, const int32_t* force, int n_force,
                      int V, int C, void* stream);

/*
 * The final RMSNorm and nb_lm_head_argmax in one launch: h = bf16((x /
 * sqrt(mean(x^2) + eps)) * norm_w) of the fp32 residual x [C] (norm_w fp32
 * [C]), then the tied head, soft cap and greedy choice exactly as
 * nb_lm_head_argmax on that h.  Every workgroup forms h itself with
 * nb_add_rmsnorm's arithmetic, so the logits are bit for bit those of
 * nb_add_rmsnorm (x unchanged, y and emb NULL) followed by
 * nb_lm_head_argmax.  Same state, tokens and forcing contract.
 * Replaces: the final norm, head and argmax of PackedGPT.forward / benchmark
 *           (inference/generate_torch.py:29-38, 157-159, 311).
 */
int nb_rmsnorm_lm_head_argmax(const float* x, const float* norm_w, float eps, const void* emb,
                              float* logits, nb_decode_state* state, int32_t* tokens_out,
                              int tokens_cap, const int32_t* force, int n_force, int V, int C,
                              void* stream);

/* ------------------------------------------------------------------------
 * Batched forward pass over T tokens (a prompt fed as one sequence, as
 * PackedGPT.forward does with T > 1, inference/generate_torch.py:299-302):
 * the non-matmul kernels; the packed matmuls are nb_gemm_prefill.  Rows are
 * contiguous (row stride = width).  The caches are those of the decode
 * step (keys [n_head][head_dim][ctx], values [n_head][ctx][head_dim], fp32).
 * ------------------------------------------------------------------------ */
/*
 * Per row t < T: with emb (vocab rows of C) and tokens, x[t] =
 * emb[tokens[t]] (the embedding lookup); with add, x[t] += add[t] (a
 * residual add); then h[t] = (x[t] / sqrt(mean(x[t]^2) + eps)) * w (C wide;
 * x, add, emb, w fp32; h NB_F32 or NB_BF16).  x is updated in place.  A
 * token outside [0, vocab) reads no memory: its rows of x and h are set to
 * NaN (the reference's lookup raises; a kernel cannot).  vocab is ignored
 * without emb.
 * Replaces: RMSNorm.forward over a sequence (inference/generate_torch.py:
 *           29-38) with the residual adds of TransformerBlock.forward
 *           (128-132) and the embedding lookup of PackedGPT.forward (150).
 */
int nb_rmsnorm_rows(float* x, const float* add, const float* emb, const int32_t* tokens,
                    int vocab, const float* w, void* h, int h_dtype, int T, int C, float eps,
                    void* stream);
/*
 * act[t][i] = silu(gu[t][2i]) * gu[t][2i+1] for i < F (gu: T rows of 2F fp32,
 * gate and up interleaved by column, as a gate|up layer with alternating
 * rows produces them; act NB_F32 or NB_BF16).
 * Replaces: F.silu(gate(x)) * up(x) over a sequence (generate_torch.py:116-117).
 */
int nb_silu_pairs_rows(const float* gu, void* act, int act_dtype, int T, int F, void* stream);
/*
 * For tokens t < T at positions pos0 + t: RoPE of the query and key heads of
 * qkv (T rows of 3 * n_head * head_dim fp32, q | k | v), the rotated keys
 * and the values appended to the caches, and q_out[t] = rotated q *
 * head_dim^-0.5 (T rows of n_head * head_dim fp32).  pos0 + T <= ctx,
 * head_dim even and <= 128.
 * Replaces: apply_rope and the cache writes of CausalAttention.forward
 *           (inference/generate_torch.py:48-60, 80-88) for T tokens.
 */
int nb_rope_kv_rows(const float* qkv, float* k_cache, float* v_cache, const float* cos_t,
                    const float* sin_t, int pos0, int T, float* q_out, int n_head, int head_dim,
                    int ctx, void* stream);
/*
 * out[t] = softmax(q[t] . k[0 .. pos0 + t]) . v[0 .. pos0 + t] for every
 * head (causal: query t sees cache positions up to its own, pos0 + t); q
 * as nb_rope_kv_rows writes it, out T rows of n_head * head_dim (NB_F32 or
 * NB_BF16).
 * Replaces: the masked attention of CausalAttention.forward with the cache
 *           (inference/generate_torch.py:89-98) for T > 1 queries.
 */
int nb_attention_rows(const float* q, const float* k_cache, const float* v_cache, int pos0, int T,
                      void* out, int out_dtype, int n_head, int head_dim, int ctx, void* stream);

/* ------------------------------------------------------------------------
 * Persistent decode: many greedy tokens of the whole packed decoder in one
 * cooperative launch (one workgroup per CU), the phases of a token separated
 * by grid barriers instead of kernel boundaries, and the packed weights of
 * the next phases streamed while a phase waits.
 * ------------------------------------------------------------------------ */
/* The packed matmuls, norms and caches of one decoder layer (device
 * pointers).  Streams are 3-bit with 8-entry fp32 codebooks per block of 128
 * (the format above), 16-byte aligned.  q|k|v and gate|up are fused by rows:
 * qkv is the q, k and v weights stacked (3C x C, the reference's fused qkv,
 * inference/generate_torch.py:68), gu the gate then the up weights (2F x C). */
typedef struct nb_decode_layer {
    const uint8_t* qkv_packed;   const float* qkv_codebook;   /* 3C x C          */
    const uint8_t* o_packed;     const float* o_codebook;     /* C x C           */
    const uint8_t* gu_packed;    const float* gu_codebook;    /* 2F x C          */
    const uint8_t* down_packed;  const float* down_codebook;  /* C x F           */
    const float* ln1;            const float* ln2;            /* C fp32 each     */
    float* k_cache;                                           /* [H][D][ctx] fp32 */
    float* v_cache;                                           /* [H][ctx][D] fp32 */
} nb_decode_layer;
typedef struct nb_decode_model {
    int32_t n_layers, n_embd, n_head, head_dim, ffn_hidden, vocab, ctx;
    float eps;                       /* RMSNorm epsilon                        */
    const nb_decode_layer* layers;   /* device array of n_layers entries       */
    const float* ln_f;               /* final norm weight, n_embd fp32         */
    const float* emb_f32;            /* [vocab][n_embd] fp32 (token lookup)    */
    const void* emb_bf16;            /* [vocab][n_embd] bf16 (tied head)       */
    const float* rope_cos;           /* [ctx][head_dim / 2] fp32               */
    const float* rope_sin;
} nb_decode_model;
/* Byte offset, inside the workspace, of a uint32 that is 0 after a call that
 * completed and 1 after one whose grid barrier wait ran past the spin limit
 * (its outputs are then invalid). */
#define NB_DECODE_ERR_OFFSET 2304
/* Workspace bytes nb_decode_persistent needs for this model (0 if the
 * shapes are outside its limits; nb_last_error says why). */
int64_t nb_decode_workspace_bytes(const nb_decode_model* model);
/*
 * Feeds state->token at state->pos and runs n_steps greedy steps -- the same
 * model and the same state updates as n_steps of nb_add_rmsnorm ...
 * nb_lm_head_argmax per layer (forced tokens, tokens_out, pos and step
 * advance) -- in one launch.  logits (may be NULL) receives the last step's
 * capped logits.  The workspace (256-byte aligned, caller-owned device
 * memory) holds activations and barrier counters; the call clears its
 * control block.  Limits: n_embd and ffn_hidden multiples of 128, n_embd <=
 * 4096, ffn_hidden <= 8192, head_dim even and <= 128, ctx <= 1024, and
 * every layer large enough to give each CU a chunk of rows.  state->pos +
 * n_steps must not exceed ctx.  spin_limit bounds each grid barrier wait
 * (polls of about 100 ns; <= 0 selects 2^20).
 * Replaces: the token loop of PackedGPT generation (inference/
 *           generate_torch.py:135-162, 298-313) with its packed linears
 *           (inference/triton_kernel.py:223-286).
 */
int nb_decode_persistent(const nb_decode_model* model, void* workspace, int64_t workspace_bytes,
                         nb_decode_state* state, float* logits, int32_t* tokens_out,
                         int tokens_cap, const int32_t* force, int n_force, int n_steps,
                         int spin_limit, void* stream);
#ifdef __cplusplus
}
#endif
#endif /* NATIVEBIT_AMD_H */
