/*
 * inferno_hip — C ABI of the MI355X (gfx950) speculative-verify hot path.
 *
 * Plain pointers, sizes and an opaque stream handle (a hipStream_t passed as
 * void*; NULL = the default stream). No exceptions cross this ABI: the
 * ihip_* functions return IHIP_OK (0) or a negative status, and
 * ihip_last_error() gives a message for the calling thread.
 *
 * Citations are to the reference (Inferno.jl) interface each entry point
 * replaces, relative to its repository root.
 */
#ifndef INFERNO_HIP_H
#define INFERNO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---- */
#define IHIP_OK       0
#define IHIP_EFAULT (-14)   /* NULL pointer argument */
#define IHIP_EINVAL (-22)   /* bad shape / type / flag */
#define IHIP_ENOMEM (-12)   /* workspace too small or allocation failed */
#define IHIP_ENODEV (-19)   /* no usable gfx950 device */
#define IHIP_EHIP  (-1000)  /* HIP runtime error; see ihip_last_error() */

/* ---- GGML quant type ids (src/GGUF.jl:25-60) ---- */
#define IHIP_Q8_0 8
#define IHIP_Q4_K 12
#define IHIP_Q5_K 13
#define IHIP_Q6_K 14

/* ---- ihip_gemm_q flags ---- */
#define IHIP_GEMM_AUTO   0  /* fp32-accurate for M < 16, half MFMA for M >= 16 */
#define IHIP_GEMM_F32    1  /* force fp32-accurate: split-fp16 MFMA, rel-L2 <= 1e-5 */
#define IHIP_GEMM_HALF   2  /* force single-limb fp16 MFMA, rel-L2 <= 1e-2 */
#define IHIP_GEMM_ACCUM  4  /* y += W x (y is not cleared first) */
#define IHIP_GEMM_PACKED 8  /* w_dev is in the packed layout of ihip_pack_weights */
#define IHIP_GEMM_REUSE 16  /* ihip_gemm_q_ex: the activations prepared in ws by the
                               previous call (same x, act, M, K, flags) are reused */

/* ---- ihip_gemm_q_ex input transforms ---- */
#define IHIP_ACT_PLAIN    0  /* x */
#define IHIP_ACT_RMSNORM  1  /* RMSNorm(x) * norm_w (src/ModelCPU.jl:110-122) */
#define IHIP_ACT_SILU_MUL 2  /* silu(x[:, :K]) * x[:, K:2K] (src/ModelCPU.jl:447-473) */

/* Message for the last failing call on this thread ("" if none). */
const char *ihip_last_error(void);

/* Select the device and create the library stream used by the host-pointer
 * drop-in entry points; also looks up `device`'s fixed scratch of
 * ihip_gemm_q_noalloc. Called implicitly by the first drop-in call.
 * Replaces the library probe of QuantizedKernels._load_libquant
 * (src/QuantizedKernels.jl:34-47). */
int ihip_init(int device);

/* 1 if the library initialised on a gfx950 device and was not disabled by
 * INFERNO_NO_QUANT_KERNELS; replaces quant_kernels_available()
 * (src/QuantizedKernels.jl:49-50). */
int ihip_available(void);

/* ======================================================================
 * 1. Drop-in exports: same symbol names and argument order as the
 *    reference C kernel (src/kernels/quant_kernels.c:602-697), bound by
 *    QuantizedKernels.q{4,5,6}_k_gemv! / q8_0_gemv!
 *    (src/QuantizedKernels.jl:82-146).
 *    Host pointers; synchronous. weight is GGUF row-major blocks, row r
 *    owning blocks [r*K/QK, (r+1)*K/QK). The device copy of each weight is
 *    cached by (host pointer, byte size, type, outer_dim, inner_dim) with a
 *    fingerprint of sampled bytes (first, middle, last 256) checked on each
 *    call, so a host buffer freed and reused at the same address with other
 *    contents is uploaded again; weights are otherwise taken as immutable
 *    after their first use (ihip_weight_cache_clear() drops the cache).
 *    Cached bytes stay under INFERNO_HIP_WEIGHT_CACHE_BYTES (default 3/4 of
 *    device memory), least recently used evicted first. q8_buf is accepted
 *    and ignored (NULL allowed): the GPU path needs no Q8_K scratch.
 *    out[r] = sum_k W[r,k] x[k] computed fp32-accurately. On error out[0 ..
 *    outer_dim) is filled with NaN (these entry points return void like the
 *    reference's, so the failure shows downstream), the status is kept for
 *    ihip_last_error() and ihip_last_status(), and a message is printed to
 *    stderr.
 * ====================================================================== */
void q4_k_gemv(const uint8_t *weight, const float *x, float *out, void *q8_buf,
               int inner_dim, int outer_dim);
void q5_k_gemv(const uint8_t *weight, const float *x, float *out, void *q8_buf,
               int inner_dim, int outer_dim);
void q6_k_gemv(const uint8_t *weight, const float *x, float *out, void *q8_buf,
               int inner_dim, int outer_dim);
void q8_0_gemv(const uint8_t *weight, const float *x, float *out,
               int inner_dim, int outer_dim);

/* The remaining exports of the reference library, computed on the GPU with
 * the same host-pointer, synchronous convention (the matmul path does not use
 * them; they let this library stand in for libquant_kernels.so symbol for
 * symbol). Results equal the reference's bit for bit.
 *   quantize_row_q8_K: k fp32 values (k a multiple of 256) to k/256
 *     block_q8_K (float d = amax/127; int8 qs[256] = round(x/d) half away
 *     from zero; int16 bsums[16] of 16 values each): 292 bytes per block
 *     (src/kernels/quant_kernels.c:166-194). Bound by quantize_q8_k!
 *     (src/QuantizedKernels.jl:149-154), whose ccall passes (q8_buf, x, k) in
 *     the wrong order and width for this C signature, as it does for the
 *     reference's own library. On error every block's d is set to NaN.
 *   vec_dot_q{4,5,6}_K_q8_K: one row of nb K-quant blocks x nb block_q8_K
 *     (src/kernels/quant_kernels.c:204-521; vec_dot_q*_k_q8_k,
 *     src/QuantizedKernels.jl:157-175). NaN on error. */
void  quantize_row_q8_K(const float *x, void *y, int64_t k);
float vec_dot_q4_K_q8_K(const void *x, const void *y, int nb);
float vec_dot_q5_K_q8_K(const void *x, const void *y, int nb);
float vec_dot_q6_K_q8_K(const void *x, const void *y, int nb);

/* Status of the last drop-in call on this thread (IHIP_OK or negative). */
int ihip_last_status(void);
/* Drop every cached device weight copy. */
void ihip_weight_cache_clear(void);

/* ======================================================================
 * 2. Device-pointer API (status-returning, explicit stream).
 * ====================================================================== */

/* Y[M x N] (row-major, token-major) = X[M x K] * W^T for GGUF weight W
 * [N rows x K] resident on the device. M in 1..64; K a multiple of the
 * block size (256 for K-quants, 32 for Q8_0); x, w and ws 16-byte aligned.
 * ws: caller-owned device workspace of at least ihip_gemm_q_ws_bytes()
 * bytes, holding the prepared activations and the split-K
 * partials; calls that overlap in time need separate workspaces. The result
 * is deterministic (no floating-point atomics).
 * Batched form of q*_gemv (src/kernels/quant_kernels.c:602-697) over the
 * M verify tokens that forward_cpu! streams one at a time
 * (src/ModelCPU.jl:970-980). */
int ihip_gemm_q_ws_bytes(int qtype, int M, int N, int K, int flags,
                         size_t *bytes);
int ihip_gemm_q(int qtype, const void *w_dev, const float *x_dev, float *y_dev,
                int M, int N, int K, int flags, void *ws, size_t ws_bytes,
                void *stream);

/* ihip_gemm_q without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). No counterpart in the reference. The workspace is
 * a fixed 64 MiB device array of the library (one per GPU, held from module
 * load to process exit); shapes whose ihip_gemm_q_ws_bytes exceed it are
 * rejected with IHIP_ENOMEM (e.g. the 151936-row LM head at M = 64). The
 * call allocates nothing. All calls on one GPU share its array: calls that
 * overlap in time on one GPU (other streams, other threads) race, so
 * serialize them. The kernels write every scratch byte they read, so the
 * previous call's contents need no clearing. Same results, bit for bit, as
 * ihip_gemm_q with the same arguments. The array's device address is looked
 * up by ihip_init(device) (else on the first call on a device): call
 * ihip_init on each device before capturing this entry point. */
int ihip_gemm_q_noalloc(int qtype, const void *w_dev, const float *x_dev,
                        float *y_dev, int M, int N, int K, int flags,
                        void *stream);

/* ihip_gemm_q with the producer of its input fused in: Y = f(X') W^T.
 *   X' = x, or, with add != NULL, x + (add[0] + add[1] + ... + add[n_add-1])
 *        (slices [M x K], row stride K, slice stride add_stride floats, e.g.
 *        the K-slice partials an IHIP_GEMM_DEFER call left in its
 *        workspace), stored back into x: the residual add of the decoder
 *        layer (src/ModelCPU.jl:870-891) folded into the next matmul.
 *   f  = IHIP_ACT_PLAIN, IHIP_ACT_RMSNORM (per row: x / sqrt(mean(x^2) +
 *        eps) * norm_w, norm_w may be NULL for unit weight; the RMSNorm of
 *        src/ModelCPU.jl:110-122 before the projections of :755-760 and
 *        :455-471, applied as a row scale of the product) or
 *        IHIP_ACT_SILU_MUL (x rows are [gate | up], 2K wide).
 * ldx: floats between rows of x (>= K, or >= 2K for SILU_MUL; a multiple of
 * 4). IHIP_GEMM_REUSE skips the input stage when ws already holds the
 * prepared f(X') of the previous call (e.g. two projections of one hidden
 * state); not with add, nor with fp32-accurate M > 32. IHIP_GEMM_DEFER
 * leaves the product in ws as K-slice partials (ihip_gemm_q_partials) and
 * does not touch y; not with IHIP_GEMM_ACCUM, nor with fp32-accurate M > 32.
 * Same workspace size as ihip_gemm_q; a deferring call and the call that
 * adds its partials need separate workspaces. IHIP_GEMM_SUM_OUT (with add
 * and x, act PLAIN or RMSNORM, K a multiple of 256, ldx of 8): the input is
 * the sum of the [M x ldx] add slices, which the input stage also stores
 * into x (all ldx columns; x is written, not read), so a deferred product
 * wider than this call's K (e.g. [q; k; v] feeding o from its q columns) is
 * materialised without a reduce launch of its own. No counterpart in the
 * reference (its products are never K-split). */
#define IHIP_GEMM_DEFER 32
#define IHIP_GEMM_SUM_OUT 64
typedef struct ihip_gemm_input {
    const float *x;        /* activations (written back when add != NULL), or
                              NULL when the add slices are the input */
    int ldx;
    int act;               /* IHIP_ACT_* */
    const float *norm_w;   /* RMSNorm weight [K] or NULL */
    float eps;
    const float *add;      /* NULL or n_add slices: with x, [M x K] slices
                              folded into x first (x += sum, stored back);
                              without x, [M x ldx] slices whose sum is the
                              input (e.g. the deferred [gate | up] product
                              feeding IHIP_ACT_SILU_MUL). Summed in slice
                              order, as the reduce of a non-deferred call. */
    int n_add;
    int64_t add_stride;
} ihip_gemm_input;
int ihip_gemm_q_ex(int qtype, const void *w_dev, const ihip_gemm_input *in,
                   float *y_dev, int M, int N, int K, int flags, void *ws,
                   size_t ws_bytes, void *stream);
/* Partials of a deferred call with the same (qtype, M, N, K, flags): n
 * slices [M x N] at *slices, slice stride *stride floats. */
int ihip_gemm_q_partials(int qtype, int M, int N, int K, int flags, void *ws,
                         float **slices, int *n_slices, int64_t *stride);

/* ---- chained matmuls: one input stage per decoder layer instead of four ----
 * fp32-accurate calls on packed weights with one token tile (M <= 8) can hand
 * their output to the next matmul without its input stage. The producer's
 * epilogue (ihip_chain_out) stores the fp32 result y and writes the next
 * matmul's split-fp16 operand of v = y w (w: the next input's RMSNorm weight,
 * or 1) in the consumer's layout (consumer_qtype), each 16-row output tile
 * (8 channels for IHIP_EPI_GATE) scaled by its own power of two (its largest
 * |v| in [2^14, 2^15)) and tagged with that exponent; beside it the tile's sum
 * of v (min terms of Q4_K/Q5_K consumers) and, for an RMSNorm that follows,
 * the tile's sum of y^2. The consumer (ihip_chain_in) loads that operand as a
 * classic call loads its prepared one and rescales it to the power of two of
 * each 256-element unit (the input stage's), exactly wherever the result
 * stays a normal fp16; it applies the RMSNorm row scale 1 / sqrt(sum ssq / K
 * + eps) to its result. The layer arithmetic stays that of
 * src/ModelCPU.jl:110-122 (RMSNorm), :447-473 (SiLU gating) and :870-891
 * (residual adds).
 * Epilogues:
 *   IHIP_EPI_STORE: y = the product (no operand, no statistics);
 *   IHIP_EPI_STATS: y = the product; operand and statistics of rows
 *                   [0, stat_rows) (e.g. the q rows of [q; k; v], the input
 *                   of o);
 *   IHIP_EPI_RESID: y += the product (y: the residual), operand and
 *                   statistics of the sum (the input of the next RMSNorm'd
 *                   matmul);
 *   IHIP_EPI_GATE:  the weights were packed by ihip_pack_weights_gated (tiles
 *                   of 8 gate rows and their 8 up rows, N = 2F rows); y [M x
 *                   ldy] receives h = silu(gate) * up, F values per row, and
 *                   the operand and statistics are of h (tiles of 8
 *                   channels: the consumer's tiles_per_unit is 32).
 * Tile sums: tile_sum [8 tokens][sum_stride] (16-byte aligned, sum_stride a
 * multiple of 4 covering every tile), tile_ssq [tiles][8]. */
#define IHIP_EPI_STORE 0
#define IHIP_EPI_STATS 1
#define IHIP_EPI_RESID 2
#define IHIP_EPI_GATE  3
/* Bytes of a chained operand for a consumer with K inputs (K a multiple of
 * 256): limbs, then one exponent byte per lane entry, per 256-element unit. */
size_t ihip_chain_operand_bytes(int K);
typedef struct ihip_chain_in {
    const void *operand;     /* the producer's operand (ihip_chain_operand_bytes(K), 16-byte aligned) */
    const float *tile_sum;   /* the producer's tile sums [8][sum_stride]
                                (Q4_K/Q5_K consumers; may be NULL otherwise) */
    int sum_stride;
    int tiles_per_unit;      /* 16, or 32 after IHIP_EPI_GATE */
    const float *tile_ssq;   /* the producer's tile sums of squares [ssq_tiles][8]
                                (RMSNorm row scale), or NULL (none) */
    int ssq_tiles;
    float eps;
} ihip_chain_in;
typedef struct ihip_chain_out {
    int epi;                 /* IHIP_EPI_* */
    float *y;
    int ldy;                 /* floats between rows of y */
    const float *norm_w;     /* RMSNorm weight of the next input [width], or NULL */
    int consumer_qtype;      /* IHIP_Q4_K / Q5_K / Q6_K / Q8_0: the next matmul's */
    void *operand;           /* ihip_chain_operand_bytes(width) bytes, or NULL */
    float *tile_sum;         /* [8][sum_stride], or NULL (needed by Q4_K/Q5_K consumers) */
    int sum_stride;
    float *tile_ssq;         /* [tiles][8], or NULL */
    int stat_rows;           /* IHIP_EPI_STATS: rows [0, stat_rows), a multiple of 256 */
} ihip_chain_out;
/* Y = f(X) W^T for packed weights, fp32-accurate, M <= 8, one of in (the usual
 * input stage, e.g. RMSNorm with the previous layer's partials folded) or cin
 * (a chained producer's operand), and cout (NULL only with IHIP_GEMM_DEFER,
 * which leaves K-slice partials as ihip_gemm_q_ex does). flags: IHIP_GEMM_F32,
 * IHIP_GEMM_PACKED, IHIP_GEMM_DEFER. A matmul split over K (K above 8192 for
 * Q4_K, 4096 for Q5_K / Q6_K, 2048 for Q8_0: e.g. the down projection)
 * finishes each 16-row tile in the workgroup of the last K-slice to reach
 * it, which sums the slices in slice order and runs the epilogue: the
 * workspace then holds per-tile slice counts that must be zero before the
 * first such call (a zeroed workspace; the calls leave them zero). Shapes
 * off the one-tile streaming plan return IHIP_EINVAL. The width an operand
 * covers (N; N / 2 for IHIP_EPI_GATE; stat_rows for IHIP_EPI_STATS) must be
 * a multiple of 256. Workspace as ihip_gemm_q. */
int ihip_gemm_q_chain(int qtype, const void *w_packed, const ihip_gemm_input *in,
                      const ihip_chain_in *cin, const ihip_chain_out *cout,
                      int M, int N, int K, int flags, void *ws, size_t ws_bytes,
                      void *stream);
/* The [gate; up] GGUF matrix [2F x K] (gate rows, then up rows) packed into
 * tiles of 8 gate rows and their 8 up rows, for IHIP_EPI_GATE (F a multiple
 * of 8; ihip_packed_bytes(qtype, 2F, K) bytes). */
int ihip_pack_weights_gated(int qtype, const void *w_gguf_dev, void *w_packed_dev,
                            int F, int K, void *stream);

/* Packed weight layout: the GGUF blocks of each 16-row tile and 256-element
 * K-unit stored as one contiguous chunk, swizzled so that every lane of the
 * matmul kernel fetches its operand bytes with whole-cache-line 16-byte
 * loads (bytes and values unchanged, only moved; rows past N and Q8_0 blocks
 * past K are zero). ihip_packed_bytes gives the size (a multiple of 16);
 * ihip_pack_weights converts one [N x K] GGUF matrix on the device, once,
 * at model load: the reference reads GGUF tensors as-is
 * (src/LoaderCPU.jl:358-372, src/ModelCPU.jl:295-296), and packed matrices
 * are then passed to ihip_gemm_q with IHIP_GEMM_PACKED. */
int ihip_packed_bytes(int qtype, int N, int K, size_t *bytes);
int ihip_pack_weights(int qtype, const void *w_gguf_dev, void *w_packed_dev,
                      int N, int K, void *stream);

/* Bit-exact dequantization of n_elems weights (a multiple of the block
 * size) to fp32: the dequantize_*_block! formulas of
 * src/QuantsCPU.jl:491-658. */
int ihip_dequant(int qtype, const void *w_dev, float *out_dev, int64_t n_elems,
                 void *stream);

/* RMSNorm of rows x n fp32 values (src/ModelCPU.jl:110-122); w_dev may be
 * NULL (unit weight). In place allowed. */
int ihip_rmsnorm(const float *x_dev, const float *w_dev, float *out_dev,
                 int rows, int n, float eps, void *stream);

/* out[m, i] = silu(gu[m, i]) * gu[m, F + i] for M rows of [gate | up]
 * (the SiLU gating of mlp_forward, src/ModelCPU.jl:447-473). */
int ihip_silu_mul(const float *gu_dev, int M, int F, float *out_dev, void *stream);

/* y[i] += x[i], i < n (the residual adds of the decoder layer,
 * src/ModelCPU.jl:870-891). */
int ihip_add(float *y_dev, const float *x_dev, int64_t n, void *stream);

/* The MLP half of a decoder layer (DecoderLayerCPU, src/ModelCPU.jl:884-889,
 * with mlp_forward, src/ModelCPU.jl:447-473), in place on the residual:
 *   n = rmsnorm(x, norm_w, eps);  x += W_down (silu(W_gate n) * (W_up n))
 * x: [M x H] fp32 row-major. w_gate_up: the [gate; up] matrix, 2F rows x H
 * (the gate rows, then the up rows: concatenate the two GGUF tensors; with
 * IHIP_GEMM_PACKED pack the concatenation). w_down: [H x F]. flags:
 * IHIP_GEMM_F32 / IHIP_GEMM_HALF / IHIP_GEMM_PACKED (the precision and layout
 * of both matmuls). Workspace: ihip_mlp_ws_bytes (holds the [M x 2F] gate/up
 * product). Two input-stage + matmul launches on the stream; the same result
 * bit for bit as ihip_gemm_q_ex with IHIP_ACT_RMSNORM into a [M x 2F] buffer
 * followed by ihip_gemm_q_ex with IHIP_ACT_SILU_MUL and IHIP_GEMM_ACCUM. */
int ihip_mlp_ws_bytes(int qt_gate_up, int qt_down, int M, int H, int F,
                      int flags, size_t *bytes);
int ihip_mlp_forward(int qt_gate_up, const void *w_gate_up, int qt_down,
                     const void *w_down, float *x, const float *norm_w,
                     float eps, int M, int H, int F, int flags, void *ws,
                     size_t ws_bytes, void *stream);

/* ---- LM-head softmax statistics and speculative acceptance ---- */

/* Per row r of logits [rows x V]: zmax[r] = max_j L[r,j]/T and
 * zsum[r] = sum_j exp(L[r,j]/T - zmax[r]) (the softmax of
 * src/ModelCPU.jl:1130-1148 and src/SpeculativeDecoding.jl:79-80). */
int ihip_accept_ws_bytes(int rows, int V, size_t *bytes);
int ihip_softmax_stats(const float *logits_dev, int rows, int V, float T,
                       float *zmax_dev, float *zsum_dev, void *ws,
                       size_t ws_bytes, void *stream);

/* Rejection-sampling verify for `steps` independent verify steps
 * (speculate_and_verify, src/SpeculativeDecoding.jl:37-107, accept loop
 * :75-104). Per step s (all arrays device-resident, step-major):
 *   tgt  [(k+1) x V] target logits, drf [k x V] draft logits,
 *   draft_tok [k] 0-based draft ids, u_acc [k], u_res [1], u_bonus [1].
 * mode 0 = standard (p, q at temperature T; residual max(0, p - q)),
 * mode 1 = reference-compatible (T = 1 ratio with a scalar draft
 * probability and scalar residual, src/SpeculativeDecoding.jl:61-63,79-93).
 * out_tok [k+1] receives the accepted drafts followed by the resampled or
 * bonus token (out_n + 1 tokens); out_n [1] the number of accepted drafts
 * (0..k), or -1 for a draft id outside [0, V). Mode 1 also reproduces the
 * reference's bonus after a rejection of the last draft: when out_n ==
 * k - 1, out_tok[k] holds a bonus token drawn from target row k at T with
 * u_bonus (k + 1 tokens; src/SpeculativeDecoding.jl:100 appends it whenever
 * length(accepted) == gamma). T must be > 0 (use ihip_greedy_verify for
 * T = 0); V <= 4194304, k <= 127. ws: ihip_spec_accept_ws_bytes() bytes, 16-byte
 * aligned. */
int ihip_spec_accept_ws_bytes(int steps, int k, int V, size_t *bytes);
int ihip_spec_accept(const float *tgt_dev, const float *drf_dev,
                     const int32_t *draft_tok_dev, int steps, int k, int V,
                     float T, const float *u_acc_dev, const float *u_res_dev,
                     const float *u_bonus_dev, int mode, int32_t *out_tok_dev,
                     int32_t *out_n_dev, void *ws, size_t ws_bytes,
                     void *stream);

/* ihip_spec_accept with speculate_and_verify's top_k / top_p keywords
 * (src/SpeculativeDecoding.jl:44-45) and softmax_sample's min_p: every bonus
 * token (after an all-accept, and mode 1's after a rejection of the last
 * draft) is softmax_sample(target row k; T, top_p, top_k, min_p) with
 * u_bonus (src/SpeculativeDecoding.jl:100-104, src/ModelCPU.jl:1123-1200),
 * drawn by ihip_sample_ex's kernels. The ratio tests and the residual are
 * unchanged: the reference takes them from the unfiltered softmaxes at
 * T = 1 (mode 1); mode 0 uses the unfiltered softmaxes at T, so with
 * filtered drafting its q is not the distribution the drafts came from.
 * Filters that keep the whole vocabulary (top_k = 0 or >= V, top_p >= 1,
 * min_p <= 0) give ihip_spec_accept exactly. ws:
 * ihip_spec_accept_ex_ws_bytes() bytes (the
 * steps' bonus rows and the sampler's workspace on top of the accept's). */
int ihip_spec_accept_ex_ws_bytes(int steps, int k, int V, int top_k,
                                 float top_p, float min_p, size_t *bytes);
int ihip_spec_accept_ex(const float *tgt_dev, const float *drf_dev,
                        const int32_t *draft_tok_dev, int steps, int k, int V,
                        float T, int top_k, float top_p, float min_p,
                        const float *u_acc_dev, const float *u_res_dev,
                        const float *u_bonus_dev, int mode,
                        int32_t *out_tok_dev, int32_t *out_n_dev, void *ws,
                        size_t ws_bytes, void *stream);

/* Greedy verify (mtp_verify_step!, src/ModelCPU.jl:1914-1930): per step,
 * logits [(k+1) x V]; out_argmax [k+1] = first-index argmax of each row in
 * Julia's isless order (-0.0 below +0.0, NaN above every number, so the
 * first NaN wins; a row of -Inf gives index 0); out_n = leading i < k with
 * out_argmax[i] == draft_tok[i]. */
int ihip_greedy_verify(const float *logits_dev, const int32_t *draft_tok_dev,
                       int steps, int k, int V, int32_t *out_n_dev,
                       int32_t *out_argmax_dev, void *ws, size_t ws_bytes,
                       void *stream);

/* Tree accept walk over n draft-tree nodes (node 0 = root, parent[i] < i),
 * no counterpart in the reference (it has no tree speculation): node i is
 * accepted iff its parent is accepted and
 * u[i] < min(1, p_parent[tok[i]] / q_parent[tok[i]]), p and q the target and
 * draft softmax at T of the parent's rows. out_path [n] receives the root..
 * deepest accepted node (ties -> smallest node index); out_len [1] its
 * length, or -1 for a malformed node. ws: ihip_accept_ws_bytes(3 n, V)
 * bytes. */
int ihip_tree_accept(const float *tgt_dev, const float *drf_dev,
                     const int32_t *tok_dev, const int32_t *parent_dev, int n,
                     int V, float T, const float *u_dev, int32_t *out_path_dev,
                     int32_t *out_len_dev, void *ws, size_t ws_bytes,
                     void *stream);

/* ---- applying the outcome of a verify step (csrc/rollback.hip) ---- */

/* The reference keeps no rollback (src/SpeculativeDecoding.jl:69-70); these
 * read n = n_accepted_dev[s] (the out_n of ihip_spec_accept / greedy verify:
 * drafts accepted, -1 for an invalid draft) on the device, so a captured
 * verify step needs no host round trip. For each step s < steps:
 *   commit_state: state[s] = snapshot n of step s, the recurrent (SSM) state
 *   after the verify forward consumed positions 0..n; snapshot j of step s
 *   at snap_dev + s * snap_step_bytes + j * snap_stride_bytes, j = 0..k;
 *   state of step s at state_dev + s * state_step_bytes;
 *   advance_len: len[s] += n + 1 (the KV-cache entries that stand).
 * n = -1 or n > k leaves the step's state / length unchanged. Sizes, strides
 * and pointers are multiples of 4 bytes. */
int ihip_spec_commit_state(void *state_dev, const void *snap_dev, size_t bytes,
                           int64_t snap_stride_bytes, int k,
                           const int32_t *n_accepted_dev, int steps,
                           int64_t state_step_bytes, int64_t snap_step_bytes,
                           void *stream);
int ihip_spec_advance_len(int32_t *len_dev, const int32_t *n_accepted_dev,
                          int steps, void *stream);

/* ---- draft-side sampler (csrc/sample.hip) ---- */

/* softmax_sample (src/ModelCPU.jl:1123-1200) on each row of logits
 * [rows x V], one token per row (0-based) into out_tok_dev:
 *   T = 0: first-index argmax. Otherwise z = L / T; top_k > 0 keeps the
 *   top_k largest z (ties lowest index first; top_k >= V keeps all);
 *   softmax; top_p < 1 keeps the shortest prefix of the probabilities in
 *   descending order (ties by index) whose sum reaches top_p, renormalized;
 *   min_p > 0 drops probabilities below max * min_p, renormalized; the token
 *   is the first j with u[r] <= cumsum_j (V - 1 if none). A row whose
 *   reference probabilities are all NaN (all -Inf, a +Inf, or a NaN
 *   anywhere: the reference's top-k keeps a NaN first) draws V - 1 for any
 *   u; any other row draws 0 when u[r] <= 0, as the reference's loop
 *   returns its first index then.
 * Any V in [1, 4194304], any top_k, logits at any 4-byte alignment (a
 * top_k above 4096 takes a threshold path: the k-th element by count, the
 * softmax over the kept entries). No workspace. Sums are trees where the
 * reference adds sequentially, so a draw can differ only where u lies
 * within rounding of a step of the cumulative distribution. */
int ihip_sample(const float *logits_dev, int rows, int V, float T, int top_k,
                float top_p, float min_p, const float *u_dev,
                int32_t *out_tok_dev, void *stream);
/* ihip_sample with a caller workspace (ihip_sample_ws_bytes; 16-byte
 * aligned; 4104 bytes per 4096 logits of each row plus 49408 per row):
 * plain draws (T > 0, no top-k, top-p or min-p: the speculative defaults)
 * spread each row over workgroups of 4096 logits (their softmax
 * statistics, then the draw inside the round that holds u); so do top-k
 * from 1 to 64 at V <= 262144 (each chunk's top-k, then the row's among
 * them: the tokens of ihip_sample), top-p and / or min-p without top-k
 * (the threshold's histograms merged per row), a larger top-k (its
 * threshold by count, the kept entries compacted, then ihip_sample's
 * candidate draw: its tokens; above 4096, ihip_sample's threshold path),
 * and T = 0 (each chunk's first argmax: the tokens of ihip_sample). The
 * same limits and the same softmax_sample
 * (src/ModelCPU.jl:1123-1200) and the same contract: draws match the exact
 * cumulative distribution except within rounding of a step. */
int ihip_sample_ws_bytes(int rows, int V, size_t *bytes);
int ihip_sample_ex(const float *logits_dev, int rows, int V, float T, int top_k,
                   float top_p, float min_p, const float *u_dev,
                   int32_t *out_tok_dev, void *ws, size_t ws_bytes,
                   void *stream);

/* The penalties the generation loop applies before sampling
 * (apply_presence_penalty!, apply_repetition_penalty!,
 * src/ModelCPU.jl:1202-1225), in place on logits [rows x V]: row r's token
 * ids are tok_dev[r * tok_stride + i], i < n_tok (tok_stride 0: one list for
 * every row); for each distinct id in [0, V): x -= presence (presence != 0),
 * then x = x > 0 ? x / repetition : x * repetition (repetition != 1).
 * Any V >= 1. */
int ihip_apply_penalties(float *logits_dev, int rows, int V,
                         const int32_t *tok_dev, int n_tok, int64_t tok_stride,
                         float presence, float repetition, void *stream);

/* ---- GGUF file -> device weights (csrc/gguf.cpp) ---- */

/* read_gguf (src/GGUF.jl:119-165): the file is memory-mapped read-only and
 * its header, metadata and tensor table parsed with bounds checks (a
 * malformed file returns IHIP_EINVAL with the reason: "Not a valid GGUF
 * file" for a bad magic, strings over 1 MiB, unknown value types, tensor
 * data past the end). Metadata keys are unique (a repeated key: the last).
 * Tensor dims are innermost first (dims[0] = K, dims[1] = N of a matrix);
 * nbytes is 0 for GGML types whose layout this library does not know (it
 * knows F32, F16, BF16, Q8_0, Q4_K, Q5_K, Q6_K, I8..I64, F64). Returned
 * strings and tensor_data point into the mapping: valid until close. */
int ihip_gguf_open(const char *path, void **handle);
int ihip_gguf_close(void *handle);
int ihip_gguf_info(void *handle, uint32_t *version, int64_t *n_tensors,
                   int64_t *n_kv, uint64_t *alignment, uint64_t *data_offset);
int ihip_gguf_tensor(void *handle, int64_t i, const char **name,
                     int *ggml_type, int *ndim, int64_t *dims /* [4] */,
                     uint64_t *offset, uint64_t *nbytes);
int64_t ihip_gguf_find_tensor(void *handle, const char *name);  /* -1: absent */
int64_t ihip_gguf_find_key(void *handle, const char *key);      /* -1: absent */
/* vtype: GGUF value type (0..12); arrays (9): atype and count, else atype
 * -1 and count 1. */
int ihip_gguf_kv(void *handle, int64_t i, const char **key, int *vtype,
                 int *atype, uint64_t *count);
/* element index of a numeric value or array: as an integer and as a double */
int ihip_gguf_kv_number(void *handle, int64_t i, uint64_t index,
                        int64_t *as_int, double *as_float);
/* a string value (index 0) or element index of a string array (not
 * NUL-terminated: len bytes) */
int ihip_gguf_kv_string(void *handle, int64_t i, uint64_t index,
                        const char **str, uint64_t *len);
const void *ihip_gguf_tensor_data(void *handle, int64_t i);  /* host bytes */
/* Copies tensor i to device memory (through pinned staging, synchronous on
 * the stream). IHIP_GGUF_PACKED: a 2-D Q4_K/Q5_K/Q6_K/Q8_0 matrix is stored
 * in the packed layout of ihip_pack_weights (dev_bytes >= ihip_packed_bytes),
 * else the GGUF bytes as they are (dev_bytes >= nbytes). The handle's pinned
 * staging (2 x 64 MiB, kept until close) serves one upload at a time. */
#define IHIP_GGUF_PACKED 1
int ihip_gguf_upload(void *handle, int64_t i, void *dev, size_t dev_bytes,
                     int flags, void *stream);

/* ---- synthetic inputs (benchmark and tests; csrc/misc.hip) ---- */

/* n_blocks seeded GGUF blocks of qtype starting at block first_block of
 * the given 64-bit stream (byte-identical to the Python generator). */
int ihip_synth_blocks(int qtype, uint64_t stream, int64_t first_block,
                      int64_t n_blocks, void *out_dev, void *stream_handle);
/* n fp32 N(0,1) samples * scale + (add_dev ? add_dev[i] : 0). */
int ihip_synth_gaussian(uint64_t stream, int64_t n, float scale,
                        const float *add_dev, float *out_dev,
                        void *stream_handle);

/* HBM read-bandwidth probe (measurement only): streams `bytes` (a multiple
 * of 16, src 16-byte aligned) with 16-byte non-temporal loads (the policy
 * the matmuls read their weights with), each of up to 2048
 * workgroups XORing what it read into its own word of out_dev (2048
 * words), so the plain-read ceiling can be reported beside the vendor peak
 * for the matmul kernels whose bound is HBM. */
int ihip_stream_read(const void *src_dev, size_t bytes, uint32_t *out_dev,
                     void *stream);

#ifdef __cplusplus
}
#endif
#endif /* INFERNO_HIP_H */
