/*
 * CPU oracle for the speculative-verify hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU port), never as the product path.
 *
 * Every function restates an algorithm of the reference (Inferno.jl, paths
 * relative to its repository root) and cites the lines it follows.
 *
 * Pinning status of each function (what checks it besides its own formula):
 *   orc_dequant_*        pinned: reference C kernel built from source
 *                        (oracle/_ref) on inputs whose Q8_K quantization is
 *                        exact, pack/unpack brute force, special cases.
 *   orc_gemv_f64         pinned: e_k columns, linearity, reference C kernel.
 *   orc_gemv_seq_f32     pinned: against orc_gemv_f64 (rel-L2 < 1e-6).
 *   orc_quantize_q8_K,
 *   orc_q*_gemv_q8k      pinned: bit-exact / 1e-6 against oracle/_ref.
 *   orc_softmax_stats    pinned: closed forms (one-hot, uniform, V=1).
 *   orc_spec_accept      pinned: brute force at V<=8, distribution-preserving
 *                        property of mode 0 (exact enumeration), p=q accepts,
 *                        p[x]=0 rejects, hand-worked reference-mode case.
 *   orc_greedy_verify    pinned: closed form ties -> first index.
 *   orc_tree_accept      pinned: brute-force enumeration on <=8 nodes, chain
 *                        tree reduces to orc_spec_accept's accepted length.
 *                        The reference has no tree code: reference parity is
 *                        unpinned by construction (no counterpart).
 *   orc_rmsnorm          pinned: closed forms (constant vectors, [3, 4], one
 *                        nonzero element, zeros): tests/test_host_logic.py.
 *   orc_cpu_verify_step  the CPU baseline's step driver (no result of its own
 *                        to pin: it calls the reference's gemv kernels and the
 *                        functions above in forward_cpu!'s order); its
 *                        logits are checked against the same step composed
 *                        from the pinned pieces in tests/test_oracle_quant.py.
 */
#ifndef INFERNO_ORACLE_H
#define INFERNO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids, src/GGUF.jl:25-60 */
enum { ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14 };

int orc_block_bytes(int qtype);  /* 34 / 144 / 176 / 210 */
int orc_block_elems(int qtype);  /* 32 / 256 / 256 / 256 */

float orc_fp16_to_fp32(uint16_t h);

/* Dequantize n_blocks consecutive blocks (bit-exact restatement). */
int orc_dequant(int qtype, const uint8_t *data, int64_t n_blocks, float *out);

/* y[m*N + r] = sum_k W[r,k] * x[m*K + k] in double. */
int orc_gemv_f64(int qtype, const uint8_t *w, const float *x, double *y,
                 int M, int N, int K);
/* Julia fallback order: per row, dequantize block, sequential fp32 sum
 * (src/ModelCPU.jl:284-378). */
int orc_gemv_seq_f32(int qtype, const uint8_t *w, const float *x, float *y,
                     int M, int N, int K);

/* Reference fast path restated: Q8_K activation quantization + integer dot,
 * with the AVX2 kernel's lane and summation order
 * (src/kernels/quant_kernels.c:166-306,311-397,440-521,657-683). */
void  orc_quantize_q8_K(const float *x, void *q8, int64_t k);
float orc_vec_dot_q4_K_q8_K(const uint8_t *w, const void *q8, int nb);
float orc_vec_dot_q5_K_q8_K(const uint8_t *w, const void *q8, int nb);
float orc_vec_dot_q6_K_q8_K(const uint8_t *w, const void *q8, int nb);
/* Row loop of q*_gemv (quant_kernels.c:602-697); nthreads as OpenMP. */
int orc_gemv_q8k(int qtype, const uint8_t *w, const float *x, float *out,
                 void *q8_buf, int inner_dim, int outer_dim, int nthreads);

/* Softmax of z = L / T over V entries: max of z and sum of exp(z - max)
 * (fp64). T == 0 is rejected (greedy uses argmax). */
void orc_softmax_stats(const float *L, int V, float T, double *zmax,
                       double *zsum);
/* Julia argmax: the first index of the maximum in Julia's isless order
 * (-0.0 below +0.0, NaN above every number: the first NaN wins), so a row
 * of -Inf gives 0. */
int32_t orc_argmax_first(const float *L, int V);

/* Speculative accept (src/SpeculativeDecoding.jl:37-107 and the build's
 * standard contract). mode 0 = standard, mode 1 = reference-compatible.
 * Tokens are 0-based. out_tok receives *out_n + 1 tokens (the accepted
 * drafts, then the resampled or bonus token), and in mode 1 one more when
 * the last draft is rejected (*out_n == k - 1): the bonus the reference
 * appends whenever length(accepted) == gamma (:100). Returns 0 or a
 * negative error. */
int orc_spec_accept(const float *Lt, const float *Ld, const int32_t *draft,
                    int k, int V, float T, const float *u_acc, float u_res,
                    float u_bonus, int mode, int32_t *out_tok, int32_t *out_n);
/* orc_spec_accept over `steps` independent steps laid out step-major as
 * ihip_spec_accept takes them (Lt [steps][k+1][V], Ld [steps][k][V],
 * draft / u_acc [steps][k], out_tok [steps][k+1], out_n [steps]); steps in
 * parallel (OpenMP). out_n[s] = -1 for a step with an invalid draft id. */
int orc_spec_accept_batch(const float *Lt, const float *Ld,
                          const int32_t *draft, int steps, int k, int V,
                          float T, const float *u_acc, const float *u_res,
                          const float *u_bonus, int mode, int32_t *out_tok,
                          int32_t *out_n);

/* Greedy verify (src/ModelCPU.jl:1914-1930): logits [(k+1) x V]; accepted =
 * leading i < k with argmax(logits[i]) == draft[i]. */
int orc_greedy_verify(const float *logits, const int32_t *draft, int k, int V,
                      int32_t *out_n, int32_t *out_argmax);

/* Tree accept walk: node i >= 1 accepted iff parent accepted and
 * u[i] < min(1, p_par[tok_i] / q_par[tok_i]) at temperature T.
 * out_path receives root..deepest accepted node, *out_len its length. */
int orc_tree_accept(const float *Lt, const float *Ld, const int32_t *tok,
                    const int32_t *parent, int n, int V, float T,
                    const float *u, int32_t *out_path, int32_t *out_len);

/* RMSNorm (src/ModelCPU.jl:110-122); w may be NULL (all ones). */
void orc_rmsnorm(const float *x, const float *w, int n, float eps, float *out);

/* CPU baseline of one verify step, timed: the reference C path as the
 * Julia host drives it, with its glue in C. forward_cpu! streams the M
 * tokens one at a time through every layer (src/ModelCPU.jl:970-980); per
 * token and layer: RMSNorm, q / k / v projections, o projection added to the
 * residual (attention itself is outside the path), RMSNorm, gate and up,
 * silu(gate) * up, down added to the residual (src/ModelCPU.jl:447-473,
 * 755-760, 870-891); then per token the final RMSNorm and the LM head
 * (full logits, :948-966), then the accept (orc_spec_accept, mode 0, on
 * the computed logits as target rows). gemv(w, x, out, q8, K, N) are the
 * reference's exported kernels (src/kernels/quant_kernels.c:602-650), the
 * Q8_K buffer preallocated as QuantizedKernels does
 * (src/QuantizedKernels.jl:59-70). Buffers are allocated before the clock
 * starts. Outputs: logits [M x V]; seconds in the layers, in the head and
 * the accept, and inside the gemv calls alone (sec_gemv[0]: the layers',
 * [1]: the head's; sec_gemv[2]: the accept's seconds). 0, or -12 / -22. */
typedef void (*orc_gemv_fn)(const uint8_t *w, const float *x, float *out,
                            void *q8, int K, int N);
struct orc_step_layer {
    const uint8_t *q, *k, *v, *o, *gate, *up, *down;
    const float *attn_norm, *ffn_norm;
};
int orc_cpu_verify_step(orc_gemv_fn q4k, orc_gemv_fn q6k,
                        const struct orc_step_layer *layers, int n_layers,
                        const uint8_t *lm, const float *out_norm, int M, int H,
                        int NQ, int NKV, int FF, int V, const float *x0,
                        const float *Ld, const int32_t *draft, float T,
                        const float *u_acc, float u_res, float u_bonus,
                        float *logits, int32_t *out_tok, int32_t *out_n,
                        double *sec_layers, double *sec_head,
                        double *sec_gemv);
/* The port's gemv with that signature (orc_gemv_q8k at OpenMP's thread
 * count). */
void orc_q4_k_gemv(const uint8_t *w, const float *x, float *out, void *q8,
                   int K, int N);
void orc_q6_k_gemv(const uint8_t *w, const float *x, float *out, void *q8,
                   int K, int N);

#ifdef __cplusplus
}
#endif
#endif
