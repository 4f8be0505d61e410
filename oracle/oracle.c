/*
 * CPU oracle for the speculative-verify hot path (TEST INFRASTRUCTURE ONLY:
 * loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
 * never by the product path). Built with -ffp-contract=off so that every
 * multiply and add rounds separately, as Julia evaluates the reference
 * formulas. Pinning status of each function is listed in oracle.h.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int orc_block_bytes(int qtype) {
    switch (qtype) {  /* src/QuantsCPU.jl:22-25 */
    case ORC_Q4_K: return 144;
    case ORC_Q5_K: return 176;
    case ORC_Q6_K: return 210;
    case ORC_Q8_0: return 34;
    }
    return -1;
}

int orc_block_elems(int qtype) {
    switch (qtype) {
    case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: return 256;
    case ORC_Q8_0: return 32;
    }
    return -1;
}

/* IEEE binary16 -> binary32, exact for every input (normals, subnormals,
 * +-0, Inf, NaN payloads). Same value as Julia Float32(::Float16) and the
 * reference's fp16_to_fp32 (src/kernels/quant_kernels.c:67-88). */
float orc_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff, f;
    if (e == 0) {
        if (m == 0) {
            f = sign;
        } else {  /* subnormal: value m * 2^-24, renormalize */
            int sh = 0;
            while (!(m & 0x400)) { m <<= 1; sh++; }
            f = sign | ((uint32_t)(113 - sh) << 23) | ((m & 0x3ff) << 13);
        }
    } else if (e == 31) {
        f = sign | 0x7f800000u | (m << 13);
    } else {
        f = sign | ((e + 112) << 23) | (m << 13);
    }
    float r;
    memcpy(&r, &f, 4);
    return r;
}

static inline float rd_f16(const uint8_t *p) {
    return orc_fp16_to_fp32((uint16_t)(p[0] | (p[1] << 8)));
}

/* 6-bit scale/min of sub-block s of a Q4_K/Q5_K block,
 * src/QuantsCPU.jl:501-513 (0-based restatement of the 1-based indexing). */
static inline void scale_min_k4(const uint8_t *scales, int s, uint8_t *sc,
                                uint8_t *m) {
    if (s < 4) {
        *sc = scales[s] & 63;
        *m = scales[s + 4] & 63;
    } else {
        *sc = (uint8_t)((scales[s + 4] & 0x0f) | ((scales[s - 4] >> 6) << 4));
        *m = (uint8_t)((scales[s + 4] >> 4) | ((scales[s] >> 6) << 4));
    }
}

/* src/QuantsCPU.jl:491-527 (dequantize_q4_k_block!); also
 * src/Dequant.jl:325-375. w = (d*sc)*q - (dmin*m), no fusion. */
static void dq_q4_k(const uint8_t *b, float *out) {
    const float d = rd_f16(b), dmin = rd_f16(b + 2);
    const uint8_t *scales = b + 4, *qs = b + 16;
    for (int j = 0; j < 4; j++) {
        uint8_t sc1, m1, sc2, m2;
        scale_min_k4(scales, 2 * j, &sc1, &m1);
        scale_min_k4(scales, 2 * j + 1, &sc2, &m2);
        const float d1 = d * (float)sc1, min1 = dmin * (float)m1;
        const float d2 = d * (float)sc2, min2 = dmin * (float)m2;
        for (int l = 0; l < 32; l++) {
            const uint8_t q = qs[32 * j + l];
            out[64 * j + l] = d1 * (float)(q & 0x0f) - min1;
            out[64 * j + 32 + l] = d2 * (float)(q >> 4) - min2;
        }
    }
}

/* src/QuantsCPU.jl:529-607 (dequantize_q5_k_block!); src/Dequant.jl:379-441.
 * v = float(low) + (bit ? 16 : 0) is exact; w = d1*v - m1. */
static void dq_q5_k(const uint8_t *b, float *out) {
    const float d = rd_f16(b), dmin = rd_f16(b + 2);
    const uint8_t *scales = b + 4, *qh = b + 16, *qs = b + 48;
    for (int j = 0; j < 4; j++) {
        uint8_t sc1, m1, sc2, m2;
        scale_min_k4(scales, 2 * j, &sc1, &m1);
        scale_min_k4(scales, 2 * j + 1, &sc2, &m2);
        const float d1 = d * (float)sc1, mv1 = dmin * (float)m1;
        const float d2 = d * (float)sc2, mv2 = dmin * (float)m2;
        const uint8_t u1 = (uint8_t)(1u << (2 * j)), u2 = (uint8_t)(2u << (2 * j));
        for (int l = 0; l < 32; l++) {
            const uint8_t q = qs[32 * j + l];
            const float v1 = (float)(q & 0x0f) + ((qh[l] & u1) ? 16.0f : 0.0f);
            const float v2 = (float)(q >> 4) + ((qh[l] & u2) ? 16.0f : 0.0f);
            out[64 * j + l] = d1 * v1 - mv1;
            out[64 * j + 32 + l] = d2 * v2 - mv2;
        }
    }
}

/* src/QuantsCPU.jl:609-646 (dequantize_q6_k_block!); src/Dequant.jl:558-601.
 * w = (d*sc)*q, q in -32..31. The non-! dequantize_q6_k_block
 * (src/QuantsCPU.jl:289-324) is defective and not followed. */
static void dq_q6_k(const uint8_t *b, float *out) {
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    const float d = rd_f16(b + 208);
    for (int n = 0; n < 2; n++) {
        const uint8_t *qln = ql + 64 * n, *qhn = qh + 32 * n;
        const int8_t *scn = sc + 8 * n;
        for (int l = 0; l < 32; l++) {
            const int is = l / 16;
            const uint8_t h = qhn[l];
            const int q1 = (int)((qln[l] & 0x0f) | ((h & 3) << 4)) - 32;
            const int q2 = (int)((qln[l + 32] & 0x0f) | (((h >> 2) & 3) << 4)) - 32;
            const int q3 = (int)((qln[l] >> 4) | (((h >> 4) & 3) << 4)) - 32;
            const int q4 = (int)((qln[l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32;
            out[128 * n + l] = d * (float)scn[is] * (float)q1;
            out[128 * n + l + 32] = d * (float)scn[is + 2] * (float)q2;
            out[128 * n + l + 64] = d * (float)scn[is + 4] * (float)q3;
            out[128 * n + l + 96] = d * (float)scn[is + 6] * (float)q4;
        }
    }
}

/* src/QuantsCPU.jl:648-658; src/Dequant.jl:304-321. w = d*q. */
static void dq_q8_0(const uint8_t *b, float *out) {
    const float d = rd_f16(b);
    for (int i = 0; i < 32; i++) out[i] = d * (float)(int8_t)b[2 + i];
}

typedef void (*dq_fn)(const uint8_t *, float *);
static dq_fn dq_for(int qtype) {
    switch (qtype) {
    case ORC_Q4_K: return dq_q4_k;
    case ORC_Q5_K: return dq_q5_k;
    case ORC_Q6_K: return dq_q6_k;
    case ORC_Q8_0: return dq_q8_0;
    }
    return NULL;
}

int orc_dequant(int qtype, const uint8_t *data, int64_t n_blocks, float *out) {
    dq_fn f = dq_for(qtype);
    if (!f) return -22;
    const int bb = orc_block_bytes(qtype), be = orc_block_elems(qtype);
    for (int64_t i = 0; i < n_blocks; i++) f(data + i * bb, out + i * be);
    return 0;
}

/* Row r owns blocks [r*K/QK, (r+1)*K/QK) (src/QuantsCPU.jl:471-472,
 * src/ModelCPU.jl:295-296, src/kernels/quant_kernels.c:612). */
int orc_gemv_f64(int qtype, const uint8_t *w, const float *x, double *y,
                 int M, int N, int K) {
    dq_fn f = dq_for(qtype);
    if (!f) return -22;
    const int bb = orc_block_bytes(qtype), be = orc_block_elems(qtype);
    if (K % be) return -22;
    const int nb = K / be;
    /* Each output is one sequential fp64 sum over k; up to 8 outputs of a row
     * are summed side by side (independent accumulators, same order each),
     * which changes no result. */
    #pragma omp parallel
    {
        float *row = (float *)malloc(sizeof(float) * (size_t)K);
        #pragma omp for schedule(static)
        for (int r = 0; r < N; r++) {
            for (int b = 0; b < nb; b++)
                f(w + ((size_t)r * nb + b) * bb, row + (size_t)b * be);
            for (int m0 = 0; m0 < M; m0 += 8) {
                const int mn = M - m0 < 8 ? M - m0 : 8;
                double s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                const float *xm = x + (size_t)m0 * K;
                for (int k = 0; k < K; k++) {
                    const double wk = (double)row[k];
                    for (int j = 0; j < mn; j++) s[j] += wk * (double)xm[(size_t)j * K + k];
                }
                for (int j = 0; j < mn; j++) y[(size_t)(m0 + j) * N + r] = s[j];
            }
        }
        free(row);
    }
    return 0;
}

/* src/ModelCPU.jl:284-378: sum_val += block_values[i] * x[col] in fp32,
 * blocks in order, elements in order. */
int orc_gemv_seq_f32(int qtype, const uint8_t *w, const float *x, float *y,
                     int M, int N, int K) {
    dq_fn f = dq_for(qtype);
    if (!f) return -22;
    const int bb = orc_block_bytes(qtype), be = orc_block_elems(qtype);
    if (K % be) return -22;
    const int nb = K / be;
    #pragma omp parallel
    {
        float blk[256];
        #pragma omp for schedule(static)
        for (int r = 0; r < N; r++) {
            for (int m = 0; m < M; m++) {
                const float *xm = x + (size_t)m * K;
                float s = 0.0f;
                for (int b = 0; b < nb; b++) {
                    f(w + ((size_t)r * nb + b) * bb, blk);
                    for (int i = 0; i < be; i++) s += blk[i] * xm[b * be + i];
                }
                y[(size_t)m * N + r] = s;
            }
        }
    }
    return 0;
}

/* ---- Reference fast path (Q8_K integer dot), restated ---- */

/* block_q8_K, src/kernels/quant_kernels.c:52-56: float d; int8 qs[256];
 * int16 bsums[16] (292 bytes, no padding). */
typedef struct {
    float d;
    int8_t qs[256];
    int16_t bsums[16];
} orc_q8K;

/* src/kernels/quant_kernels.c:166-194. */
void orc_quantize_q8_K(const float *x, void *q8v, int64_t k) {
    orc_q8K *y = (orc_q8K *)q8v;
    const int nb = (int)(k / 256);
    for (int i = 0; i < nb; i++) {
        const float *src = x + (size_t)i * 256;
        float amax = 0.0f;
        for (int j = 0; j < 256; j++) {
            const float ax = fabsf(src[j]);
            if (ax > amax) amax = ax;
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = d;
        for (int j = 0; j < 256; j += 16) {
            int sum = 0;
            for (int l = 0; l < 16; l++) {
                const int8_t q = (int8_t)roundf(src[j + l] * id);
                y[i].qs[j + l] = q;
                sum += q;
            }
            y[i].bsums[j / 16] = (int16_t)sum;
        }
    }
}

/* hsum_float_8 (quant_kernels.c:91-98): ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) */
static inline float hsum8(const float *a) {
    const float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
    return (s0 + s2) + (s1 + s3);
}

/* utmp rearrangement (quant_kernels.c:221-226) expressed per value. */
static void unpack_sc_m(const uint8_t *scales, int *sc, int *m) {
    for (int s = 0; s < 8; s++) {
        uint8_t a, b;
        scale_min_k4(scales, s, &a, &b);
        sc[s] = a;
        m[s] = b;
    }
}

/* quant_kernels.c:204-278. Lane t of the 8-lane int32 accumulator covers
 * bytes 4t..4t+3 of each 32-byte slice; the mins use 4 lanes. */
float orc_vec_dot_q4_K_q8_K(const uint8_t *w, const void *q8v, int nb) {
    const orc_q8K *y = (const orc_q8K *)q8v;
    float acc[8] = {0}, accm[4] = {0};
    for (int i = 0; i < nb; i++) {
        const uint8_t *x = w + (size_t)i * 144;
        const float d = y[i].d * rd_f16(x);
        const float dmin = -y[i].d * rd_f16(x + 2);
        int sc[8], m[8];
        unpack_sc_m(x + 4, sc, m);
        int s8[8];
        for (int u = 0; u < 8; u++) s8[u] = y[i].bsums[2 * u] + y[i].bsums[2 * u + 1];
        for (int t = 0; t < 4; t++) {
            const int prod = m[2 * t] * s8[2 * t] + m[2 * t + 1] * s8[2 * t + 1];
            accm[t] = fmaf(dmin, (float)prod, accm[t]);
        }
        int sumi[8] = {0};
        const uint8_t *q4 = x + 16;
        const int8_t *q8 = y[i].qs;
        for (int j = 0; j < 4; j++) {
            for (int t = 0; t < 8; t++) {
                int pl = 0, ph = 0;
                for (int b = 4 * t; b < 4 * t + 4; b++) {
                    pl += (q4[32 * j + b] & 0xf) * q8[64 * j + b];
                    ph += (q4[32 * j + b] >> 4) * q8[64 * j + 32 + b];
                }
                sumi[t] += sc[2 * j] * pl + sc[2 * j + 1] * ph;
            }
        }
        for (int t = 0; t < 8; t++) acc[t] = fmaf(d, (float)sumi[t], acc[t]);
    }
    const float am = (accm[0] + accm[2]) + (accm[1] + accm[3]);
    return hsum8(acc) + am;
}

/* quant_kernels.c:311-397. */
float orc_vec_dot_q5_K_q8_K(const uint8_t *w, const void *q8v, int nb) {
    const orc_q8K *y = (const orc_q8K *)q8v;
    float acc[8] = {0}, summs = 0.0f;
    for (int i = 0; i < nb; i++) {
        const uint8_t *x = w + (size_t)i * 176;
        const float d = y[i].d * rd_f16(x);
        const float dmin = -y[i].d * rd_f16(x + 2);
        int sc[8], m[8];
        unpack_sc_m(x + 4, sc, m);
        int hs = 0;
        for (int u = 0; u < 8; u++)
            hs += m[u] * (y[i].bsums[2 * u] + y[i].bsums[2 * u + 1]);
        summs = fmaf(dmin, (float)hs, summs);  /* gcc contracts this line of the reference (-ffp-contract=fast) */
        const uint8_t *qh = x + 16, *q5 = x + 48;
        const int8_t *q8 = y[i].qs;
        int sumi[8] = {0};
        for (int j = 0; j < 4; j++) {
            for (int t = 0; t < 8; t++) {
                int p0 = 0, p1 = 0;
                for (int b = 4 * t; b < 4 * t + 4; b++) {
                    const int v0 = (q5[32 * j + b] & 0xf) + (((qh[b] >> (2 * j)) & 1) << 4);
                    const int v1 = (q5[32 * j + b] >> 4) + (((qh[b] >> (2 * j + 1)) & 1) << 4);
                    p0 += v0 * q8[64 * j + b];
                    p1 += v1 * q8[64 * j + 32 + b];
                }
                sumi[t] += sc[2 * j] * p0 + sc[2 * j + 1] * p1;
            }
        }
        for (int t = 0; t < 8; t++) acc[t] = fmaf(d, (float)sumi[t], acc[t]);
    }
    return hsum8(acc) + summs;
}

/* quant_kernels.c:440-521. Per 128-element half j and quarter i, lanes
 * t<4 use scale 8j+2i, lanes t>=4 use 8j+2i+1. */
float orc_vec_dot_q6_K_q8_K(const uint8_t *w, const void *q8v, int nb) {
    const orc_q8K *y = (const orc_q8K *)q8v;
    float acc[8] = {0};
    for (int i = 0; i < nb; i++) {
        const uint8_t *x = w + (size_t)i * 210;
        const float d = y[i].d * rd_f16(x + 208);
        const int8_t *sc = (const int8_t *)(x + 192);
        int sumi[8] = {0};
        for (int j = 0; j < 2; j++) {
            const uint8_t *ql = x + 64 * j, *qh = x + 128 + 32 * j;
            const int8_t *q8 = y[i].qs + 128 * j;
            for (int qi = 0; qi < 4; qi++) {
                for (int t = 0; t < 8; t++) {
                    int p = 0;
                    for (int b = 4 * t; b < 4 * t + 4; b++) {
                        int q;
                        const uint8_t h = qh[b];
                        switch (qi) {
                        case 0: q = (ql[b] & 0xf) | ((h & 3) << 4); break;
                        case 1: q = (ql[32 + b] & 0xf) | (((h >> 2) & 3) << 4); break;
                        case 2: q = (ql[b] >> 4) | (((h >> 4) & 3) << 4); break;
                        default: q = (ql[32 + b] >> 4) | (((h >> 6) & 3) << 4); break;
                        }
                        p += (q - 32) * q8[32 * qi + b];
                    }
                    const int s = sc[8 * j + 2 * qi + (t >= 4 ? 1 : 0)];
                    sumi[t] += s * p;
                }
            }
        }
        for (int t = 0; t < 8; t++) acc[t] = fmaf(d, (float)sumi[t], acc[t]);
    }
    return hsum8(acc);
}

/* quant_kernels.c:657-683: fp32 x directly, 8 lanes, single-threaded. */
static void q8_0_gemv_port(const uint8_t *w, const float *x, float *out,
                           int inner_dim, int outer_dim) {
    const int nb = inner_dim / 32;
    for (int r = 0; r < outer_dim; r++) {
        float acc[8] = {0};
        for (int b = 0; b < nb; b++) {
            const uint8_t *blk = w + ((size_t)r * nb + b) * 34;
            const float d = rd_f16(blk);
            const float *xv = x + b * 32;
            for (int j = 0; j < 32; j += 8)
                for (int t = 0; t < 8; t++) {
                    const float prod = (float)(int8_t)blk[2 + j + t] * xv[j + t];
                    acc[t] = fmaf(d, prod, acc[t]);
                }
        }
        out[r] = hsum8(acc);
    }
}

/* quant_kernels.c:602-650: quantize once, rows in parallel when N > 64. */
int orc_gemv_q8k(int qtype, const uint8_t *w, const float *x, float *out,
                 void *q8_buf, int inner_dim, int outer_dim, int nthreads) {
    if (qtype == ORC_Q8_0) {
        if (inner_dim % 32) return -22;
        q8_0_gemv_port(w, x, out, inner_dim, outer_dim);
        return 0;
    }
    if (inner_dim % 256) return -22;
    const int nb = inner_dim / 256, bb = orc_block_bytes(qtype);
    float (*dot)(const uint8_t *, const void *, int) =
        qtype == ORC_Q4_K ? orc_vec_dot_q4_K_q8_K :
        qtype == ORC_Q5_K ? orc_vec_dot_q5_K_q8_K :
        qtype == ORC_Q6_K ? orc_vec_dot_q6_K_q8_K : NULL;
    if (!dot) return -22;
    orc_quantize_q8_K(x, q8_buf, inner_dim);
    (void)nthreads;
    #pragma omp parallel for schedule(static) if (outer_dim > 64) num_threads(nthreads > 0 ? nthreads : 1)
    for (int r = 0; r < outer_dim; r++)
        out[r] = dot(w + (size_t)r * nb * bb, q8_buf, nb);
    return 0;
}

/* ---- Softmax and acceptance ---- */

void orc_softmax_stats(const float *L, int V, float T, double *zmax,
                       double *zsum) {
    double mx = -INFINITY;
    for (int j = 0; j < V; j++) {
        const double z = (double)(L[j] / T);
        if (z > mx) mx = z;
    }
    double s = 0.0;
    for (int j = 0; j < V; j++) s += exp((double)(L[j] / T) - mx);
    *zmax = mx;
    *zsum = s;
}

/* Julia argmax: first index of the maximum (tests/unit/test_engine.jl:56-69).
 * findmax replaces its current maximum m by x iff isless(m, x), Julia's total
 * order of floats: -Inf < ... < -0.0 < +0.0 < ... < +Inf < NaN, NaNs equal.
 * So a NaN replaces a number, +0.0 replaces -0.0, and a later equal value
 * (or a later NaN) never replaces the current one. */
static inline int beats(float a, float b) {
    if (isnan(a) || isnan(b)) return isnan(a) && !isnan(b);
    return a > b || (a == b && signbit(b) && !signbit(a));
}
int32_t orc_argmax_first(const float *L, int V) {
    int32_t best = 0;
    for (int j = 1; j < V; j++)
        if (beats(L[j], L[best])) best = j;
    return best;
}

static inline double prob_at(const float *L, int j, float T, double mx,
                             double s) {
    return exp((double)(L[j] / T) - mx) / s;
}

/* Inverse CDF: first j with u*S <= C_j (C = inclusive prefix sum of w),
 * fallback V-1 (src/SpeculativeDecoding.jl:20-30, src/ModelCPU.jl:1191-1199
 * with the uniform passed explicitly). */
static int32_t inv_cdf(const double *w, int V, double S, float u) {
    const double target = (double)u * S;
    double c = 0.0;
    for (int j = 0; j < V; j++) {
        c += w[j];
        if (target <= c) return j;
    }
    return V - 1;
}

int orc_spec_accept(const float *Lt, const float *Ld, const int32_t *draft,
                    int k, int V, float T, const float *u_acc, float u_res,
                    float u_bonus, int mode, int32_t *out_tok, int32_t *out_n) {
    if (k < 0 || V < 1 || (mode != 0 && mode != 1)) return -22;
    if (mode == 0 && !(T > 0.0f)) return -22;
    for (int i = 0; i < k; i++)
        if (draft[i] < 0 || draft[i] >= V) return -22;
    double *w = (double *)malloc(sizeof(double) * (size_t)V);
    if (!w) return -12;
    /* mode 1 follows src/SpeculativeDecoding.jl:75-97: both softmaxes at
     * T = 1, the draft probability is a scalar, the residual subtracts it
     * from every entry. */
    const float Tr = mode == 0 ? T : 1.0f;
    int n = 0;
    for (int i = 0; i < k; i++) {
        const float *lt = Lt + (size_t)i * V, *ld = Ld + (size_t)i * V;
        double tm, ts, dm, ds;
        orc_softmax_stats(lt, V, Tr, &tm, &ts);
        orc_softmax_stats(ld, V, Tr, &dm, &ds);
        const int x = draft[i];
        const double p = prob_at(lt, x, Tr, tm, ts);
        const double q = prob_at(ld, x, Tr, dm, ds);
        const double ratio = q > 0.0 ? (p / q < 1.0 ? p / q : 1.0) : 1.0;
        if ((double)u_acc[i] < ratio) {
            out_tok[n++] = x;
            continue;
        }
        /* reject: residual resample */
        double S = 0.0;
        for (int j = 0; j < V; j++) {
            const double pj = prob_at(lt, j, Tr, tm, ts);
            const double qj = mode == 0 ? prob_at(ld, j, Tr, dm, ds) : q;
            const double r = pj - qj;
            w[j] = r > 0.0 ? r : 0.0;
            S += w[j];
        }
        int32_t tok;
        if (S > 0.0) {
            tok = inv_cdf(w, V, S, u_res);
        } else if (mode == 0) {
            for (int j = 0; j < V; j++) w[j] = prob_at(lt, j, Tr, tm, ts);
            tok = inv_cdf(w, V, 1.0, u_res);
        } else {
            tok = V - 1;  /* all-NaN residual returns length(probs) */
        }
        out_tok[n] = tok;
        *out_n = n;
        /* mode 1: the reference appends the bonus whenever length(accepted)
         * == gamma (src/SpeculativeDecoding.jl:100), which a rejection at the
         * last draft also reaches (k - 1 drafts + the residual): the bonus
         * from target row k at T follows the residual token. */
        if (mode == 1 && n == k - 1) {
            const float *lk = Lt + (size_t)k * V;
            double m, s;
            orc_softmax_stats(lk, V, T, &m, &s);
            for (int j = 0; j < V; j++) w[j] = prob_at(lk, j, T, m, s);
            out_tok[n + 1] = inv_cdf(w, V, 1.0, u_bonus);
        }
        free(w);
        return 0;
    }
    /* all accepted: bonus token from the last target row at T
     * (src/SpeculativeDecoding.jl:100-104 via softmax_sample) */
    const float *lk = Lt + (size_t)k * V;
    int32_t tok;
    if (T == 0.0f) {
        tok = orc_argmax_first(lk, V);
    } else {
        double m, s;
        orc_softmax_stats(lk, V, T, &m, &s);
        for (int j = 0; j < V; j++) w[j] = prob_at(lk, j, T, m, s);
        tok = inv_cdf(w, V, 1.0, u_bonus);
    }
    out_tok[n] = tok;
    *out_n = n;
    free(w);
    return 0;
}

int orc_spec_accept_batch(const float *Lt, const float *Ld,
                          const int32_t *draft, int steps, int k, int V,
                          float T, const float *u_acc, const float *u_res,
                          const float *u_bonus, int mode, int32_t *out_tok,
                          int32_t *out_n) {
    if (steps < 0 || k < 0 || V < 1) return -22;
    int bad = 0;
    #pragma omp parallel for schedule(dynamic, 4) reduction(| : bad)
    for (int s = 0; s < steps; s++) {
        const int rc = orc_spec_accept(Lt + (size_t)s * (k + 1) * V, Ld + (size_t)s * k * V, draft + (size_t)s * k,
                                       k, V, T, u_acc + (size_t)s * k, u_res[s], u_bonus[s], mode,
                                       out_tok + (size_t)s * (k + 1), out_n + s);
        if (rc == -22) out_n[s] = -1;
        else if (rc != 0) bad = 1;
    }
    return bad ? -12 : 0;
}

int orc_greedy_verify(const float *logits, const int32_t *draft, int k, int V,
                      int32_t *out_n, int32_t *out_argmax) {
    if (k < 0 || V < 1) return -22;
    int n = 0, stop = 0;
    for (int i = 0; i <= k; i++) {
        const int32_t a = orc_argmax_first(logits + (size_t)i * V, V);
        if (out_argmax) out_argmax[i] = a;
        if (i < k && !stop) {
            if (a == draft[i]) n++;
            else stop = 1;
        }
    }
    *out_n = n;
    return 0;
}

int orc_tree_accept(const float *Lt, const float *Ld, const int32_t *tok,
                    const int32_t *parent, int n, int V, float T,
                    const float *u, int32_t *out_path, int32_t *out_len) {
    if (n < 1 || V < 1 || !(T > 0.0f)) return -22;
    for (int i = 1; i < n; i++)
        if (parent[i] < 0 || parent[i] >= i || tok[i] < 0 || tok[i] >= V) return -22;
    char *acc = (char *)calloc((size_t)n, 1);
    int *depth = (int *)calloc((size_t)n, sizeof(int));
    if (!acc || !depth) { free(acc); free(depth); return -12; }
    acc[0] = 1;
    int best = 0;
    for (int i = 1; i < n; i++) {
        const int p = parent[i];
        depth[i] = depth[p] + 1;
        if (!acc[p]) continue;
        const float *lt = Lt + (size_t)p * V, *ld = Ld + (size_t)p * V;
        double tm, ts, dm, ds;
        orc_softmax_stats(lt, V, T, &tm, &ts);
        orc_softmax_stats(ld, V, T, &dm, &ds);
        const double pp = prob_at(lt, tok[i], T, tm, ts);
        const double qq = prob_at(ld, tok[i], T, dm, ds);
        const double ratio = qq > 0.0 ? (pp / qq < 1.0 ? pp / qq : 1.0) : 1.0;
        if ((double)u[i] < ratio) {
            acc[i] = 1;
            if (depth[i] > depth[best]) best = i;  /* ties keep the smaller index */
        }
    }
    const int len = depth[best] + 1;
    for (int v = best, d = len - 1; d >= 0; d--) {
        out_path[d] = v;
        v = d > 0 ? parent[v] : 0;
    }
    *out_len = len;
    free(acc);
    free(depth);
    return 0;
}

void orc_rmsnorm(const float *x, const float *w, int n, float eps, float *out) {
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * (double)x[i];
    const float scale = 1.0f / sqrtf((float)(ss / n) + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * scale * (w ? w[i] : 1.0f);
}

/* ---- CPU baseline: one verify step through the reference's kernels ---- */

#include <time.h>

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* y = gemv(w, x) with the time spent inside added to *t */
static void timed_gemv(orc_gemv_fn f, const uint8_t *w, const float *x, float *y, void *q8, int K, int N,
                       double *t) {
    const double t0 = now_s();
    f(w, x, y, q8, K, N);
    *t += now_s() - t0;
}

int orc_cpu_verify_step(orc_gemv_fn q4k, orc_gemv_fn q6k, const struct orc_step_layer *layers, int n_layers,
                        const uint8_t *lm, const float *out_norm, int M, int H, int NQ, int NKV, int FF, int V,
                        const float *x0, const float *Ld, const int32_t *draft, float T, const float *u_acc,
                        float u_res, float u_bonus, float *logits, int32_t *out_tok, int32_t *out_n,
                        double *sec_layers, double *sec_head, double *sec_gemv) {
    if (!q4k || !q6k || !layers || n_layers < 0 || M < 1 || H % 256 || NQ % 256 || FF % 256) return -22;
    const int KMAX = FF > H ? (FF > NQ ? FF : NQ) : (H > NQ ? H : NQ);
    float *x = (float *)malloc(sizeof(float) * (size_t)M * H);
    float *h = (float *)malloc(sizeof(float) * (size_t)KMAX);
    float *q = (float *)malloc(sizeof(float) * (size_t)NQ);
    float *kv = (float *)malloc(sizeof(float) * (size_t)2 * NKV);
    float *t = (float *)malloc(sizeof(float) * (size_t)(H > FF ? H : FF));
    float *g = (float *)malloc(sizeof(float) * (size_t)FF);
    float *u = (float *)malloc(sizeof(float) * (size_t)FF);
    void *q8 = malloc((size_t)(KMAX / 256) * 292);
    int rc = 0;
    if (!x || !h || !q || !kv || !t || !g || !u || !q8) {
        rc = -12;
        goto done;
    }
    memcpy(x, x0, sizeof(float) * (size_t)M * H);
    double tg = 0.0;
    const double t0 = now_s();
    for (int m = 0; m < M; m++) {  /* token-major, as forward_cpu! */
        float *xm = x + (size_t)m * H;
        for (int l = 0; l < n_layers; l++) {
            const struct orc_step_layer *L = layers + l;
            orc_rmsnorm(xm, L->attn_norm, H, 1e-6f, h);
            timed_gemv(q4k, L->q, h, q, q8, H, NQ, &tg);
            timed_gemv(q4k, L->k, h, kv, q8, H, NKV, &tg);
            timed_gemv(q4k, L->v, h, kv + NKV, q8, H, NKV, &tg);
            timed_gemv(q4k, L->o, q, t, q8, NQ, H, &tg);
            for (int i = 0; i < H; i++) xm[i] += t[i];
            orc_rmsnorm(xm, L->ffn_norm, H, 1e-6f, h);
            timed_gemv(q4k, L->gate, h, g, q8, H, FF, &tg);
            timed_gemv(q4k, L->up, h, u, q8, H, FF, &tg);
            for (int i = 0; i < FF; i++) g[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
            timed_gemv(q6k, L->down, g, t, q8, FF, H, &tg);
            for (int i = 0; i < H; i++) xm[i] += t[i];
        }
    }
    const double t1 = now_s();
    const double tg_layers = tg;
    for (int m = 0; m < M; m++) {
        orc_rmsnorm(x + (size_t)m * H, out_norm, H, 1e-6f, h);
        timed_gemv(q6k, lm, h, logits + (size_t)m * V, q8, H, V, &tg);
    }
    const double ta = now_s();
    if (Ld && draft && u_acc) rc = orc_spec_accept(logits, Ld, draft, M - 1, V, T, u_acc, u_res, u_bonus, 0, out_tok,
                                                    out_n);
    const double t2 = now_s();
    sec_gemv[2] = t2 - ta;
    *sec_layers = t1 - t0;
    *sec_head = t2 - t1;
    sec_gemv[0] = tg_layers;
    sec_gemv[1] = tg - tg_layers;
done:
    free(x); free(h); free(q); free(kv); free(t); free(g); free(u); free(q8);
    return rc;
}

/* The port's q4_k_gemv / q6_k_gemv with the reference's signature (the
 * CPU baseline when the reference build is absent): OpenMP's current
 * thread count. */
void orc_q4_k_gemv(const uint8_t *w, const float *x, float *out, void *q8, int K, int N) {
    orc_gemv_q8k(ORC_Q4_K, w, x, out, q8, K, N, omp_get_max_threads());
}
void orc_q6_k_gemv(const uint8_t *w, const float *x, float *out, void *q8, int K, int N) {
    orc_gemv_q8k(ORC_Q6_K, w, x, out, q8, K, N, omp_get_max_threads());
}
