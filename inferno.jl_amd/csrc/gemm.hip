// Fused GGUF dequant-matmul on gfx950 MFMA: Y[M x N] = X[M x K] W^T.
//
// Weights stay in the GGUF byte layout (row r owns blocks [r*K/QK,
// (r+1)*K/QK)) and are streamed from HBM exactly once per call. Every wave
// owns 16 weight rows, the N side of v_mfma_f32_16x16x{32,16}_f16. Lane
// (n = lane%16, g = lane/16) loads the bytes of row n that hold K-elements
// [g*CK/4, (g+1)*CK/4) of each chunk of CK (32, or 16 for Q6_K) weights
// sharing one scale, and turns the packed quants into fp16 in registers:
// v_perm_b32 drops each 4/5/6/8-bit quant under the fp16 exponent of 1024,
// one packed fp16 op removes the offset. Quants are small integers, so these
// fp16 values are exact.
//
// Activations (prep kernel, once per call): each 256-element unit of every
// token row is scaled by a power of two so its largest magnitude sits in
// [2^14, 2^15) and written to the workspace directly in the MFMA A-operand
// lane layout:
//  * fp32-accurate mode: two A rows per token, hi = fp16(x), lo = fp16(x-hi)
//    (22 significant bits; products are exact and MFMA accumulates in fp32):
//    rel-L2 ~1e-7 against the fp64 product.
//  * half mode: one A row per token, hi only (rel-L2 ~3e-4).
// plus the per-sub-block sums of x (for the Q4_K/Q5_K mins) and the inverse
// unit scales.
//
// Scales: Q4_K/Q5_K fold the 6-bit sub-block scale into B (sc*q <= 63*31 is
// exact in fp16, one packed fma from (1024+q)), accumulate a whole 256-block
// in the MFMA accumulator and apply d once:
//   y = sum_b [ d_b * sum_s sc_s * (q . x)_s  -  dmin_b * sum_s m_s * X_s ].
// Q6_K (int8 scales: sc*q can leave fp16's exact range) and Q8_0 scale the
// MFMA result per sub-block in fp32.
//
// Split-K is deterministic: a grid of (row groups of 64) x (K-slices); each
// workgroup stores its partial tile and a reduce kernel sums the partials in
// slice order (no floating-point atomics).
#include "common.h"

#include <algorithm>
#include <cstdlib>

namespace {

constexpr int WG_THREADS = 256;  // 4 waves
constexpr int ROWS_PER_WG = 64;
constexpr int UNIT = 256;        // K elements per loop unit
constexpr int UNIT_A1 = 8192;    // A-operand bytes per unit and 16-slot token tile

template <int QT> struct GemmCfg {
    static constexpr int BB = QTraits<QT>::BB;
    static constexpr int QK = QTraits<QT>::QK;
    static constexpr int CK = (QT == QT_Q6_K) ? 16 : 32;     // MFMA K per chunk
    static constexpr int CHUNKS = UNIT / CK;                 // chunks per unit
    static constexpr int LANE_HALVES = CK / 4;               // A/B halves per lane
    static constexpr bool MINS = (QT == QT_Q4_K || QT == QT_Q5_K);
};

// Raw bytes of one 256-element unit that one lane (row n, lane group g)
// needs, fetched with 16-byte loads.
//  Q4_K: header (d, dmin, scales) and quants qs[16g, +16), qs[64 + 16g, +16)
//  Q5_K: as Q4_K plus high bits qh[16(g&1), +16)
//  Q6_K: after a 4x4 transpose across lane groups, a/b/h[i] hold the dwords
//        ql[64n + 16h + 4g], ql[64n + 32 + 16h + 4g], qh[32n + 16h + 4g]
//        for i = 2n + h; sc all 16 scales; d the fp16 super-scale
//  Q8_0: w0/w1[b] hold qs dwords g and 4 + g of block b (transposed), d[b]
template <int QT> struct Unit;
template <> struct Unit<QT_Q4_K> { uint4 hdr, q0, q1; };
template <> struct Unit<QT_Q5_K> { uint4 hdr, q0, q1, qh; };
template <> struct Unit<QT_Q6_K> { uint32_t a[4], b[4], h[4]; uint4 sc; uint32_t d; };
template <> struct Unit<QT_Q8_0> { uint32_t d[8], w0[8], w1[8]; };

__device__ __forceinline__ uint4 ld_u128(const uint8_t *p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);  // gfx950 global loads accept any alignment
    return v;
}

// 4x4 dword transpose across the four 16-lane groups: on entry lane group i
// holds dwords D[i][0..3] in r0..r3, on exit lane group g holds D[0..3][g].
__device__ __forceinline__ void xpose4(uint32_t &r0, uint32_t &r1, uint32_t &r2, uint32_t &r3) {
    const auto a = __builtin_amdgcn_permlane32_swap(r0, r2, false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(r1, r3, false, false);
    r0 = a[0]; r2 = a[1]; r1 = b[0]; r3 = b[1];
    const auto c = __builtin_amdgcn_permlane16_swap(r0, r1, false, false);
    const auto d = __builtin_amdgcn_permlane16_swap(r2, r3, false, false);
    r0 = c[0]; r1 = c[1]; r2 = d[0]; r3 = d[1];
}

// Raw loads (issued early); finish_unit() applies the cross-lane transposes
// right before use. u: first byte of the unit in this lane's row; nblk: Q8_0
// blocks present in the unit (a row tail with K % 256 != 0 has fewer than 8).
template <int QT>
__device__ __forceinline__ void load_unit(const uint8_t *__restrict__ u, int g, int nblk, Unit<QT> &r) {
    if constexpr (QT == QT_Q4_K) {
        r.hdr = *(const uint4 *)u;
        r.q0 = *(const uint4 *)(u + 16 + 16 * g);
        r.q1 = *(const uint4 *)(u + 80 + 16 * g);
    } else if constexpr (QT == QT_Q5_K) {
        r.hdr = *(const uint4 *)u;
        r.qh = *(const uint4 *)(u + 16 + 16 * (g & 1));
        r.q0 = *(const uint4 *)(u + 48 + 16 * g);
        r.q1 = *(const uint4 *)(u + 112 + 16 * g);
    } else if constexpr (QT == QT_Q6_K) {
        // lane group g fetches chunk g of each transpose group
        const int n = g >> 1, h = g & 1;
        const uint4 A = ld_u128(u + 64 * n + 16 * h);
        const uint4 B = ld_u128(u + 64 * n + 32 + 16 * h);
        const uint4 H = ld_u128(u + 128 + 32 * n + 16 * h);
        r.a[0] = A.x; r.a[1] = A.y; r.a[2] = A.z; r.a[3] = A.w;
        r.b[0] = B.x; r.b[1] = B.y; r.b[2] = B.z; r.b[3] = B.w;
        r.h[0] = H.x; r.h[1] = H.y; r.h[2] = H.z; r.h[3] = H.w;
        r.sc = ld_u128(u + 192);
        r.d = ld_u16(u + 208);
    } else {
        // transpose k covers blocks 2k, 2k+1: lane group g fetches half (g&1)
        // of block 2k + (g>>1)
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int b = 2 * k + (g >> 1);
            const bool live = b < nblk;
            const uint4 v = ld_u128(u + 34 * (live ? b : 0) + 2 + 16 * (g & 1));
            r.w0[2 * k] = live ? v.x : 0x80808080u;
            r.w1[2 * k] = live ? v.y : 0x80808080u;
            r.w0[2 * k + 1] = live ? v.z : 0x80808080u;
            r.w1[2 * k + 1] = live ? v.w : 0x80808080u;
        }
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const bool live = b < nblk;
            const uint32_t d = ld_u16(u + 34 * (live ? b : 0));
            r.d[b] = live ? d : 0u;
        }
    }
}

template <int QT>
__device__ __forceinline__ void finish_unit(Unit<QT> &r) {
    if constexpr (QT == QT_Q6_K) {
        xpose4(r.a[0], r.a[1], r.a[2], r.a[3]);
        xpose4(r.b[0], r.b[1], r.b[2], r.b[3]);
        xpose4(r.h[0], r.h[1], r.h[2], r.h[3]);
    } else if constexpr (QT == QT_Q8_0) {
        // before: (w0[2k], w1[2k], w0[2k+1], w1[2k+1]) = dwords 0..3 of this
        // lane group's half-block; after: dword g of each of the 4 halves
#pragma unroll
        for (int k = 0; k < 4; k++) xpose4(r.w0[2 * k], r.w1[2 * k], r.w0[2 * k + 1], r.w1[2 * k + 1]);
    }
}

__device__ __forceinline__ f4 mfma32(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma16(h4 a, h4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float half_bits(uint32_t v) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xffffu));
}

// Four fp16 pairs (elements 0..7 of a lane) from two dwords of byte-sized
// quants (each byte < 128), times scale pair s, minus 1024*s.
__device__ __forceinline__ h8 b_frag_scaled(uint32_t x0, uint32_t x1, h2 s, h2 ns) {
    h8 r;
    const h2 p0 = __builtin_elementwise_fma(as_h2(pair_lo(x0)), s, ns);
    const h2 p1 = __builtin_elementwise_fma(as_h2(pair_hi(x0)), s, ns);
    const h2 p2 = __builtin_elementwise_fma(as_h2(pair_lo(x1)), s, ns);
    const h2 p3 = __builtin_elementwise_fma(as_h2(pair_hi(x1)), s, ns);
    r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
    r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
    return r;
}

template <int MT, bool SPLIT>
struct Acc {
    static constexpr int TPL = SPLIT ? 2 : 4;  // tokens per lane per tile
    f4 acc[MT];
    float macc[MT][TPL];
};

// Token index held by lane group g, tile mt, lane-token u; and the lane-token
// of accumulator element v.
template <bool SPLIT>
__device__ __forceinline__ int lane_token(int mt, int g, int u) {
    return SPLIT ? mt * 8 + 2 * g + u : mt * 16 + 4 * g + u;
}
template <bool SPLIT>
__device__ __forceinline__ constexpr int acc_token_u(int v) {
    return SPLIT ? (v >> 1) : v;
}

template <int QT, int MT, bool SPLIT>
__device__ __forceinline__ void compute_unit(const Unit<QT> &r, const uint8_t *a_lane, const float *x_lds,
                                             const float *i_lds, int g, Acc<MT, SPLIT> &A) {
    // a_lane: this lane's A entries of the unit; entry (chunk c, tile mt) is
    // at a_lane + (c * MT + mt) * 64 * ENTRY
    constexpr int TPL = Acc<MT, SPLIT>::TPL;
    constexpr int TOK = MT * (SPLIT ? 8 : 16);
    float inv[MT][TPL];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int u = 0; u < TPL; u++) inv[mt][u] = i_lds[lane_token<SPLIT>(mt, g, u)];

    if constexpr (QT == QT_Q4_K || QT == QT_Q5_K) {
        // MFMA m (0..7) of the unit takes from lane group g the 8 elements
        //   128(m>>2) + 64(g>>1) + 32((m>>1)&1) + 16(g&1) + 8(m&1) + e,
        // i.e. bytes 8(m&1).. of q0 (m < 4) or q1, low nibbles for even
        // (m>>1), high nibbles for odd, of sub-block 4(m>>2) + 2(g>>1) + ((m>>1)&1).
        const float d = half_bits(r.hdr.x), dmin = half_bits(r.hdr.x >> 16);
        const uint32_t s0 = r.hdr.y, s1 = r.hdr.z, s2 = r.hdr.w;
        const uint32_t sc_lo = s0 & 0x3f3f3f3fu, m_lo = s1 & 0x3f3f3f3fu;
        const uint32_t sc_hi = (s2 & 0x0f0f0f0fu) | (((s0 >> 6) & 0x03030303u) << 4);
        const uint32_t m_hi = ((s2 >> 4) & 0x0f0f0f0fu) | (((s1 >> 6) & 0x03030303u) << 4);
        const int sh = 16 * (g >> 1);
        const h2 neg1024 = as_h2(0xE400E400u);  // (-1024, -1024)
        h2 hs[4], ns[4];
        hs[0] = h2_of_small((sc_lo >> sh) & 0xffu);
        hs[1] = h2_of_small((sc_lo >> (sh + 8)) & 0xffu);
        hs[2] = h2_of_small((sc_hi >> sh) & 0xffu);
        hs[3] = h2_of_small((sc_hi >> (sh + 8)) & 0xffu);
#pragma unroll
        for (int i = 0; i < 4; i++) ns[i] = hs[i] * neg1024;
        f4 c[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) c[mt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const int ah = m >> 2, b = (m >> 1) & 1, hw = m & 1;
            const uint4 Q = ah ? r.q1 : r.q0;
            const uint32_t x0 = hw ? Q.z : Q.x, x1 = hw ? Q.w : Q.y;
            uint32_t n0 = (b ? (x0 >> 4) : x0) & 0x0f0f0f0fu;
            uint32_t n1 = (b ? (x1 >> 4) : x1) & 0x0f0f0f0fu;
            if constexpr (QT == QT_Q5_K) {
                const int hb = 4 * ah + 2 * (g >> 1) + b;  // bit 2j + b of qh[l]
                const uint32_t h0 = hw ? r.qh.z : r.qh.x, h1 = hw ? r.qh.w : r.qh.y;
                n0 |= ((h0 >> hb) & 0x01010101u) << 4;
                n1 |= ((h1 >> hb) & 0x01010101u) << 4;
            }
            const h8 bf = b_frag_scaled(n0, n1, hs[2 * ah + b], ns[2 * ah + b]);
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
                c[mt] = mfma32(*(const h8 *)(a_lane + (m * MT + mt) * 1024), bf, c[mt]);
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int v = 0; v < 4; v++)
                A.acc[mt][v] = __builtin_fmaf(d * inv[mt][acc_token_u<SPLIT>(v)], c[mt][v], A.acc[mt][v]);
        // mins: dmin * sum_s m_s * X_s for the lane's tokens
        float mv[8];
#pragma unroll
        for (int s = 0; s < 4; s++) {
            mv[s] = (float)((m_lo >> (8 * s)) & 0xffu);
            mv[s + 4] = (float)((m_hi >> (8 * s)) & 0xffu);
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
#pragma unroll
            for (int u = 0; u < TPL; u++) {
                const int t = lane_token<SPLIT>(mt, g, u);
                float sm = 0.f;
#pragma unroll
                for (int sb = 0; sb < 8; sb++) sm = __builtin_fmaf(mv[sb], x_lds[sb * TOK + t], sm);
                A.macc[mt][u] = __builtin_fmaf(dmin, sm, A.macc[mt][u]);
            }
        }
    } else if constexpr (QT == QT_Q6_K) {
        const float d = half_bits(r.d);
        float dinv[MT][TPL];
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int u = 0; u < TPL; u++) dinv[mt][u] = d * inv[mt][u];
        const h2 off = as_h2(0xE420E420u);  // (-1056, -1056): (1024 + q) - 1056 = q - 32
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = i >> 1, h = i & 1;
            uint32_t q[4];
            q[0] = (r.a[i] & 0x0f0f0f0fu) | ((r.h[i] & 0x03030303u) << 4);
            q[1] = (r.b[i] & 0x0f0f0f0fu) | (((r.h[i] >> 2) & 0x03030303u) << 4);
            q[2] = ((r.a[i] >> 4) & 0x0f0f0f0fu) | (((r.h[i] >> 4) & 0x03030303u) << 4);
            q[3] = ((r.b[i] >> 4) & 0x0f0f0f0fu) | (((r.h[i] >> 6) & 0x03030303u) << 4);
#pragma unroll
            for (int qq = 0; qq < 4; qq++) {
                const int s = 8 * n + 2 * qq + h;  // sub-block = chunk of 16
                const h2 p0 = as_h2(pair_lo(q[qq])) + off, p1 = as_h2(pair_hi(q[qq])) + off;
                h4 b;
                b[0] = p0[0]; b[1] = p0[1]; b[2] = p1[0]; b[3] = p1[1];
                const uint32_t scw = (s >> 2) == 0 ? r.sc.x : (s >> 2) == 1 ? r.sc.y : (s >> 2) == 2 ? r.sc.z : r.sc.w;
                const float scf = (float)(int)(int8_t)((scw >> (8 * (s & 3))) & 0xffu);
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    const h4 a = *(const h4 *)(a_lane + (s * MT + mt) * 512);
                    const f4 c = mfma16(a, b, f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                    for (int v = 0; v < 4; v++)
                        A.acc[mt][v] = __builtin_fmaf(dinv[mt][acc_token_u<SPLIT>(v)] * scf, c[v], A.acc[mt][v]);
                }
            }
        }
    } else {  // Q8_0: 8 blocks of 32, one chunk each
        const h2 off = as_h2(0xE480E480u);  // (-1152, -1152): (1024 + (q^0x80)) - 1152 = q
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float d = half_bits(r.d[i]);
            const uint32_t t0 = r.w0[i] ^ 0x80808080u, t1 = r.w1[i] ^ 0x80808080u;
            const h2 p0 = as_h2(pair_lo(t0)) + off, p1 = as_h2(pair_hi(t0)) + off;
            const h2 p2 = as_h2(pair_lo(t1)) + off, p3 = as_h2(pair_hi(t1)) + off;
            h8 b;
            b[0] = p0[0]; b[1] = p0[1]; b[2] = p1[0]; b[3] = p1[1];
            b[4] = p2[0]; b[5] = p2[1]; b[6] = p3[0]; b[7] = p3[1];
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const h8 a = *(const h8 *)(a_lane + (i * MT + mt) * 1024);
                const f4 c = mfma32(a, b, f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                for (int v = 0; v < 4; v++)
                    A.acc[mt][v] = __builtin_fmaf(d * inv[mt][acc_token_u<SPLIT>(v)], c[v], A.acc[mt][v]);
            }
        }
    }
}

// ---------------------------------------------------------------- prep
// A-operand layout of one unit: entry (chunk c, tile mt, lane l) holds
// LANE_HALVES fp16 values for token slot l%16 and lane group G = l/16. Which
// unit elements an entry holds depends on the weight format (LK):
//  LK 0 (Q4_K, Q5_K; chunk = MFMA m): items e = 0..7 are elements
//       128(m>>2) + 64(G>>1) + 32((m>>1)&1) + 16(G&1) + 8(m&1) + e
//  LK 1 (Q6_K; chunk = 16-element sub-block s): items e = 0..3 are 16s + 4G + e
//  LK 2 (Q8_0; chunk = 32-element block b): items e < 4 are 32b + 4G + e,
//       items e >= 4 are 32b + 16 + 4G + (e - 4)
template <int LK> struct Layout {
    static constexpr int ENTRY = LK == 1 ? 8 : 16;  // bytes per lane entry
};

// Grid (units, token blocks of 8). Thread (tl = tid/32, gi = tid%32) owns
// elements [8 gi, 8 gi + 8) of unit blockIdx.x for token blockIdx.y*8 + tl.
// Padding tokens (M <= t < TOK) get zero operands and unit scale.
template <int LK, int MT, bool SPLIT, bool MINS>
__global__ __launch_bounds__(256) void prep_kernel(const float *__restrict__ X, int M, int K,
                                                   uint8_t *__restrict__ afrag, float *__restrict__ xs,
                                                   float *__restrict__ inv) {
    constexpr int TOK = MT * (SPLIT ? 8 : 16);
    constexpr int ENTRY = Layout<LK>::ENTRY;
    const int u = blockIdx.x, tid = threadIdx.x;
    const int tl = tid >> 5, gi = tid & 31;
    const int t = blockIdx.y * 8 + tl;
    const int k = u * UNIT + gi * 8;
    float v[8];
    if (t < M && k < K) {
        const float4 a = *(const float4 *)(X + (size_t)t * K + k);
        const float4 b = *(const float4 *)(X + (size_t)t * K + k + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = 0.f;
    }
    float mx = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) mx = fmaxf(mx, fabsf(v[e]));
    float sm = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    // token max over the 32 threads of this token (one half-wave)
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    // sub-block (32 elements = 4 threads) sums
    sm += __shfl_xor(sm, 1);
    sm += __shfl_xor(sm, 2);
    int e2 = 0;
    if (mx > 0.f && mx < __builtin_huge_valf()) {
        int ex;
        frexpf(mx, &ex);  // mx = f * 2^ex, f in [0.5, 1)
        e2 = min(max(15 - ex, -120), 120);
    }
    const float scale = ldexpf(1.f, e2);
    if (t >= TOK) return;
    if (gi == 0) inv[(size_t)u * TOK + t] = ldexpf(1.f, -e2);
    if (MINS && (gi & 3) == 0) xs[((size_t)u * 8 + (gi >> 2)) * TOK + t] = sm;
    const int mt = SPLIT ? t / 8 : t / 16;
    const int slot = SPLIT ? (t % 8) * 2 : t % 16;
    _Float16 hi[8], lo[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float xsc = v[e] * scale;
        hi[e] = (_Float16)xsc;
        lo[e] = (_Float16)(xsc - (float)hi[e]);
    }
    uint8_t *base = afrag + (size_t)u * UNIT_A1 * MT;
    // two runs of 4 elements: run p covers elements 8 gi + 4p .. + 3
#pragma unroll
    for (int p = 0; p < 2; p++) {
        int c, G, item;
        if constexpr (LK == 0) {
            c = (gi & 1) + 2 * ((gi >> 2) & 1) + 4 * ((gi >> 4) & 1);
            G = ((gi >> 1) & 1) + 2 * ((gi >> 3) & 1);
            item = 4 * p;
        } else if constexpr (LK == 1) {
            c = gi >> 1;
            G = 2 * (gi & 1) + p;
            item = 0;
        } else {
            const int q = gi & 3;  // 8-element group inside the 32-element block
            c = gi >> 2;
            G = 2 * (q & 1) + p;
            item = q < 2 ? 0 : 4;
        }
        h4 H, L;
#pragma unroll
        for (int e = 0; e < 4; e++) { H[e] = hi[4 * p + e]; L[e] = lo[4 * p + e]; }
        uint8_t *dst = base + ((size_t)(c * MT + mt) * 64 + G * 16 + slot) * ENTRY + item * 2;
        *(h4 *)dst = H;
        if (SPLIT) *(h4 *)(dst + ENTRY) = L;  // slot + 1
    }
}

// ---------------------------------------------------------------- gemm
// Persistent streaming: workgroup (w, s) keeps the prepared activations of
// K-slice s in LDS and walks the row groups w, w + G, w + 2G, ... (G =
// gridDim.x). Each wave owns 16 rows of every row group and streams the
// (row group, unit) items through a ring of RING units whose loads are issued
// RING - 1 items ahead, across row-group boundaries.
template <int QT, int MT> struct Ring { static constexpr int R = (QT == QT_Q6_K && MT >= 3) ? 2 : 4; };

template <int QT, int MT, bool SPLIT>
__global__ __launch_bounds__(WG_THREADS)
void gemm_q_kernel(const uint8_t *__restrict__ W, float *__restrict__ Y, int M, int N, int K, int ups, int S,
                   int accum, const uint8_t *__restrict__ afrag, const float *__restrict__ xs,
                   const float *__restrict__ invs, float *__restrict__ part) {
    using C = GemmCfg<QT>;
    constexpr int TOK = MT * (SPLIT ? 8 : 16);
    constexpr int TPL = Acc<MT, SPLIT>::TPL;
    constexpr int UNIT_A = UNIT_A1 * MT;
    constexpr int UNIT_BYTES = (QT == QT_Q8_0) ? 8 * 34 : C::BB;
    constexpr int R = Ring<QT, MT>::R;
    extern __shared__ __align__(16) uint8_t smem[];

    const int n_units = (K + UNIT - 1) / UNIT;
    const int u0 = blockIdx.y * ups;
    const int nu = min(ups, n_units - u0);
    const size_t row_bytes = (size_t)(K / C::QK) * C::BB;
    const int tail_blk = (QT == QT_Q8_0 && (K % UNIT)) ? (K % UNIT) / 32 : 8;
    const int rowgroups = (N + ROWS_PER_WG - 1) / ROWS_PER_WG;
    const int G = gridDim.x;
    const int n_rg = blockIdx.x < rowgroups ? (rowgroups - 1 - blockIdx.x) / G + 1 : 0;
    const int n_items = n_rg * nu;

    uint8_t *a_lds = smem;                                      // [ups][UNIT_A]
    float *x_lds = (float *)(smem + (size_t)ups * UNIT_A);      // [ups][8][TOK]
    float *i_lds = x_lds + (C::MINS ? ups * 8 * TOK : 0);       // [ups][TOK]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n_in = lane & 15, g = lane >> 4;
    // weight bytes of item it (row group blockIdx.x + G*(it/nu), unit u0 + it%nu)
    auto item_ptr = [&](int it) {
        const int rg = blockIdx.x + G * (it / nu);
        const int row = min(rg * ROWS_PER_WG + wave * 16 + n_in, N - 1);
        return W + (size_t)row * row_bytes + (size_t)(u0 + it % nu) * UNIT_BYTES;
    };
    auto item_nblk = [&](int it) { return (u0 + it % nu == n_units - 1) ? tail_blk : 8; };

    // 1. start streaming this lane's weights
    Unit<QT> buf[R];
#pragma unroll
    for (int p = 0; p < R - 1; p++)
        if (p < n_items) load_unit<QT>(item_ptr(p), g, item_nblk(p), buf[p]);

    // 2. copy this slice's prepared activations into LDS (one round of loads)
    {
        const uint4 *src = (const uint4 *)(afrag + (size_t)u0 * UNIT_A);
        uint4 *dst = (uint4 *)a_lds;
        const int n16 = nu * (UNIT_A / 16);
        for (int i0 = 0; i0 < n16; i0 += WG_THREADS * 8) {
            uint4 tmp[8];
#pragma unroll
            for (int j = 0; j < 8; j++) tmp[j] = src[min(i0 + j * WG_THREADS + tid, n16 - 1)];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int i = i0 + j * WG_THREADS + tid;
                if (i < n16) dst[i] = tmp[j];
            }
        }
        if constexpr (C::MINS)
            for (int i = tid; i < nu * 8 * TOK; i += WG_THREADS) x_lds[i] = xs[(size_t)u0 * 8 * TOK + i];
        for (int i = tid; i < nu * TOK; i += WG_THREADS) i_lds[i] = invs[(size_t)u0 * TOK + i];
    }
    __syncthreads();

    // 3. stream items through the MFMA pipe; a row group's epilogue follows
    //    its last unit
    Acc<MT, SPLIT> A;
    auto reset = [&]() {
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            A.acc[mt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < TPL; u++) A.macc[mt][u] = 0.f;
        }
    };
    reset();
    const uint8_t *a_lane = a_lds + lane * (QT == QT_Q6_K ? 8 : 16);
    for (int ib = 0; ib < n_items; ib += R) {
#pragma unroll
        for (int p = 0; p < R; p++) {
            const int it = ib + p;
            if (it < n_items) {
                const int nxt = it + R - 1;
                if (nxt < n_items) load_unit<QT>(item_ptr(nxt), g, item_nblk(nxt), buf[(p + R - 1) % R]);
                const int uu = it % nu;
                finish_unit<QT>(buf[p]);
                compute_unit<QT, MT, SPLIT>(buf[p], a_lane + (size_t)uu * UNIT_A, x_lds + (size_t)uu * 8 * TOK,
                                            i_lds + (size_t)uu * TOK, g, A);
                if (uu == nu - 1) {
                    // epilogue: lane values are rows row0 + n_in, tokens lane_token(mt, g, u)
                    const int rg = blockIdx.x + G * (it / nu);
                    const int r = rg * ROWS_PER_WG + wave * 16 + n_in;
                    if (r < N) {
#pragma unroll
                        for (int mt = 0; mt < MT; mt++)
#pragma unroll
                            for (int u = 0; u < TPL; u++) {
                                const int t = lane_token<SPLIT>(mt, g, u);
                                if (t >= M) continue;
                                float v = SPLIT ? (A.acc[mt][2 * u] + A.acc[mt][2 * u + 1]) : A.acc[mt][u];
                                if constexpr (C::MINS) v = v - A.macc[mt][u];
                                if (S == 1) {
                                    float *dst = Y + (size_t)t * N + r;
                                    *dst = accum ? *dst + v : v;
                                } else {
                                    part[((size_t)blockIdx.y * M + t) * N + r] = v;
                                }
                            }
                    }
                    reset();
                }
            }
        }
    }
}

// Y[i] (+)= sum_s part[s][i] in slice order, i over M*N outputs.
__global__ __launch_bounds__(256) void reduce_kernel(const float *__restrict__ part, float *__restrict__ Y,
                                                     int S, int64_t MN, int accum) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= MN) return;
    if (i + 4 <= MN && (MN & 3) == 0) {
        float4 s = *(const float4 *)(part + i);
        for (int sl = 1; sl < S; sl++) {
            const float4 v = *(const float4 *)(part + (size_t)sl * MN + i);
            s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
        }
        float4 *dst = (float4 *)(Y + i);
        if (accum) {
            const float4 y = *dst;
            s.x += y.x; s.y += y.y; s.z += y.z; s.w += y.w;
        }
        *dst = s;
    } else {
        for (int64_t j = i; j < min(i + 4, MN); j++) {
            float s = part[j];
            for (int sl = 1; sl < S; sl++) s += part[(size_t)sl * MN + j];
            Y[j] = accum ? Y[j] + s : s;
        }
    }
}

template <int QT, int MT, bool SPLIT>
hipError_t launch_t(const uint8_t *W, const float *X, float *Y, int M, int N, int K, int ups, int S, int G, int accum,
                    uint8_t *afrag, float *xs, float *inv, float *part, hipStream_t st) {
    using C = GemmCfg<QT>;
    constexpr int TOK = MT * (SPLIT ? 8 : 16);
    const int n_units = (K + UNIT - 1) / UNIT;
    prep_kernel<QT == QT_Q6_K ? 1 : QT == QT_Q8_0 ? 2 : 0, MT, SPLIT, C::MINS><<<dim3(n_units, TOK / 8), 256, 0, st>>>(X, M, K, afrag, xs, inv);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const size_t lds = (size_t)ups * UNIT_A1 * MT + (C::MINS ? (size_t)ups * 8 * TOK * 4 : 0) + (size_t)ups * TOK * 4;
    if (lds > 65536) {
        e = hipFuncSetAttribute((const void *)gemm_q_kernel<QT, MT, SPLIT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds);
        if (e != hipSuccess) return e;
    }
    gemm_q_kernel<QT, MT, SPLIT><<<dim3(G, S), WG_THREADS, lds, st>>>(W, Y, M, N, K, ups, S, accum, afrag, xs, inv,
                                                                     part);
    e = hipGetLastError();
    if (e != hipSuccess || S == 1) return e;
    const int64_t MN = (int64_t)M * N;
    reduce_kernel<<<(unsigned)((MN + 1023) / 1024), 256, 0, st>>>(part, Y, S, MN, accum);
    return hipGetLastError();
}

}  // namespace

// ---------------------------------------------------------------- host plan
struct GemmPlan {
    bool split;      // fp32-accurate two-limb mode
    int MT;          // MFMA token tiles (16 slots each)
    int ups;         // 256-element units per K-slice
    int S;           // K-slices (grid.y)
    int G;           // persistent workgroups per K-slice (grid.x)
    size_t off_xs, off_inv, off_part, ws_bytes;
};

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    return v ? atoi(v) : dflt;
}

static GemmPlan plan_gemm(int qt, int M, int N, int K, int flags) {
    GemmPlan p{};
    const bool force_f32 = flags & 1, force_half = flags & 2;
    p.split = force_f32 ? true : force_half ? false : (M < 16);
    p.MT = p.split ? (M + 7) / 8 : (M + 15) / 16;
    const int n_units = (K + UNIT - 1) / UNIT;
    const int rowgroups = (N + ROWS_PER_WG - 1) / ROWS_PER_WG;
    // tuning overrides: IHIP_GEMM_LDS_A (A-operand bytes per workgroup),
    // IHIP_GEMM_WGS (target resident workgroups)
    static const int lds_a = env_int("IHIP_GEMM_LDS_A", 32768);
    static const int target = env_int("IHIP_GEMM_WGS", 1024);
    const int ups_max = std::max(1, lds_a / (UNIT_A1 * p.MT));
    p.S = (n_units + ups_max - 1) / ups_max;
    p.ups = (n_units + p.S - 1) / p.S;
    p.S = (n_units + p.ups - 1) / p.ups;
    p.G = std::max(1, std::min(rowgroups, (target + p.S - 1) / p.S));
    const int TOK = p.MT * (p.split ? 8 : 16);
    const bool mins = (qt == QT_Q4_K || qt == QT_Q5_K);
    size_t o = align256((size_t)n_units * UNIT_A1 * p.MT);
    p.off_xs = o;
    o += mins ? align256((size_t)n_units * 8 * TOK * 4) : 0;
    p.off_inv = o;
    o += align256((size_t)n_units * TOK * 4);
    p.off_part = o;
    o += p.S > 1 ? align256((size_t)p.S * M * N * 4) : 0;
    p.ws_bytes = o;
    return p;
}

// Largest per-launch token count: fp32-accurate batches above 32 tokens run
// as two launches over token halves.
static int launch_m(int M, int flags) {
    const bool split = (flags & 1) ? true : (flags & 2) ? false : (M < 16);
    return (split && M > 32) ? 32 : M;
}

size_t gemm_ws_bytes(int qt, int M, int N, int K, int flags) {
    const int m0 = launch_m(M, flags);
    const int f = (m0 != M) ? (flags | 1) : flags;
    return plan_gemm(qt, m0, N, K, f).ws_bytes;
}

template <int QT>
static hipError_t dispatch_mt(const GemmPlan &p, const uint8_t *W, const float *X, float *Y, int M, int N, int K,
                              int accum, uint8_t *ws, hipStream_t st) {
    float *xs = (float *)(ws + p.off_xs), *inv = (float *)(ws + p.off_inv), *part = (float *)(ws + p.off_part);
#define L(mt, sp) return launch_t<QT, mt, sp>(W, X, Y, M, N, K, p.ups, p.S, p.G, accum, ws, xs, inv, part, st)
    if (p.split) {
        switch (p.MT) {
        case 1: L(1, true); case 2: L(2, true); case 3: L(3, true); case 4: L(4, true);
        }
    } else {
        switch (p.MT) {
        case 1: L(1, false); case 2: L(2, false); case 3: L(3, false); case 4: L(4, false);
        }
    }
#undef L
    return hipErrorInvalidValue;
}

hipError_t launch_gemm(int qt, const void *W, const float *X, float *Y, int M, int N, int K, int flags, void *ws,
                       hipStream_t st) {
    const int m0 = launch_m(M, flags);
    if (m0 != M) {
        hipError_t e = launch_gemm(qt, W, X, Y, m0, N, K, flags | 1, ws, st);
        if (e != hipSuccess) return e;
        return launch_gemm(qt, W, X + (size_t)m0 * K, Y + (size_t)m0 * N, M - m0, N, K, flags | 1, ws, st);
    }
    const GemmPlan p = plan_gemm(qt, M, N, K, flags);
    const int accum = (flags & 4) ? 1 : 0;
    const uint8_t *w = (const uint8_t *)W;
    uint8_t *wsp = (uint8_t *)ws;
    switch (qt) {
    case QT_Q4_K: return dispatch_mt<QT_Q4_K>(p, w, X, Y, M, N, K, accum, wsp, st);
    case QT_Q5_K: return dispatch_mt<QT_Q5_K>(p, w, X, Y, M, N, K, accum, wsp, st);
    case QT_Q6_K: return dispatch_mt<QT_Q6_K>(p, w, X, Y, M, N, K, accum, wsp, st);
    case QT_Q8_0: return dispatch_mt<QT_Q8_0>(p, w, X, Y, M, N, K, accum, wsp, st);
    }
    return hipErrorInvalidValue;
}
