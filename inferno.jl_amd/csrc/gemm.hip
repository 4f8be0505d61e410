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
#include "chain.h"

#include <algorithm>
#include <cstdlib>

namespace {

constexpr int WG_THREADS = 256;  // 4 waves
constexpr int ROWS_PER_WG = 64;
constexpr int UNIT = 256;        // K elements per loop unit
constexpr int UNIT_A1 = 8192;    // A-operand bytes per unit and 16-slot token tile
constexpr int CHAIN_MAX_TILES = 32;  // 16-row tiles per workgroup of a chained producer

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
//  Q6_K: after a 4x4 transpose across lane groups, a/b/c[i] hold the dwords
//        ql[64n + 16h + 4g], ql[64n + 32 + 16h + 4g], qh[32n + 16h + 4g]
//        for i = 2n + h, which finish_unit regroups to the decoder's words
//        (q6_regroup); sc all 16 scales; d the fp16 super-scale
//  Q8_0: w0/w1[b] hold qs dwords g and 4 + g of block b (transposed), d[b]
template <int QT> struct Unit;
template <> struct Unit<QT_Q4_K> { uint4 hdr, q0, q1; };
template <> struct Unit<QT_Q5_K> { uint4 hdr, q0, q1, qh; };
template <> struct Unit<QT_Q6_K> { uint32_t a[4], b[4], c[4]; uint4 sc; uint32_t d; };
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

// Q6_K words of one lane and group, from GGUF order (a, b = ql dwords
// ql[p, +4), ql[p + 32, +4), h = the qh dword qh[p', +4) of the same four
// elements j: byte j of each) to the order q6_pairs decodes. Pair 2 qq + t
// is elements 2t, 2t + 1 of sub-block qq (the 6-bit value of element j of
// sub-block qq is nibble qq>>1 of byte j of a (qq even) or b, with bits
// 2qq, 2qq + 1 of byte j of h above it), at bits o..o+5 (element 2t) and
// 16+o..21+o (element 2t + 1) of one word:
//   A: pair 0 at o = 0, pair 1 at o = 6, the low nibbles of pair 6 at o = 12
//   B: pair 2 at 0, pair 3 at 6, the low nibbles of pair 7 at 12
//   C: pair 4 at 0, the high 2 bits of pair 6 at 6 and of pair 7 at 8,
//      pair 5 at 10
// The same bits, rearranged (the packer stores them so; the GGUF-layout
// loader regroups after its transposes).
__host__ __device__ inline void q6_regroup(uint32_t a, uint32_t b, uint32_t h, uint32_t &A, uint32_t &B,
                                           uint32_t &C) {
    const uint32_t q0 = (a & 0x0f0f0f0fu) | ((h & 0x03030303u) << 4);  // (one 6-bit value a byte)
    const uint32_t q1 = (b & 0x0f0f0f0fu) | (((h >> 2) & 0x03030303u) << 4);
    const uint32_t q2 = ((a >> 4) & 0x0f0f0f0fu) | (((h >> 4) & 0x03030303u) << 4);
    const uint32_t q3 = ((b >> 4) & 0x0f0f0f0fu) | (((h >> 6) & 0x03030303u) << 4);
    // pair t of a byte word: bytes 2t, 2t + 1 at bits 0 and 16
    auto pr = [](uint32_t q, int t) {
        return t ? ((q >> 16) & 0xffu) | ((q >> 8) & 0xff0000u) : (q & 0xffu) | ((q << 8) & 0xff0000u);
    };
    A = pr(q0, 0) | (pr(q0, 1) << 6) | ((pr(q3, 0) & 0x000f000fu) << 12);
    B = pr(q1, 0) | (pr(q1, 1) << 6) | ((pr(q3, 1) & 0x000f000fu) << 12);
    C = pr(q2, 0) | (((pr(q3, 0) >> 4) & 0x00030003u) << 6) | (((pr(q3, 1) >> 4) & 0x00030003u) << 8) |
        (pr(q2, 1) << 10);
}

// The eight weight pairs q - 32 (exact fp16) of one group's words A, B, C
// (q6_regroup's order): a mask-and-or puts a 6-bit field at bits 0..5 under
// the fp16 exponent 0x6400 (1024 + q, pairs 0-5, one shift first for a field
// above bit 0); for pairs 6 and 7 one byte permute puts the low nibbles at
// bits 4..7 and the high bits at 8..9 (1024 + 16 q), another mask-and-or
// keeps those. 14 bit operations for 8 pairs (GGUF order: 29).
__device__ __forceinline__ void q6_pairs(uint32_t A, uint32_t B, uint32_t C, h2 (&p)[8]) {
    uint32_t ex = 0x64006400u;
    asm("" : "+v"(ex));  // (a VGPR: see k_frag)
    const uint32_t m6 = 0x003f003fu, m46 = 0x03f003f0u;
    const h2 off = as_h2(0xE420E420u);                                  // (1024 + q) - 1056
    const h2 s16 = as_h2(0x2C002C00u), off16 = as_h2(0xD600D600u);      // (1024 + 16 q) / 16 - 96
    p[0] = as_h2((A & m6) | ex) + off;
    p[1] = as_h2(((A >> 6) & m6) | ex) + off;
    p[2] = as_h2((B & m6) | ex) + off;
    p[3] = as_h2(((B >> 6) & m6) | ex) + off;
    p[4] = as_h2((C & m6) | ex) + off;
    p[5] = as_h2(((C >> 10) & m6) | ex) + off;
    // bytes (A1, C'1, A3, C'3) with C' = C << 2, and (B1, C1, B3, C3)
    p[6] = __builtin_elementwise_fma(as_h2((__builtin_amdgcn_perm(A, C << 2, 0x03070105u) & m46) | ex), s16, off16);
    p[7] = __builtin_elementwise_fma(as_h2((__builtin_amdgcn_perm(B, C, 0x03070105u) & m46) | ex), s16, off16);
}

// Raw loads (issued early); finish_unit() applies the cross-lane transposes
// (and the Q4_K byte order of k_frag) right before use. u: first byte of the unit in this lane's row; nblk: Q8_0
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
        r.c[0] = H.x; r.c[1] = H.y; r.c[2] = H.z; r.c[3] = H.w;
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
    if constexpr (QT == QT_Q4_K) {
        // GGUF byte order to the order the decoder reads: bytes 1 and 2 of
        // each quant dword swapped (the packer stores them so)
        const uint32_t sel = 0x03010200u;
        r.q0 = make_uint4(__builtin_amdgcn_perm(r.q0.x, r.q0.x, sel), __builtin_amdgcn_perm(r.q0.y, r.q0.y, sel),
                          __builtin_amdgcn_perm(r.q0.z, r.q0.z, sel), __builtin_amdgcn_perm(r.q0.w, r.q0.w, sel));
        r.q1 = make_uint4(__builtin_amdgcn_perm(r.q1.x, r.q1.x, sel), __builtin_amdgcn_perm(r.q1.y, r.q1.y, sel),
                          __builtin_amdgcn_perm(r.q1.z, r.q1.z, sel), __builtin_amdgcn_perm(r.q1.w, r.q1.w, sel));
    } else if constexpr (QT == QT_Q6_K) {
        xpose4(r.a[0], r.a[1], r.a[2], r.a[3]);
        xpose4(r.b[0], r.b[1], r.b[2], r.b[3]);
        xpose4(r.c[0], r.c[1], r.c[2], r.c[3]);
#pragma unroll
        for (int i = 0; i < 4; i++) q6_regroup(r.a[i], r.b[i], r.c[i], r.a[i], r.b[i], r.c[i]);
    } else if constexpr (QT == QT_Q8_0) {
        // before: (w0[2k], w1[2k], w0[2k+1], w1[2k+1]) = dwords 0..3 of this
        // lane group's half-block; after: dword g of each of the 4 halves
#pragma unroll
        for (int k = 0; k < 4; k++) xpose4(r.w0[2 * k], r.w1[2 * k], r.w0[2 * k + 1], r.w1[2 * k + 1]);
    }
}

// ---------------------------------------------------------------- packed weights
// Tile-contiguous layout: the 16 rows x 256 K-elements of tile t, unit u form
// one chunk of CHUNK = 16 * UB bytes at (t * n_units + u) * CHUNK, arranged so
// that lane l = n + 16 g (row n, lane group g) fetches exactly its operand
// bytes with 16-byte loads at i * 1024 + 16 l plus per-row header loads. Every
// load of a wave then covers whole cache lines, and no cross-lane transposes
// remain. Byte map (row n of the tile, offsets into the GGUF block):
//  Q4_K (2304 B): [1024 i + 16 l, +16) = qs[64 i + 16 g, +16) (i = 0, 1)
//                 with bytes 1 and 2 of each dword swapped (the order
//                 k_frag decodes); [2048 + 16 n, +16) = d, dmin, scales
//  Q5_K (2816 B): quants as Q4_K; [2048 + 16 (n + 16 h), +16) = qh[16 h, +16)
//                 (h = 0, 1); [2560 + 16 n, +16) = d, dmin, scales
//  Q6_K (3360 B): for i = 0..3, p = 64 (i>>1) + 16 (i&1) + 4 g, the
//                 dwords ql[p, +4), ql[p + 32, +4), qh[32 (i>>1) + 16 (i&1)
//                 + 4 g, +4) regrouped (q6_regroup) to words A, B, C at
//                 [16 l + 4 i], [1024 + 16 l + 4 i], [2048 + 16 l + 4 i];
//                 [3072 + 16 n, +16) = scales; [3328 + 2 n, +2) = d
//  Q8_0 (4352 B): [1024 i + 16 l + 8 j + 4 h, +4) = qs dword (g + 4 h) of
//                 block 2 i + j (i = 0..3; j, h = 0, 1); [4096 + 16 n + 2 b,
//                 +2) = d of block b
// Rows past N and Q8_0 blocks past K are zero bytes: they contribute zero.
template <int QT> struct Packed {
    static constexpr int UB = (QT == QT_Q8_0) ? 8 * 34 : QTraits<QT>::BB;
    static constexpr int CHUNK = 16 * UB;
};

template <int QT>
__device__ __forceinline__ void load_unit_packed(const uint8_t *__restrict__ ch, int lane, Unit<QT> &r) {
    const int n = lane & 15;
    if constexpr (QT == QT_Q4_K || QT == QT_Q5_K) {
        r.q0 = *(const uint4 *)(ch + 16 * lane);
        r.q1 = *(const uint4 *)(ch + 1024 + 16 * lane);
        if constexpr (QT == QT_Q5_K) {
            r.qh = *(const uint4 *)(ch + 2048 + 16 * (n + 16 * ((lane >> 4) & 1)));
            r.hdr = *(const uint4 *)(ch + 2560 + 16 * n);
        } else {
            r.hdr = *(const uint4 *)(ch + 2048 + 16 * n);
        }
    } else if constexpr (QT == QT_Q6_K) {
        const uint4 A = *(const uint4 *)(ch + 16 * lane);
        const uint4 B = *(const uint4 *)(ch + 1024 + 16 * lane);
        const uint4 H = *(const uint4 *)(ch + 2048 + 16 * lane);
        r.a[0] = A.x; r.a[1] = A.y; r.a[2] = A.z; r.a[3] = A.w;
        r.b[0] = B.x; r.b[1] = B.y; r.b[2] = B.z; r.b[3] = B.w;
        r.c[0] = H.x; r.c[1] = H.y; r.c[2] = H.z; r.c[3] = H.w;
        r.sc = *(const uint4 *)(ch + 3072 + 16 * n);
        r.d = ld_u16(ch + 3328 + 2 * n);
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 v = *(const uint4 *)(ch + 1024 * i + 16 * lane);
            r.w0[2 * i] = v.x; r.w1[2 * i] = v.y; r.w0[2 * i + 1] = v.z; r.w1[2 * i + 1] = v.w;
        }
        const uint4 dv = *(const uint4 *)(ch + 4096 + 16 * n);
        const uint32_t dw[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
        for (int b = 0; b < 8; b++) r.d[b] = (dw[b >> 1] >> (16 * (b & 1))) & 0xffffu;
    }
}

// The same lane bytes through a buffer resource over the packed matrix: the
// chunk offset is wave-uniform (a scalar operand), the lane offsets are fixed
// per lane, so a load needs no per-item vector address arithmetic. Loads
// past the resource's size return zero.
__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t rs, int voff, int soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}

template <int QT>
__device__ __forceinline__ void load_unit_buf(__amdgpu_buffer_rsrc_t rs, int soff, int lane, Unit<QT> &r) {
    const int n = lane & 15, l16 = 16 * lane, n16 = 16 * n;
    if constexpr (QT == QT_Q4_K || QT == QT_Q5_K) {
        r.q0 = bload16(rs, l16, soff);
        r.q1 = bload16(rs, l16 + 1024, soff);
        if constexpr (QT == QT_Q5_K) {
            r.qh = bload16(rs, 2048 + 16 * (n + 16 * ((lane >> 4) & 1)), soff);
            r.hdr = bload16(rs, n16 + 2560, soff);
        } else {
            r.hdr = bload16(rs, n16 + 2048, soff);
        }
    } else if constexpr (QT == QT_Q6_K) {
        const uint4 A = bload16(rs, l16, soff);
        const uint4 B = bload16(rs, l16 + 1024, soff);
        const uint4 H = bload16(rs, l16 + 2048, soff);
        r.a[0] = A.x; r.a[1] = A.y; r.a[2] = A.z; r.a[3] = A.w;
        r.b[0] = B.x; r.b[1] = B.y; r.b[2] = B.z; r.b[3] = B.w;
        r.c[0] = H.x; r.c[1] = H.y; r.c[2] = H.z; r.c[3] = H.w;
        r.sc = bload16(rs, n16 + 3072, soff);
        r.d = __builtin_amdgcn_raw_buffer_load_b16(rs, 3328 + 2 * n, soff, 0);
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 v = bload16(rs, l16 + 1024 * i, soff);
            r.w0[2 * i] = v.x; r.w1[2 * i] = v.y; r.w0[2 * i + 1] = v.z; r.w1[2 * i + 1] = v.w;
        }
        const uint4 dv = bload16(rs, n16 + 4096, soff);
        const uint32_t dw[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
        for (int b = 0; b < 8; b++) r.d[b] = (dw[b >> 1] >> (16 * (b & 1))) & 0xffffu;
    }
}

// One thread per (unit, tile, lane): copies that lane's bytes of the chunk.
// gated > 0: W is a [gate; up] matrix of 2 gated rows and tile t holds gate
// rows 8t .. 8t + 7 followed by the same up rows (row gated + 8t + n - 8 for
// n >= 8), the layout a chained EPI_GATE epilogue reads.
template <int QT>
__global__ __launch_bounds__(64) void pack_kernel(const uint8_t *__restrict__ W, int N, int K,
                                                  uint8_t *__restrict__ P, int gated) {
    constexpr int BB = QTraits<QT>::BB;
    const int n_units = (K + UNIT - 1) / UNIT;
    const int u = blockIdx.x, tile = blockIdx.y;
    const int l = threadIdx.x, n = l & 15, g = l >> 4;
    const int row = gated > 0 ? (n < 8 ? 8 * tile + n : gated + 8 * tile + n - 8) : tile * 16 + n;
    const bool live = gated > 0 ? 8 * tile + (n & 7) < gated : row < N;
    const size_t row_bytes = (size_t)(K / QTraits<QT>::QK) * BB;
    uint8_t *ch = P + ((size_t)tile * n_units + u) * Packed<QT>::CHUNK;
    const uint8_t *src = W + (size_t)(live ? row : 0) * row_bytes + (size_t)u * Packed<QT>::UB;
    auto cp = [&](uint8_t *dst, const uint8_t *s, int nbytes, bool ok) {
        for (int e = 0; e < nbytes; e++) dst[e] = ok ? s[e] : (uint8_t)0;
    };
    if constexpr (QT == QT_Q4_K) {
        for (int i = 0; i < 2; i++)
            for (int e = 0; e < 16; e++) {
                const int se = (e & 12) | ((e & 3) == 1 ? 2 : (e & 3) == 2 ? 1 : (e & 3));  // bytes 1, 2 swapped
                ch[1024 * i + 16 * l + e] = live ? src[16 + 64 * i + 16 * g + se] : (uint8_t)0;
            }
        if (g == 0) cp(ch + 2048 + 16 * n, src, 16, live);
    } else if constexpr (QT == QT_Q5_K) {
        for (int i = 0; i < 2; i++) cp(ch + 1024 * i + 16 * l, src + 48 + 64 * i + 16 * g, 16, live);
        if (g < 2) cp(ch + 2048 + 16 * (n + 16 * g), src + 16 + 16 * g, 16, live);
        if (g == 0) cp(ch + 2560 + 16 * n, src, 16, live);
    } else if constexpr (QT == QT_Q6_K) {
        auto dw = [&](const uint8_t *s) {  // (little-endian; rows are not 4-byte aligned)
            return live ? (uint32_t)s[0] | ((uint32_t)s[1] << 8) | ((uint32_t)s[2] << 16) | ((uint32_t)s[3] << 24) : 0u;
        };
        for (int i = 0; i < 4; i++) {
            const int p = 64 * (i >> 1) + 16 * (i & 1) + 4 * g;
            uint32_t w[3];
            q6_regroup(dw(src + p), dw(src + p + 32), dw(src + 128 + 32 * (i >> 1) + 16 * (i & 1) + 4 * g), w[0], w[1],
                       w[2]);
            for (int k = 0; k < 3; k++)
                for (int e = 0; e < 4; e++) ch[1024 * k + 16 * l + 4 * i + e] = (uint8_t)(w[k] >> (8 * e));
        }
        if (g == 0) {
            cp(ch + 3072 + 16 * n, src + 192, 16, live);
            cp(ch + 3328 + 2 * n, src + 208, 2, live);
        }
    } else {
        const int nblk = min(8, K / 32 - 8 * u);  // blocks of this unit inside the row
        for (int i = 0; i < 4; i++)
            for (int j = 0; j < 2; j++)
                for (int h = 0; h < 2; h++) {
                    const int b = 2 * i + j;
                    cp(ch + 1024 * i + 16 * l + 8 * j + 4 * h, src + 34 * b + 2 + 4 * (g + 4 * h), 4, live && b < nblk);
                }
        if (g == 0)
            for (int b = 0; b < 8; b++) cp(ch + 4096 + 16 * n + 2 * b, src + 34 * b, 2, live && b < nblk);
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

// Exact fp16 pair of v / 16 for a small non-negative integer v (< 1024):
// 64 + v / 16 has ulp 1/16, so the subtraction rounds nothing.
__device__ __forceinline__ h2 h2_of_small_16th(uint32_t v) {
    const uint32_t b = 0x5400u | v;
    return as_h2(b | (b << 16)) - as_h2(0x54005400u);
}

// Per-lane scales of a Q4_K/Q5_K unit (lane group g): hs[2 ah + b] is the
// 6-bit scale sc of sub-block 4 ah + 2 (g >> 1) + b as an exact fp16 pair
// (sc / 16 for the Q4_K high nibble plane, b = 1: see k_frag), ns = -1024 hs;
// m_lo / m_hi hold the 6-bit mins of sub-blocks 0..3 / 4..7 as bytes.
struct KScales { h2 hs[4], ns[4]; uint32_t m_lo, m_hi; };

template <int QT>
__device__ __forceinline__ KScales k_scales(const uint4 &hdr, int g) {
    KScales k;
    const uint32_t s0 = hdr.y, s1 = hdr.z, s2 = hdr.w;
    const uint32_t sc_lo = s0 & 0x3f3f3f3fu;
    const uint32_t sc_hi = (s2 & 0x0f0f0f0fu) | (((s0 >> 6) & 0x03030303u) << 4);
    k.m_lo = s1 & 0x3f3f3f3fu;
    k.m_hi = ((s2 >> 4) & 0x0f0f0f0fu) | (((s1 >> 6) & 0x03030303u) << 4);
    const int sh = 16 * (g >> 1);
    k.hs[0] = h2_of_small((sc_lo >> sh) & 0xffu);
    k.hs[2] = h2_of_small((sc_hi >> sh) & 0xffu);
    if constexpr (QT == QT_Q4_K) {
        k.hs[1] = h2_of_small_16th((sc_lo >> (sh + 8)) & 0xffu);
        k.hs[3] = h2_of_small_16th((sc_hi >> (sh + 8)) & 0xffu);
    } else {
        k.hs[1] = h2_of_small((sc_lo >> (sh + 8)) & 0xffu);
        k.hs[3] = h2_of_small((sc_hi >> (sh + 8)) & 0xffu);
    }
    const h2 neg1024 = as_h2(0xE400E400u);
#pragma unroll
    for (int i = 0; i < 4; i++) k.ns[i] = k.hs[i] * neg1024;
    return k;
}

// B operand of MFMA m (0..7) of a Q4_K/Q5_K unit: from lane group g the 8
// elements 128(m>>2) + 64(g>>1) + 32((m>>1)&1) + 16(g&1) + 8(m&1) + e of
// sub-block 4(m>>2) + 2(g>>1) + ((m>>1)&1), i.e. the dwords 2(m&1), +1 of q0
// (m < 4) or q1, low nibbles for even (m>>1), high for odd, as exact fp16
// q * sc (fma(1024 + q, sc, -1024 sc) rounds nothing).
//  Q4_K: each quant dword holds the bytes of elements (0, 2, 1, 3) (the
//        packer and finish_unit swap bytes 1 and 2 of the GGUF dword), so a
//        mask-and-or puts the nibbles of elements 0 and 1 of either plane
//        under the fp16 exponent 0x6400, and the same after a shift by 8
//        those of elements 2 and 3: 5 bit operations per dword for both
//        planes instead of 7. The high plane sits at mantissa bits 4..7,
//        1024 + 16 q, against the scale sc / 16 (and -64 sc): the same exact
//        q * sc.
//  Q5_K: GGUF byte order; the plane's nibbles with the qh bit as bit 4,
//        widened to fp16 pairs by byte permutes.
template <int QT>
__device__ __forceinline__ h8 k_frag(const Unit<QT> &r, int m, int g, const KScales &k) {
    const int ah = m >> 2, b = (m >> 1) & 1, hw = m & 1;
    const uint4 Q = ah ? r.q1 : r.q0;
    const uint32_t x0 = hw ? Q.z : Q.x, x1 = hw ? Q.w : Q.y;
    const h2 s = k.hs[2 * ah + b], ns = k.ns[2 * ah + b];
    if constexpr (QT == QT_Q4_K) {
        // the exponent as a VGPR value: a VOP3 and-or has no literal slot and
        // reads at most one SGPR (the mask), so with two constants it would
        // split in two
        const uint32_t mk = b ? 0x00f000f0u : 0x000f000fu;
        uint32_t ex = 0x64006400u;
        asm("" : "+v"(ex));
        const h2 p0 = __builtin_elementwise_fma(as_h2((x0 & mk) | ex), s, ns);
        const h2 p1 = __builtin_elementwise_fma(as_h2(((x0 >> 8) & mk) | ex), s, ns);
        const h2 p2 = __builtin_elementwise_fma(as_h2((x1 & mk) | ex), s, ns);
        const h2 p3 = __builtin_elementwise_fma(as_h2(((x1 >> 8) & mk) | ex), s, ns);
        h8 f;
        f[0] = p0[0]; f[1] = p0[1]; f[2] = p1[0]; f[3] = p1[1];
        f[4] = p2[0]; f[5] = p2[1]; f[6] = p3[0]; f[7] = p3[1];
        return f;
    } else {
        uint32_t n0 = (b ? (x0 >> 4) : x0) & 0x0f0f0f0fu;
        uint32_t n1 = (b ? (x1 >> 4) : x1) & 0x0f0f0f0fu;
        const int hb = 4 * ah + 2 * (g >> 1) + b;  // bit 2j + b of qh[l]
        const uint32_t h0 = hw ? r.qh.z : r.qh.x, h1 = hw ? r.qh.w : r.qh.y;
        n0 |= ((h0 >> hb) & 0x01010101u) << 4;
        n1 |= ((h1 >> hb) & 0x01010101u) << 4;
        return b_frag_scaled(n0, n1, s, ns);
    }
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

// RMSNorm row scales rs[t] = 1 / sqrt(sum_u ssq[u][t] / K + eps) from the
// per-unit sums of squares the prep kernel left (1 without RMSNorm). The
// BT threads of the workgroup split the units, P = BT / TOK threads per
// token: issue() loads up to 4 units per thread (one round of independent
// loads, issued before the weight prologue so the latter need not wait for
// them), finish() adds a thread's units, then combines the P partial sums
// of each token in LDS in a fixed order. Ends with a barrier.
template <int TOK, int BT>
struct RowScales {
    static constexpr int P = BT / TOK;
    float q[4];
    __device__ __forceinline__ void issue(const float *__restrict__ ssq, int n_units, int tid) {
        const int t = tid % TOK, part = tid / TOK;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int u = part + i * P;
            q[i] = (ssq != nullptr && part < P && u < n_units) ? ssq[(size_t)u * TOK + t] : 0.f;
        }
    }
    __device__ __forceinline__ void finish(const float *__restrict__ ssq, int n_units, int K, float eps, int tid,
                                           float *rsp, float *rs) {
        const int t = tid % TOK, part = tid / TOK;
        float v = (q[0] + q[1]) + (q[2] + q[3]);
        if (ssq != nullptr && part < P)
            for (int u = part + 4 * P; u < n_units; u += P) v += ssq[(size_t)u * TOK + t];
        rsp[tid] = v;
        __syncthreads();
        if (tid < TOK) {
            float r = 1.0f;
            if (ssq != nullptr) {
                float sq = 0.f;
                for (int i = 0; i < P; i++) sq += rsp[i * TOK + tid];
                r = 1.0f / sqrtf(sq / (float)K + eps);
            }
            rs[tid] = r;
        }
        __syncthreads();
    }
};

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
        // MFMA m (0..7) of the unit takes from lane group g the elements k_frag names
        const float d = half_bits(r.hdr.x), dmin = half_bits(r.hdr.x >> 16);
        const KScales ks = k_scales<QT>(r.hdr, g);
        const uint32_t m_lo = ks.m_lo, m_hi = ks.m_hi;
        f4 c[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) c[mt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const h8 bf = k_frag<QT>(r, m, g, ks);
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
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = i >> 1, h = i & 1;
            h2 p[8];
            q6_pairs(r.a[i], r.b[i], r.c[i], p);
#pragma unroll
            for (int qq = 0; qq < 4; qq++) {
                const int s = 8 * n + 2 * qq + h;  // sub-block = chunk of 16
                const h2 p0 = p[2 * qq], p1 = p[2 * qq + 1];
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
// Input transforms applied while preparing the activations (x row t, column
// k; ldx elements between rows):
//   ACT_PLAIN:    a = x[t][k]
//   ACT_RMSNORM:  a = x[t][k] * w[k] (w = 1 if NULL) and ssq[u][t] = sum over
//                 the unit of x^2; the matmul multiplies row t of its result
//                 by 1 / sqrt(sum_u ssq[u][t] / K + eps), which is the RMSNorm
//                 of src/ModelCPU.jl:110-122 moved past the (linear) product
//   ACT_SILU_MUL: a = silu(x[t][k]) * x[t][K + k] for rows [gate | up]
//                 (mlp_forward, src/ModelCPU.jl:447-473)
enum { ACT_PLAIN = 0, ACT_RMSNORM = 1, ACT_SILU_MUL = 2 };
struct ActIn {
    int op, ldx;
    const float *norm_w;
    float eps;
    bool reuse;          // activations already prepared in the workspace
    const float *add;    // n_add slices [M][K] folded into x first (x += sum, stored back)
    int n_add;
    int64_t add_stride;  // floats between slices
    bool defer;          // leave the product as K-slice partials in the workspace
    float *sum_out = nullptr;  // (input = the [M][ldx] slices' sum) also store that sum here, all ldx columns
};

__device__ __forceinline__ float silu_mul1(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// Half-wave (32-lane) butterflies: levels lane ^ 1, lane ^ 2 (DPP quad
// permutes), lane 7 - i within 8 and 15 - i within 16 (DPP mirrors: after
// the quad levels every lane of a quad holds the same value, so a mirror
// pairs the same two partial results as lane ^ 4 and lane ^ 8 would), then
// lane ^ 16 (one swizzle through the LDS crossbar). Every lane ends with the
// full result; the additions are the xor tree's, in the same pairs.
template <int CTRL> __device__ __forceinline__ float dppf(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float xor16(float v) {  // bitmask swizzle: and 0x1f, or 0, xor 0x10
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}
__device__ __forceinline__ float rows_sum(float v) { return v + xor16(v); }
__device__ __forceinline__ float rows_max(float v) { return fmaxf(v, xor16(v)); }
__device__ __forceinline__ float half_wave_sum(float v) {
    v += dppf<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dppf<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dppf<0x141>(v);  // row_half_mirror
    v += dppf<0x140>(v);  // row_mirror
    return rows_sum(v);
}
__device__ __forceinline__ float half_wave_max(float v) {
    v = fmaxf(v, dppf<0xB1>(v));
    v = fmaxf(v, dppf<0x4E>(v));
    v = fmaxf(v, dppf<0x141>(v));
    v = fmaxf(v, dppf<0x140>(v));
    return rows_max(v);
}

// RMSNorm weights of elements [k, k + 8), loaded with the activations (1 when
// there are none)
__device__ __forceinline__ void norm_weights(const float *__restrict__ norm_w, int op, int k, int K, float4 &a,
                                             float4 &b) {
    a = make_float4(1.f, 1.f, 1.f, 1.f);
    b = a;
    if (op == ACT_RMSNORM && norm_w != nullptr && k < K) {
        a = *(const float4 *)(norm_w + k);
        b = *(const float4 *)(norm_w + k + 4);
    }
}

// The transform and layout of one thread's 8 elements (token t, unit u,
// elements [8 gi, 8 gi + 8) of the unit). The 32 threads of a token (one
// half-wave, gi = lane % 32) must all call it: the token max, the RMSNorm sum
// of squares and the sub-block sums are reduced across them.
template <int LK, int MT, bool SPLIT, bool MINS>
__device__ __forceinline__ void prep_finish(float (&v)[8], float4 wa, float4 wb, int u, int t, int gi, int op,
                                            uint8_t *__restrict__ afrag, float *__restrict__ xs,
                                            float *__restrict__ inv, uint8_t *__restrict__ mfrag,
                                            float *__restrict__ ssq, int sl) {
    constexpr int TOK = MT * (SPLIT ? 8 : 16);
    constexpr int ENTRY = Layout<LK>::ENTRY;
    if (op == ACT_RMSNORM) {
        float q = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) q = __builtin_fmaf(v[e], v[e], q);
        q = half_wave_sum(q);
        if (gi == 0 && t < TOK) ssq[(size_t)u * TOK + t] = q;
        const float w[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] *= w[e];
    }
    float mx = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) mx = fmaxf(mx, fabsf(v[e]));
    float sm = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    // token max over the 32 threads of this token (one half-wave)
    mx = half_wave_max(mx);
    // sub-block (32 elements = 4 threads) sums
    sm += dppf<0xB1>(sm);
    sm += dppf<0x4E>(sm);
    int e2 = 0;
    if (mx > 0.f && mx < __builtin_huge_valf()) {
        int ex;
        frexpf(mx, &ex);  // mx = f * 2^ex, f in [0.5, 1)
        e2 = min(max(15 - ex, -120), 120);
    }
    const float scale = ldexpf(1.f, e2);
    if (t >= TOK) return;
    if (gi == 0) inv[(size_t)u * TOK + t] = ldexpf(1.f, -e2);
    if (MINS && xs != nullptr && (gi & 3) == 0) xs[((size_t)u * 8 + (gi >> 2)) * TOK + t] = sm;
    const int mt = SPLIT ? t / 8 : t / 16;
    const int slot = SPLIT ? (t % 8) * 2 : t % 16;
    if (MINS && mfrag != nullptr && (gi & 3) == 0) {
        // A operand of the mins MFMA (16x16x16): lane (slot, G) item e holds
        // sub-block 4G + e of the scaled sub-block sums (G < 2; zero for
        // G >= 2). X_s * scale / 32 stays below 2^15.
        const int sb = gi >> 2, G = sb >> 2, e = sb & 3;
        const float xsum = sm * scale * (1.0f / 32.0f);
        const _Float16 h = (_Float16)xsum, l = (_Float16)(xsum - (float)h);
        _Float16 *mf = (_Float16 *)(mfrag + ((size_t)u * MT + mt) * 512);
        mf[(G * 16 + slot) * 4 + e] = h;
        mf[((G + 2) * 16 + slot) * 4 + e] = (_Float16)0.0f;
        if (SPLIT) {
            mf[(G * 16 + slot + 1) * 4 + e] = l;
            mf[((G + 2) * 16 + slot + 1) * 4 + e] = (_Float16)0.0f;
        }
    }
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
        // (sl > 0: the compact one-tile layout, sl slots of 16 bytes per lane
        // group, padding tokens absent; Q6_K's 8-byte entries 2j and 2j + 1
        // share a slot)
        if (sl > 0) {
            if (slot >= sl) continue;
            const int cc = LK == 1 ? c >> 1 : c, sub = LK == 1 ? (c & 1) * 8 : 0;
            uint8_t *dst = base + ((size_t)(cc * 4 + G) * sl + slot) * 16 + sub + item * 2;
            *(h4 *)dst = H;
            if (SPLIT) *(h4 *)(dst + 16) = L;  // slot + 1
            continue;
        }
        uint8_t *dst = base + ((size_t)(c * MT + mt) * 64 + G * 16 + slot) * ENTRY + item * 2;
        *(h4 *)dst = H;
        if (SPLIT) *(h4 *)(dst + ENTRY) = L;  // slot + 1
    }
}

// add != nullptr: x[t][k] += ((add_0 + add_1) + ...)[t][k] (the K-slice
// partials of a previous matmul, the order its reduce would use), stored back
// into x (each element has one owner thread), before the transform; slices
// [M][K]. X == nullptr: x is that sum itself (slices [M][ldx], rows of 2K
// for ACT_SILU_MUL), stored into xw when xw != nullptr (all ldx columns: the
// workgroups past the units of K fold and store columns K.. only; K is then
// a multiple of 256 and ldx of 8).
template <int LK, int MT, bool SPLIT, bool MINS, int TPW>
__global__ __launch_bounds__(32 * TPW) void prep_kernel(const float *__restrict__ X, int ldx, int M, int K, int op,
                                                   const float *__restrict__ norm_w,
                                                   uint8_t *__restrict__ afrag, float *__restrict__ xs,
                                                   float *__restrict__ inv, uint8_t *__restrict__ mfrag,
                                                   float *__restrict__ ssq, const float *__restrict__ add, int n_add,
                                                   int64_t add_stride, float *__restrict__ xw, int sl) {
    const int u = blockIdx.x, tid = threadIdx.x;
    const int tl = tid >> 5, gi = tid & 31;  // (a token per 32 threads, TPW per workgroup)
    const int t = blockIdx.y * TPW + tl;
    const int k = u * UNIT + gi * 8;
    const bool tail = u >= (K + UNIT - 1) / UNIT;  // (whole workgroups: no transform)
    float4 wa, wb;
    norm_weights(norm_w, op, k, K, wa, wb);
    float v[8];
    if (t < M && (k < K || (tail && k < ldx))) {
        // the sum of the partial slices at column c of row t, in slice order:
        // up to MAXS slices (of both columns when two are asked for) in one
        // round of loads issued before any sum, more four at a time
        constexpr int MAXS = 8;
        auto slices_loop = [&](int64_t rs, int c, float (&sum)[8]) {
#pragma unroll
            for (int e = 0; e < 8; e++) sum[e] = 0.f;
            for (int s0 = 0; s0 < n_add; s0 += 4) {
                float4 va[4], vb[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float *pa = add + (size_t)min(s0 + j, n_add - 1) * add_stride + (size_t)t * rs + c;
                    va[j] = *(const float4 *)pa;
                    vb[j] = *(const float4 *)(pa + 4);
                }
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    if (s0 + j >= n_add) break;
                    const float pv[8] = {va[j].x, va[j].y, va[j].z, va[j].w, vb[j].x, vb[j].y, vb[j].z, vb[j].w};
#pragma unroll
                    for (int e = 0; e < 8; e++) sum[e] = s0 + j == 0 ? pv[e] : sum[e] + pv[e];
                }
            }
        };
        auto issue = [&](int64_t rs, int c, auto &va, auto &vb) {
            constexpr int NS = sizeof(va) / sizeof(va[0]);
#pragma unroll
            for (int j = 0; j < NS; j++) {
                if (j < n_add) {
                    const float *pa = add + (size_t)j * add_stride + (size_t)t * rs + c;
                    va[j] = *(const float4 *)pa;
                    vb[j] = *(const float4 *)(pa + 4);
                }
            }
        };
        auto fold = [&](const auto &va, const auto &vb, float (&sum)[8]) {
            constexpr int NS = sizeof(va) / sizeof(va[0]);
#pragma unroll
            for (int e = 0; e < 8; e++) sum[e] = 0.f;  // (no slices: zero, as the loop gives)
#pragma unroll
            for (int j = 0; j < NS; j++) {
                if (j < n_add) {
                    const float pv[8] = {va[j].x, va[j].y, va[j].z, va[j].w, vb[j].x, vb[j].y, vb[j].z, vb[j].w};
#pragma unroll
                    for (int e = 0; e < 8; e++) sum[e] = j == 0 ? pv[e] : sum[e] + pv[e];
                }
            }
        };
        // one column's slices
        auto slices = [&](int64_t rs, int c, float (&sum)[8]) {
            if (n_add > MAXS) {
                slices_loop(rs, c, sum);
                return;
            }
            float4 va[MAXS], vb[MAXS];
            issue(rs, c, va, vb);
            fold(va, vb, sum);
        };
        float up[8];
        if (X != nullptr) {
            const float *row = X + (size_t)t * ldx + k;
            const float4 a = *(const float4 *)row;
            const float4 b = *(const float4 *)(row + 4);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
            if (add != nullptr) {
                float sum[8];
                slices(K, k, sum);
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = v[e] + sum[e];
                float *wrow = xw + (size_t)t * ldx + k;
                *(float4 *)wrow = make_float4(v[0], v[1], v[2], v[3]);
                *(float4 *)(wrow + 4) = make_float4(v[4], v[5], v[6], v[7]);
            }
            if (op == ACT_SILU_MUL) {
                const float4 c = *(const float4 *)(row + K);
                const float4 d = *(const float4 *)(row + K + 4);
                up[0] = c.x; up[1] = c.y; up[2] = c.z; up[3] = c.w;
                up[4] = d.x; up[5] = d.y; up[6] = d.z; up[7] = d.w;
            }
        } else if (op == ACT_SILU_MUL && n_add <= MAXS / 2) {
            // gate and up columns' slices in one round
            float4 va[MAXS / 2], vb[MAXS / 2], ua[MAXS / 2], ub[MAXS / 2];
            issue(ldx, k, va, vb);
            issue(ldx, K + k, ua, ub);
            fold(va, vb, v);
            fold(ua, ub, up);
        } else {
            slices(ldx, k, v);
            if (op == ACT_SILU_MUL) slices(ldx, K + k, up);
            if (xw != nullptr) {  // (the sum itself, stored for the caller)
                float *wrow = xw + (size_t)t * ldx + k;
                *(float4 *)wrow = make_float4(v[0], v[1], v[2], v[3]);
                *(float4 *)(wrow + 4) = make_float4(v[4], v[5], v[6], v[7]);
            }
        }
        if (op == ACT_SILU_MUL) {
#pragma unroll
            for (int e = 0; e < 8; e++) v[e] = silu_mul1(v[e], up[e]);
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = 0.f;
    }
    if (tail) return;
    prep_finish<LK, MT, SPLIT, MINS>(v, wa, wb, u, t, gi, op, afrag, xs, inv, mfrag, ssq, sl);
}

// ---------------------------------------------------------------- gemm
// Persistent streaming: workgroup (w, s) keeps the prepared activations of
// K-slice s in LDS and walks the row groups w, w + G, w + 2G, ... (G =
// gridDim.x). Each wave owns 16 rows of every row group and streams the
// (row group, unit) items through a ring of RING units whose loads are issued
// RING - 1 items ahead, across row-group boundaries.
template <int QT, int MT> struct Ring { static constexpr int R = (QT == QT_Q6_K && MT >= 3) ? 2 : 4; };

template <int QT, int MT, bool SPLIT, bool PK>
__global__ __launch_bounds__(WG_THREADS)
void gemm_q_kernel(const uint8_t *__restrict__ W, float *__restrict__ Y, int M, int N, int K, int ups, int S,
                   const uint8_t *__restrict__ afrag, const float *__restrict__ xs, const float *__restrict__ invs,
                   const float *__restrict__ ssq, float eps, float *__restrict__ part) {
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
    const int rowgroups = (N + ROWS_PER_WG - 1) / ROWS_PER_WG;
    const int G = gridDim.x;
    if ((int)blockIdx.x >= rowgroups) return;  // whole workgroup
    const int n_rg = (rowgroups - 1 - (int)blockIdx.x) / G + 1;
    const int n_items = n_rg * nu;
    const size_t row_bytes = (size_t)(K / C::QK) * C::BB;
    const int tail_blk = (QT == QT_Q8_0 && (K % UNIT)) ? (K % UNIT) / 32 : 8;

    uint8_t *a_lds = smem;                                      // [ups][UNIT_A]
    float *x_lds = (float *)(smem + (size_t)ups * UNIT_A);      // [ups][8][TOK]
    float *i_lds = x_lds + (C::MINS ? ups * 8 * TOK : 0);       // [ups][TOK]
    __shared__ float rs[TOK];                                   // RMSNorm row scales
    __shared__ float rsp[WG_THREADS];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n_in = lane & 15, g = lane >> 4;
    const int row_in = wave * 16 + n_in;

    // 1. fetch this slice's prepared activations into registers (uniform
    //    trip counts and clamped indices: no per-load branches, so every
    //    load is in flight before the first wait)
    const uint4 *a_src = (const uint4 *)(afrag + (size_t)u0 * UNIT_A);
    const int n16 = nu * (UNIT_A / 16);
    constexpr int A_PER_T = 8;  // 16-byte pieces per thread in the first pass
    uint4 a_tmp[A_PER_T];
#pragma unroll
    for (int j = 0; j < A_PER_T; j++) a_tmp[j] = a_src[min(j * WG_THREADS + tid, n16 - 1)];
    const int n_x = C::MINS ? nu * 8 * TOK : 0, n_i = nu * TOK;
    const float *xs_src = xs + (size_t)u0 * 8 * TOK;
    const float *i_src = invs + (size_t)u0 * TOK;
    float x_tmp[2], i_tmp = i_src[min(tid, n_i - 1)];
#pragma unroll
    for (int j = 0; j < 2; j++) x_tmp[j] = C::MINS ? xs_src[min(j * WG_THREADS + tid, max(n_x - 1, 0))] : 0.f;

    // 2. start streaming weights: the load stream walks items (row group
    //    blockIdx.x + G*lj, unit lu) in order; past the last item it reloads
    //    the last one, so every step issues the same batch of loads
    int lj = 0, lu = 0;
    auto load_next = [&](Unit<QT> &b) {
        const bool past = lj >= n_rg;
        const int j = past ? n_rg - 1 : lj, uu = past ? nu - 1 : lu;
        if constexpr (PK) {
            const int tile = min(((int)blockIdx.x + G * j) * (ROWS_PER_WG / 16) + wave, (N + 15) / 16 - 1);
            load_unit_packed<QT>(W + ((size_t)tile * n_units + u0 + uu) * Packed<QT>::CHUNK, lane, b);
        } else {
            const int row = min(((int)blockIdx.x + G * j) * ROWS_PER_WG + row_in, N - 1);
            load_unit<QT>(W + (size_t)row * row_bytes + (size_t)(u0 + uu) * UNIT_BYTES, g,
                          (u0 + uu == n_units - 1) ? tail_blk : 8, b);
        }
        if (++lu == nu) {
            lu = 0;
            ++lj;
        }
    };
    Unit<QT> buf[R];
#pragma unroll
    for (int p = 0; p < R - 1; p++) load_next(buf[p]);

    // 3. activations into LDS (clamped lanes rewrite the last entry with its
    //    own value); a second pass only when a slice exceeds the first
    {
        uint4 *dst = (uint4 *)a_lds;
#pragma unroll
        for (int j = 0; j < A_PER_T; j++) dst[min(j * WG_THREADS + tid, n16 - 1)] = a_tmp[j];
        for (int i = A_PER_T * WG_THREADS + tid; i < n16; i += WG_THREADS) dst[i] = a_src[i];
        if constexpr (C::MINS) {
#pragma unroll
            for (int j = 0; j < 2; j++) x_lds[min(j * WG_THREADS + tid, n_x - 1)] = x_tmp[j];
            for (int i = 2 * WG_THREADS + tid; i < n_x; i += WG_THREADS) x_lds[i] = xs_src[i];
        }
        i_lds[min(tid, n_i - 1)] = i_tmp;
        for (int i = WG_THREADS + tid; i < n_i; i += WG_THREADS) i_lds[i] = i_src[i];
    }
    {
        RowScales<TOK, WG_THREADS> rsc;
        rsc.issue(ssq, n_units, tid);
        rsc.finish(ssq, n_units, K, eps, tid, rsp, rs);
    }

    // 4. stream items through the MFMA pipe; a row group's epilogue follows
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
    int cj = 0, cu = 0;  // consume position
    auto consume = [&](Unit<QT> &b) {
        if constexpr (!PK) finish_unit<QT>(b);
        compute_unit<QT, MT, SPLIT>(b, a_lane + (size_t)cu * UNIT_A, x_lds + (size_t)cu * 8 * TOK,
                                    i_lds + (size_t)cu * TOK, g, A);
        if (++cu == nu) {
            // epilogue: lane values are row r, tokens lane_token(mt, g, u);
            // stores only (an accumulating call reduces through part)
            const int r = ((int)blockIdx.x + G * cj) * ROWS_PER_WG + row_in;
            if (r < N) {
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int u = 0; u < TPL; u++) {
                        const int t = lane_token<SPLIT>(mt, g, u);
                        if (t >= M) continue;
                        float v = SPLIT ? (A.acc[mt][2 * u] + A.acc[mt][2 * u + 1]) : A.acc[mt][u];
                        if constexpr (C::MINS) v = v - A.macc[mt][u];
                        v *= rs[t];
                        if (part == nullptr)
                            Y[(size_t)t * N + r] = v;
                        else
                            part[((size_t)blockIdx.y * M + t) * N + r] = v;
                    }
            }
            reset();
            cu = 0;
            ++cj;
        }
    };
    const int n_full = n_items - n_items % R;
    for (int ib = 0; ib < n_full; ib += R) {
#pragma unroll
        for (int p = 0; p < R; p++) {
            load_next(buf[(p + R - 1) % R]);
            consume(buf[p]);
        }
    }
    // the last n_items % R items are already in buf[0 ..]
#pragma unroll
    for (int p = 0; p < R - 1; p++)
        if (n_full + p < n_items) consume(buf[p]);
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

// ---------------------------------------------------------------- streaming kernel (one token tile)
// With one token tile (M <= 8 fp32-accurate, M <= 16 half) the activation
// operand of a few units fits in VGPRs, so the weight stream needs no LDS.
// Workgroup (w, s) of NW waves covers K-units [s*NW*UPS, (s+1)*NW*UPS):
// wave i holds the A operand of units s*NW*UPS + i*UPS + [0, UPS) and streams
// the 16-row tiles w, w + G, w + 2G, ... of those units through a ring of 4
// units issued 3 ahead. At the end of a tile the NW partial tiles meet in LDS
// and wave (tile % NW) sums them in wave order (deterministic).
template <int QT> struct AReg;
template <> struct AReg<QT_Q4_K> { h8 f[8]; h4 mins; };
template <> struct AReg<QT_Q5_K> { h8 f[8]; h4 mins; };
template <> struct AReg<QT_Q6_K> { h4 f[16]; };
template <> struct AReg<QT_Q8_0> { h8 f[8]; };

// The 16 sub-block products of a Q6_K unit against MT register tiles with
// the int8 sub-block scales folded into the weight operand: c[mt] = sum_s
// (sc_s (q - 32) . x)_s. Half (EXACT false): B = fp16(sc (q - 32)), one
// rounding (|sc (q - 32)| <= 4096), the order of error of the fp16
// activations. EXACT: two fp16 terms, hi = fp16(sc (q - 32)) and the
// residual lo = sc (q - 32) - hi (0 or +-1: the product is an integer), so
// every product is exact. Sub-blocks 2j and 2j + 1 (groups 2n and 2n + 1,
// the same qq; adjacent A operands f[2j], f[2j + 1]) share one 16x16x32
// MFMA per term, which costs the matrix core what a 16x16x16 does.
template <int MT, bool EXACT>
__device__ __forceinline__ void q6_mfma_folded(const Unit<QT_Q6_K> &r, const AReg<QT_Q6_K> (&a)[MT], f4 (&c)[MT]) {
    // the 16 scales as exact fp16: (1024 + (sc ^ 0x80)) - 1152 = sc
    const uint32_t scw[4] = {r.sc.x ^ 0x80808080u, r.sc.y ^ 0x80808080u, r.sc.z ^ 0x80808080u,
                             r.sc.w ^ 0x80808080u};
    const h2 off_sc = as_h2(0xE480E480u);
    h2 sch[8];
#pragma unroll
    for (int w = 0; w < 4; w++) {
        sch[2 * w] = as_h2(pair_lo(scw[w])) + off_sc;
        sch[2 * w + 1] = as_h2(pair_hi(scw[w])) + off_sc;
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++) c[mt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int n = 0; n < 2; n++) {
        h2 p[2][8];
        q6_pairs(r.a[2 * n], r.b[2 * n], r.c[2 * n], p[0]);
        q6_pairs(r.a[2 * n + 1], r.b[2 * n + 1], r.c[2 * n + 1], p[1]);
#pragma unroll
        for (int qq = 0; qq < 4; qq++) {
            const int s = 8 * n + 2 * qq;  // (and s + 1)
            h8 bh, bl;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const _Float16 sv = sch[(s + h) >> 1][(s + h) & 1];
                const h2 ss = {sv, sv};
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const h2 hi = p[h][2 * qq + t] * ss;
                    bh[4 * h + 2 * t] = hi[0]; bh[4 * h + 2 * t + 1] = hi[1];
                    if constexpr (EXACT) {
                        const h2 lo = __builtin_elementwise_fma(p[h][2 * qq + t], ss, -hi);
                        bl[4 * h + 2 * t] = lo[0]; bl[4 * h + 2 * t + 1] = lo[1];
                    }
                }
            }
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const h8 a8 = __builtin_shufflevector(a[mt].f[s], a[mt].f[s + 1], 0, 1, 2, 3, 4, 5, 6, 7);
                c[mt] = mfma32(a8, bh, c[mt]);
                if constexpr (EXACT) c[mt] = mfma32(a8, bl, c[mt]);
            }
        }
    }
}

// One unit against register operands of MT token tiles: each weight
// fragment is dequantized once and multiplies every tile. acc[mt]: scaled dot
// products, macc[mt]: the Q4_K/Q5_K min term / 32 (both in the MFMA D layout:
// slot 4g + v, row n); inv[mt][k]: inverse unit scales of the lane's tokens.
// A dead unit (past the end of K) contributes exactly zero.
template <int QT, bool SPLIT, int MT>
__device__ __forceinline__ void compute_v(const Unit<QT> &r, const AReg<QT> (&a)[MT], const float (&inv)[MT][SPLIT ? 2 : 4],
                                          int g, bool live, f4 (&acc)[MT], f4 (&macc)[MT]) {
    if constexpr (QT == QT_Q4_K || QT == QT_Q5_K) {
        float d = half_bits(r.hdr.x), dmin = half_bits(r.hdr.x >> 16);
        if (!live) { d = 0.f; dmin = 0.f; }
        const KScales ks = k_scales<QT>(r.hdr, g);
        const uint32_t m_lo = ks.m_lo, m_hi = ks.m_hi;
        const h2 neg1024 = as_h2(0xE400E400u);  // (-1024, -1024)
        f4 c[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) c[mt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const h8 bf = k_frag<QT>(r, m, g, ks);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) c[mt] = mfma32(a[mt].f[m], bf, c[mt]);
        }
        // min term on the matrix core: B = m_s of this row for s = 4g..4g+3
        // (lane groups 0, 1), zero for lane groups 2, 3
        const uint32_t mw = g == 0 ? m_lo : (g == 1 ? m_hi : 0u);
        const h2 p0 = as_h2(pair_lo(mw)) + neg1024, p1 = as_h2(pair_hi(mw)) + neg1024;
        h4 bm;
        bm[0] = p0[0]; bm[1] = p0[1]; bm[2] = p1[0]; bm[3] = p1[1];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const f4 cm = mfma16(a[mt].mins, bm, f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const float iv = inv[mt][acc_token_u<SPLIT>(v)];
                acc[mt][v] = __builtin_fmaf(d * iv, c[mt][v], acc[mt][v]);
                macc[mt][v] = __builtin_fmaf(dmin * iv, cm[v], macc[mt][v]);
            }
        }
    } else if constexpr (QT == QT_Q6_K) {
        const float d = live ? half_bits(r.d) : 0.f;
        f4 sacc[MT];  // sum over sub-blocks of sc_s * (q . x)_s, per tile
#pragma unroll
        for (int mt = 0; mt < MT; mt++) sacc[mt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = i >> 1, h = i & 1;
            h2 p[8];
            q6_pairs(r.a[i], r.b[i], r.c[i], p);
#pragma unroll
            for (int qq = 0; qq < 4; qq++) {
                const int sb = 8 * n + 2 * qq + h;
                const h2 p0 = p[2 * qq], p1 = p[2 * qq + 1];
                h4 b;
                b[0] = p0[0]; b[1] = p0[1]; b[2] = p1[0]; b[3] = p1[1];
                const uint32_t scw = (sb >> 2) == 0 ? r.sc.x : (sb >> 2) == 1 ? r.sc.y : (sb >> 2) == 2 ? r.sc.z : r.sc.w;
                const float scf = (float)(int)(int8_t)((scw >> (8 * (sb & 3))) & 0xffu);
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    const f4 c = mfma16(a[mt].f[sb], b, f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                    for (int v = 0; v < 4; v++) sacc[mt][v] = __builtin_fmaf(scf, c[v], sacc[mt][v]);
                }
            }
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int v = 0; v < 4; v++)
                acc[mt][v] = __builtin_fmaf(d * inv[mt][acc_token_u<SPLIT>(v)], sacc[mt][v], acc[mt][v]);
    } else {
        const h2 off = as_h2(0xE480E480u);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float d = live ? half_bits(r.d[i]) : 0.f;
            const uint32_t t0 = r.w0[i] ^ 0x80808080u, t1 = r.w1[i] ^ 0x80808080u;
            const h2 p0 = as_h2(pair_lo(t0)) + off, p1 = as_h2(pair_hi(t0)) + off;
            const h2 p2 = as_h2(pair_lo(t1)) + off, p3 = as_h2(pair_hi(t1)) + off;
            h8 b;
            b[0] = p0[0]; b[1] = p0[1]; b[2] = p1[0]; b[3] = p1[1];
            b[4] = p2[0]; b[5] = p2[1]; b[6] = p3[0]; b[7] = p3[1];
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const f4 c = mfma32(a[mt].f[i], b, f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                for (int v = 0; v < 4; v++)
                    acc[mt][v] = __builtin_fmaf(d * inv[mt][acc_token_u<SPLIT>(v)], c[v], acc[mt][v]);
            }
        }
    }
}

// ---------------------------------------------------------------- chained matmuls
// A chain of fp32-accurate one-tile matmuls (M <= 8) that hand each other
// their activations without an input stage:
//  * the producer's epilogue writes its fp32 result y and, for the next
//    matmul, the split-fp16 operand of v = y w (w: the next RMSNorm weight,
//    or 1) in the input stage's byte layout, but scaled by a power of two of
//    its own 16-row tile (8 gated channels for EPI_GATE): the tile's largest
//    |v| lands in [2^14, 2^15), as the input stage does per 256-element unit.
//    Beside the limbs it stores the tile's exponent once per lane entry, the
//    tile's sum of v (the min terms of Q4_K/Q5_K) and, where an RMSNorm
//    follows, its sum of y^2; EPI_RESID adds into the residual y itself,
//    EPI_GATE reads tiles of 8 gate rows and their 8 up rows
//    (ihip_pack_weights_gated) and writes h = silu(g) u;
//  * the consumer loads the limbs as a classic matmul loads its prepared
//    operand, takes the unit's exponent as the smallest over its tiles (the
//    input stage's, from the largest |v|) and rescales each entry by the
//    exact power of two 2^(e_unit - e_tile): the input stage's limbs wherever
//    the result stays a normal fp16 (else the same value to within 2^-24 of
//    the unit's scale).
// Sum of 8 values in the input stage's order.
__device__ __forceinline__ float sum8(const float (&v)[8]) {
    return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
}

// Exponent of a tile scale: largest |v| in [2^14, 2^15) after scaling (the
// input stage's rule), 127 for an all-zero tile (no bound on the unit's
// exponent), 0 when the tile holds Inf or NaN.
__device__ __forceinline__ int tile_exp(float mx) {
    if (mx == 0.f) return 127;
    if (!(mx < __builtin_huge_valf())) return 0;
    int ex;
    frexpf(mx, &ex);
    return min(max(15 - ex, -120), 120);
}

// What one lane stages per unit before the weight ring: its entries'
// exponents and, for the min terms, the producer's tile sums of its
// sub-blocks (the limbs go straight into the A registers).
struct XStage {
    uint4 ex;      // 16 exponent bytes (Q4_K/Q5_K use the first 8)
    float4 ts[4];  // tile sums of sub-blocks 4 G' .. 4 G' + 3 (G' = G & 1): 8 or 16
};

template <int QT>
__device__ __forceinline__ void stage_unit_x(const uint8_t *xop, const float *xsum, int xsum_stride, int tpu, int M,
                                             int un, int n_units, int lane, XStage &s) {
    const int slot = lane & 15, G = lane >> 4;
    const int t = min(slot >> 1, M - 1);
    // (compact: lane group G, slot s at G 2M + s; padding slots read a real slot's bytes, unused)
    const uint8_t *pe = xop + (size_t)n_units * CHAIN_UNIT_LIMBS + (size_t)un * CHAIN_UNIT_EXPS +
                        (size_t)(G * 2 * M + min(slot, 2 * M - 1)) * 16;
    if constexpr (QT == QT_Q4_K || QT == QT_Q5_K) {  // (8 entries)
        const uint2 e8 = *(const uint2 *)pe;
        s.ex = make_uint4(e8.x, e8.y, 0u, 0u);
    } else {
        s.ex = *(const uint4 *)pe;
    }
    if constexpr (GemmCfg<QT>::MINS) {
        // sub-blocks 4 G .. 4 G + 3 (lane groups G < 2 only): tiles 8 G .. (16-row) or 16 G .. (8-row)
        if (G < 2) {
            const float *ps = xsum + (size_t)t * xsum_stride + (size_t)un * tpu + (tpu / 2) * G;
            s.ts[0] = *(const float4 *)ps;
            s.ts[1] = *(const float4 *)(ps + 4);
            if (tpu == 32) {
                s.ts[2] = *(const float4 *)(ps + 8);
                s.ts[3] = *(const float4 *)(ps + 12);
            }
        }
    }
}

// The staged unit's operand finished in place: entries rescaled to the
// unit's power of two, the min-term operand, inv[k] (inverse unit scales of
// the accumulator tokens 2G + k). tok: the lane's token is real and the unit
// exists. Every lane must call it (the unit exponent crosses lanes).
template <int QT>
__device__ __forceinline__ void finish_unit_x(const XStage &s, int tpu, bool tok, int lane, AReg<QT> &a,
                                              float (&inv)[2]) {
    constexpr int LK = QT == QT_Q6_K ? 1 : QT == QT_Q8_0 ? 2 : 0;
    constexpr int NE = LK == 0 ? 8 : 16;  // exponent entries per lane
    const int slot = lane & 15, G = lane >> 4;
    const bool L = slot & 1;
    int e[NE];
    const uint32_t w[4] = {s.ex.x, s.ex.y, s.ex.z, s.ex.w};
#pragma unroll
    for (int i = 0; i < NE; i++) e[i] = (int)(int8_t)(w[i >> 2] >> (8 * (i & 3)));
    // the unit's exponent: the smallest over the token's tiles (its 4 lane groups hold all of them)
    int eu = 127;
#pragma unroll
    for (int i = 0; i < NE; i++) eu = min(eu, e[i]);
    eu = min(eu, __shfl_xor(eu, 16));
    eu = min(eu, __shfl_xor(eu, 32));
    if (eu == 127 || !tok) eu = 0;
    inv[0] = ldexpf(1.f, -__shfl(eu, 4 * G));
    inv[1] = ldexpf(1.f, -__shfl(eu, 4 * G + 2));
    // 2^(eu - e) as fp16: exact down to 2^-24, 0 below (and for all-zero tiles)
    auto factor = [&](int ei) -> _Float16 {
        const int d = max(e[ei] - eu, 0);  // (>= 0 for a real token; padding lanes hold zeros)
        return (_Float16)(d <= 24 ? ldexpf(1.f, -d) : 0.f);
    };
    if constexpr (LK == 0) {
#pragma unroll
        for (int c = 0; c < 8; c++) a.f[c] = a.f[c] * factor(c);
    } else if constexpr (LK == 1) {
#pragma unroll
        for (int c = 0; c < 16; c++) a.f[c] = a.f[c] * factor(c);
    } else {
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const _Float16 f0 = factor(2 * c), f1 = factor(2 * c + 1);
            const h8 f = {f0, f0, f0, f0, f1, f1, f1, f1};
            a.f[c] = a.f[c] * f;
        }
    }
    if constexpr (GemmCfg<QT>::MINS) {
        // min-term operand: lane group G < 2 holds sub-blocks 4 G .. 4 G + 3, each the sum of its
        // 2 (16-row) or 4 (8-row) tiles
        const float scale = ldexpf(1.f, eu) * (1.0f / 32.0f);
        const float t[16] = {s.ts[0].x, s.ts[0].y, s.ts[0].z, s.ts[0].w, s.ts[1].x, s.ts[1].y, s.ts[1].z, s.ts[1].w,
                             s.ts[2].x, s.ts[2].y, s.ts[2].z, s.ts[2].w, s.ts[3].x, s.ts[3].y, s.ts[3].z, s.ts[3].w};
        const bool eight = tpu == 32;
        h4 mn;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float xsb = eight ? (t[4 * j] + t[4 * j + 1]) + (t[4 * j + 2] + t[4 * j + 3])
                                    : t[2 * j] + t[2 * j + 1];
            const float xsum = xsb * scale;
            const _Float16 hi = (_Float16)xsum;
            mn[j] = (G < 2 && tok) ? (L ? (_Float16)(xsum - (float)hi) : hi) : (_Float16)0.0f;
        }
        a.mins = mn;
    }
}

// Maximum / sum over the 16 lanes of a DPP row (the lanes of one token pair).
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dppf<0xB1>(v));
    v = fmaxf(v, dppf<0x4E>(v));
    v = fmaxf(v, dppf<0x141>(v));
    return fmaxf(v, dppf<0x140>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dppf<0xB1>(v);
    v += dppf<0x4E>(v);
    v += dppf<0x141>(v);
    return v + dppf<0x140>(v);
}

// The consumer operand of one value (token t, consumer element k) at the
// tile's exponent e2, for the consumer layout ch.op_lk (operand_pos's maps,
// selected arithmetically: one copy of the code for the three layouts): hi
// and lo limbs at slots 2t, 2t + 1; the entry's exponent written by the
// entry's first element.
__device__ __forceinline__ void put_operand(const Chain &ch, int M, int t, int k, float v, int e2) {
    const int lk = ch.op_lk, o = k & 255, u = k >> 8;
    const int q = (o >> 3) & 3;
    const int c = lk == 0 ? ((o >> 3) & 1) + 2 * ((o >> 5) & 1) + 4 * ((o >> 7) & 1) : lk == 1 ? o >> 4 : o >> 5;
    const int G = lk == 0 ? ((o >> 4) & 1) + 2 * ((o >> 6) & 1) : lk == 1 ? (o >> 2) & 3 : 2 * (q & 1) + ((o >> 2) & 1);
    const int item = lk == 0 ? o & 7 : lk == 1 ? o & 3 : (q < 2 ? 0 : 4) + (o & 3);
    const int ei = lk == 2 ? 2 * c + (q >> 1) : c;
    const float xs = v * ldexpf(1.f, e2 == 127 ? 0 : e2);
    const _Float16 hi = (_Float16)xs, lo = (_Float16)(xs - (float)hi);
    // (the compact one-tile layout: 16 bytes per slot; Q6_K's 8-byte entries
    // 2j and 2j + 1 share one)
    const int sl = 2 * M, cc = lk == 1 ? c >> 1 : c, sub = lk == 1 ? (c & 1) * 8 : 0;
    uint8_t *p = ch.yop + (size_t)u * CHAIN_UNIT_LIMBS + (size_t)((cc * 4 + G) * sl + 2 * t) * 16 + sub + item * 2;
    *(_Float16 *)p = hi;
    *(_Float16 *)(p + 16) = lo;
    if ((item & 3) == 0 && (lk == 2 || item == 0)) {
        int8_t *x = (int8_t *)ch.yop + (size_t)ch.y_units * CHAIN_UNIT_LIMBS + (size_t)u * CHAIN_UNIT_EXPS +
                    (G * sl + 2 * t) * 16 + ei;
        x[0] = (int8_t)e2;
        x[16] = (int8_t)e2;
    }
}

// Epilogue of a chained producer (one 16-row tile; lanes n_in = row, g =
// token pair 2g, 2g + 1): stores the tile, the consumer's operand and the
// statistics. Whole waves call it (row reductions across the 16 lanes of
// each token pair). yold: the residual's old values (EPI_RESID), w: the
// next norm weight of this lane's row. Written to stay small (one pass per
// token, one operand writer): it runs once per tile at a kernel's end, where
// every instruction is fetched cold. One call handles one of the two tokens
// of each lane (token 2 g + k: s is its sum), so a workgroup's (tile, token)
// jobs can spread over its waves.
__device__ __forceinline__ void chain_epilogue(const Chain &ch, float *__restrict__ Y, float s, const float *rs,
                                               int M, int N, int tile, int n_in, int g, int k, float yold, float w) {
    const int r = tile * 16 + n_in;
    const bool stats = ch.epi != EPI_STATS || tile * 16 < ch.stat_rows;
    const int kcons = ch.epi == EPI_GATE ? tile * 8 + (n_in & 7) : r;  // the consumer's element
    const bool real = r < N && (ch.epi != EPI_GATE || n_in < 8);
    const int t = 2 * g + k;
    const bool ok = r < N && t < M;
    const float v0 = ok ? s * rs[t] : 0.f;
    float y = v0;
    if (ch.epi == EPI_GATE) {
        // rows 16 tile + n are gate channel 8 tile + n (n < 8) and its up row (n + 8)
        const float u = __shfl_xor(v0, 8);
        y = (n_in < 8 && ok) ? silu_mul1(v0, u) : 0.f;
        if (n_in < 8 && ok) Y[(size_t)t * ch.ldy + kcons] = y;
    } else if (ok) {
        if (ch.epi == EPI_RESID) y += yold;
        Y[(size_t)t * ch.ldy + r] = y;
    }
    if (!stats) return;
    const float v = y * w;
    if (ch.yop != nullptr) {
        const int e2 = tile_exp(row16_max(fabsf(v)));
        if (real && t < M) put_operand(ch, M, t, kcons, v, e2);
    }
    const float ts = ch.ysum != nullptr ? row16_sum(v) : 0.f;
    const float sq = ch.yssq != nullptr ? row16_sum(y * y) : 0.f;
    if (n_in == 0 && t < M) {
        if (ch.ysum != nullptr) ch.ysum[(size_t)t * ch.ysum_stride + tile] = ts;
        if (ch.yssq != nullptr) ch.yssq[(size_t)tile * 8 + t] = sq;
    }
}

// One token tile (MT = 1; several tiles run gemm_w_kernel).
template <int QT, int NW, int UPS, bool SPLIT, bool PK, int MT, bool XIN, int DE>
__global__ __launch_bounds__(NW * 64, UPS == 3 ? 1 : 8 / NW)
void gemm_v_kernel(const uint8_t *__restrict__ W, const uint8_t *__restrict__ afrag,
                   const uint8_t *__restrict__ mfrag, const float *__restrict__ invs, int M, int N, int K, int G,
                   int xs_stride, int x_tpu, float *__restrict__ Y, int accum, const float *__restrict__ ssq,
                   int n_ssq, float eps, float *__restrict__ part, Chain ch) {
    using C = GemmCfg<QT>;
    static_assert(MT == 1, "one token tile");
    // DE: where the tiles' epilogue runs: 0 in the weight loop as each batch
    // of tiles completes (plain stores); 2 (a chained producer's) after the
    // loop, from the reduced tiles kept in LDS, with the loop's registers free
    // (at most CHAIN_MAX_TILES per workgroup, which the host checks); 3 the
    // same for a producer split over K (each tile finished by the last slice
    // to arrive: a separate instantiation keeps DE 2's code unchanged).
    // Measured: plain stores after the loop are slower (the step 1.5 %): the
    // stores then all wait at the kernel's end.
    static_assert(DE == 0 || DE == 2 || DE == 3, "epilogue placement");
    static_assert((!XIN && DE == 0) || (SPLIT && MT == 1), "chained calls: fp32-accurate, one token tile");
    constexpr bool CE = DE >= 2;
    constexpr int TOKT = SPLIT ? 8 : 16;  // tokens per MFMA tile
    constexpr int TOK = MT * TOKT;
    constexpr int TPL = SPLIT ? 2 : 4;
    constexpr int UNIT_BYTES = (QT == QT_Q8_0) ? 8 * 34 : C::BB;
    constexpr int R = UPS == 3 ? 6 : 4;  // (3 units: one wave per SIMD, a deeper ring)
    static_assert(R % UPS == 0, "ring positions must map to fixed units");
    // partial tiles meet in LDS in batches of F tiles (double-buffered), one
    // barrier per batch (Q6_K, short of registers: one tile per batch)
    constexpr int F = QT == QT_Q6_K ? 1 : (TPL == 4) ? NW / 2 : NW;
    __shared__ __align__(16) float red[2][F][NW][64][TPL * MT];
    __shared__ float rs[TOK];  // RMSNorm row scales (1 without RMSNorm)
    __shared__ float rsp[NW * 64];
    __shared__ float2 pend[DE ? CHAIN_MAX_TILES : 1][64];  // reduced tiles awaiting the epilogue

    const int n_units = (K + UNIT - 1) / UNIT;
    const int n_tiles = (N + 15) / 16;
    // wave index as a scalar: everything derived from it stays in SGPRs
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n_in = lane & 15, g = lane >> 4;
    const int SL = SPLIT ? 2 * M : M;  // operand slots per lane group (compact layout)
    const int my_tiles = (n_tiles - 1 - (int)blockIdx.x) / G + 1;  // the plan keeps G <= n_tiles
    const int unit0 = ((int)blockIdx.y * NW + wave) * UPS;
    const size_t row_bytes = (size_t)(K / C::QK) * C::BB;
    const int tail_blk = (QT == QT_Q8_0 && (K % UNIT)) ? (K % UNIT) / 32 : 8;

    // 1. this wave's A operand for MT token tiles (prepared in the MFMA lane
    //    layout: entry (chunk c, tile mt) at (c MT + mt) 64 + lane)
    AReg<QT> a[UPS][MT];
    float inv[UPS][MT][TPL];
    bool live[UPS];
#pragma unroll
    for (int u = 0; u < UPS; u++) {
        live[u] = unit0 + u < n_units;
        const int un = min(unit0 + u, n_units - 1);
        // (a chained input: the producer's limbs, rescaled once the ring is in flight)
        // (the compact one-tile layout: entry c, lane group g, slot n_in at (4 c + g) SL + n_in, 16
        // bytes; Q6_K's entries 2j, 2j + 1 as the halves of slot entry j)
        const uint8_t *src = afrag + (size_t)un * UNIT_A1 + (size_t)(g * SL + n_in) * 16;
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            // slots of padding tokens are zero: not fetched
            if ((SPLIT ? (n_in >> 1) : n_in) + mt * TOKT < M) {
                if constexpr (QT == QT_Q6_K) {
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        const h8 v = *(const h8 *)(src + (size_t)j * 4 * SL * 16);
                        a[u][mt].f[2 * j] = __builtin_shufflevector(v, v, 0, 1, 2, 3);
                        a[u][mt].f[2 * j + 1] = __builtin_shufflevector(v, v, 4, 5, 6, 7);
                    }
                } else {
#pragma unroll
                    for (int c = 0; c < 8; c++) a[u][mt].f[c] = *(const h8 *)(src + (size_t)c * 4 * SL * 16);
                }
                if constexpr (C::MINS && !XIN)
                    a[u][mt].mins = *(const h4 *)(mfrag + ((size_t)un * MT + mt) * 512 + lane * 8);
            } else {
                if constexpr (QT == QT_Q6_K) {
#pragma unroll
                    for (int c = 0; c < 16; c++) a[u][mt].f[c] = h4{};
                } else {
#pragma unroll
                    for (int c = 0; c < 8; c++) a[u][mt].f[c] = h8{};
                }
                if constexpr (C::MINS) a[u][mt].mins = h4{};
            }
            if constexpr (!XIN) {
#pragma unroll
                for (int k = 0; k < TPL; k++) inv[u][mt][k] = invs[(size_t)un * TOK + lane_token<SPLIT>(mt, g, k)];
            }
        }
    }

    // 2. weight stream over items (tile j, unit u), u fastest; past the last
    //    tile the loads repeat the last one so every step issues one batch
    // packed weights: one buffer resource over the matrix (the host keeps it
    // below 4 GiB on this path)
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(W), (short)0, (int)(PK ? (uint32_t)n_tiles * n_units * Packed<QT>::CHUNK : 0u),
        0x00020000);
    auto load_item = [&](int j, int u, Unit<QT> &b) {
        j = min(j, my_tiles - 1);
        const int un = min(unit0 + u, n_units - 1);
        if constexpr (PK) {
            const int tile = (int)blockIdx.x + G * j;
            if constexpr (QT == QT_Q6_K)  // (its registers are full: global loads spill less)
                load_unit_packed<QT>(W + ((size_t)tile * n_units + un) * Packed<QT>::CHUNK, lane, b);
            else
                load_unit_buf<QT>(wrs, (tile * n_units + un) * Packed<QT>::CHUNK, lane, b);
        } else {
            const int row = min(((int)blockIdx.x + G * j) * 16 + n_in, N - 1);
            load_unit<QT>(W + (size_t)row * row_bytes + (size_t)un * UNIT_BYTES, g, un == n_units - 1 ? tail_blk : 8,
                          b);
        }
    };
    // chained producer: the old residual (EPI_RESID) and the next norm weight
    // of this wave's first epilogue tile, loaded now and used at the end
    // (the epilogue's jobs: with at most NW / 2 tiles, wave w takes token
    // 2 g + (w & 1) of tile slot w / 2; else tile slots w, w + NW, .. with both tokens)
    const bool spread = 2 * my_tiles <= NW;
    const int js0 = spread ? wave >> 1 : wave, k0 = spread ? wave & 1 : 0, k1 = spread ? k0 : 1;
    float pre_y0 = 0.f, pre_y1 = 0.f, pre_w = 1.f;
    auto load_pre = [&](int tile) {
        const int r = min(tile * 16 + n_in, N - 1);
        if (ch.epi == EPI_RESID) {
            pre_y0 = Y[(size_t)min(2 * g, M - 1) * ch.ldy + r];
            pre_y1 = Y[(size_t)min(2 * g + 1, M - 1) * ch.ldy + r];
        }
        pre_w = ch.yw != nullptr ? ch.yw[ch.epi == EPI_GATE ? tile * 8 + (n_in & 7) : r] : 1.f;
    };
    if constexpr (CE) {
        if (js0 < my_tiles) load_pre((int)blockIdx.x + G * js0);
    }
    // chained input: the exponents and tile sums of each unit, before the ring
    XStage xs[XIN ? UPS : 1];
    if constexpr (XIN) {
#pragma unroll
        for (int u = 0; u < UPS; u++)
            stage_unit_x<QT>(afrag, (const float *)mfrag, xs_stride, x_tpu, M, min(unit0 + u, n_units - 1), n_units,
                             lane, xs[u]);
    }
    RowScales<TOK, NW * 64> rsc;
    if constexpr (DE == 0) rsc.issue(ssq, n_ssq, tid);
    __builtin_amdgcn_sched_barrier(0);
    // the ring: R - 1 items in flight ahead of the one being consumed
    Unit<QT> buf[R];
#pragma unroll
    for (int p = 0; p < R - 1; p++) {
        load_item(p / UPS, p % UPS, buf[p]);
        __builtin_amdgcn_sched_barrier(0);  // ring slots fill in order
    }
    if constexpr (DE != 0) rsc.issue(ssq, n_ssq, tid);  // (needed after the loop only)
    if constexpr (XIN) {
        const bool tok = (n_in >> 1) < M;
#pragma unroll
        for (int u = 0; u < UPS; u++) {
            float iv[2];
            finish_unit_x<QT>(xs[u], x_tpu, tok && live[u], lane, a[u][0], iv);
            inv[u][0][0] = iv[0];
            inv[u][0][1] = iv[1];
        }
    }
    // (the row scales multiply outputs only: an epilogue after the loop takes
    // them there, so no wave waits here for the others' loads)
    // (without RMSNorm the scale is 1 and no wave waits for the others here)
    const bool has_rs = ssq != nullptr;
    if constexpr (DE == 0) {
        if (has_rs) rsc.finish(ssq, n_ssq, K, eps, tid, rsp, rs);
    }

    // a finished tile's plain epilogue: row scale, then the output, the
    // accumulation into it, or this K-slice's partials
    auto store_tile = [&](const float (&sum)[MT * TPL], int tile) {
        const int r = tile * 16 + n_in;
        if (r >= N) return;
#pragma unroll
        for (int k = 0; k < MT * TPL; k++) {
            const int t = lane_token<SPLIT>(k / TPL, g, k % TPL);
            if (t >= M) continue;
            const float v = has_rs ? sum[k] * rs[t] : sum[k];
            if (part != nullptr) {
                part[((size_t)blockIdx.y * M + t) * N + r] = v;
            } else {
                float *dst = Y + (size_t)t * ch.ldy + r;
                *dst = accum ? *dst + v : v;
            }
        }
    };
    f4 acc[MT], macc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[mt] = macc[mt] = f4{0.f, 0.f, 0.f, 0.f};
    auto consume = [&](int j, int u, Unit<QT> &b) {
        if constexpr (!PK) finish_unit<QT>(b);
        compute_v<QT, SPLIT, MT>(b, a[u], inv[u], g, live[u], acc, macc);
        if (u == UPS - 1) {
            float vals[MT * TPL];
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int k = 0; k < TPL; k++) {
                    float v = SPLIT ? acc[mt][2 * k] + acc[mt][2 * k + 1] : acc[mt][k];
                    if constexpr (C::MINS)
                        v -= 32.0f * (SPLIT ? macc[mt][2 * k] + macc[mt][2 * k + 1] : macc[mt][k]);
                    vals[mt * TPL + k] = v;
                }
            const int jb = j % F, hb = (j / F) & 1;
            float *slot = &red[hb][jb][wave][lane][0];
#pragma unroll
            for (int k = 0; k < MT * TPL; k++) slot[k] = vals[k];
#pragma unroll
            for (int mt = 0; mt < MT; mt++) acc[mt] = macc[mt] = f4{0.f, 0.f, 0.f, 0.f};
            // batch complete: wave i sums tile i of the batch in wave order
            if (jb == F - 1 || j == my_tiles - 1) __syncthreads();
            if ((jb == F - 1 || j == my_tiles - 1) && wave <= jb) {
                float sum[MT * TPL];
#pragma unroll
                for (int k = 0; k < MT * TPL; k++) sum[k] = red[hb][wave][0][lane][k];
#pragma unroll
                for (int w = 1; w < NW; w++)
#pragma unroll
                    for (int k = 0; k < MT * TPL; k++) sum[k] += red[hb][wave][w][lane][k];
                if constexpr (DE != 0) {
                    pend[j - jb + wave][lane] = make_float2(sum[0], sum[1]);
                } else {
                    store_tile(sum, (int)blockIdx.x + G * (j - jb + wave));
                }
            }
        }
    };
    const int n_items = my_tiles * UPS;
    const int n_full = n_items - n_items % R;
    for (int ib = 0; ib < n_full; ib += R) {
        const int jb = ib / UPS;
#pragma unroll
        for (int p = 0; p < R; p++) {
            load_item(jb + (p + R - 1) / UPS, (p + R - 1) % UPS, buf[(p + R - 1) % R]);
            consume(jb + p / UPS, p % UPS, buf[p]);
        }
    }
    {
        const int jb = n_full / UPS;
#pragma unroll
        for (int p = 0; p < R - 1; p++)
            if (n_full + p < n_items) consume(jb + p / UPS, p % UPS, buf[p]);
    }
    if constexpr (DE != 0) {
        // the epilogues, outside the weight loop (jobs as above; the row
        // scales' barriers also publish pend)
        static_assert(CE, "after-loop epilogues are the chained producer's");
        rsc.finish(ssq, n_ssq, K, eps, tid, rsp, rs);
        if constexpr (DE == 3) {
            // split over K: wave w stores its tiles' partial sums (this
            // slice's) and counts the slice in; the last slice to arrive at a
            // tile sums the slices in slice order (the same bits whichever
            // arrives last) and runs the tile's epilogue. No wave waits for
            // another: a tile's epilogue runs in whichever workgroup
            // completes it.
            // The partials and counts cross XCDs through device-scope
            // (agent) atomic stores, loads and adds, which the L2s keep
            // coherent by themselves; a wave waits for its partial's store
            // to complete before it counts the slice in (an agent-scope
            // fence would also write back and invalidate the whole L2:
            // measured 3x slower down projection).
            const int S = (int)gridDim.y, sl = (int)blockIdx.y;
            for (int js = wave; js < my_tiles; js += NW) {
                const int tile = (int)blockIdx.x + G * js;
                uint64_t *pt = (uint64_t *)(ch.tile_part + (size_t)tile * S * 64) + lane;
                __hip_atomic_store(pt + (size_t)sl * 64, __builtin_bit_cast(uint64_t, pend[js][lane]),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                wait_stores_done();  // (the partial lands before the count)
                int old = 0;
                if (lane == 0)
                    old = __hip_atomic_fetch_add(ch.tile_cnt + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                old = __shfl(old, 0);
                if (old != S - 1) continue;
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
                float2 acc = __builtin_bit_cast(float2, __hip_atomic_load(pt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
                for (int q = 1; q < S; q++) {
                    const float2 v = __builtin_bit_cast(
                        float2, __hip_atomic_load(pt + (size_t)q * 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
                    acc.x += v.x;
                    acc.y += v.y;
                }
                // (every slice has counted: zero again for the next call)
                if (lane == 0) __hip_atomic_store(ch.tile_cnt + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (spread || js != js0) load_pre(tile);
                chain_epilogue(ch, Y, acc.x, rs, M, N, tile, n_in, g, 0, pre_y0, pre_w);
                chain_epilogue(ch, Y, acc.y, rs, M, N, tile, n_in, g, 1, pre_y1, pre_w);
            }
            return;
        }
        for (int js = js0; js < my_tiles; js += NW) {
            const float2 p2 = pend[js][lane];
            const int tile = (int)blockIdx.x + G * js;
            // (the first tile's residual and weight were loaded at the start)
            if (js != js0) load_pre(tile);
#pragma unroll 1
            for (int k = k0; k <= k1; k++)
                chain_epilogue(ch, Y, k ? p2.y : p2.x, rs, M, N, tile, n_in, g, k, k ? pre_y1 : pre_y0, pre_w);
        }
    }
}

// ---------------------------------------------------------------- tall kernel
// One unit of one tile against MT register token tiles, finished: vals[mt *
// TPL + k] is the unit's contribution to token lane_token(mt, g, k) of row n
// (before the RMSNorm row scale).
//  Q4_K/Q5_K: inv * (d * (sc q . x) - 32 dmin * (m . X/32)), the 6-bit scales
//             folded into B exactly as in compute_v.
//  Q6_K: the int8 sub-block scale is folded into the fp16 weight operand
//             (q6_mfma_folded): half mode B = fp16(sc * q), one rounding;
//             fp32-accurate two exact terms. The MFMAs of a unit chain in
//             one accumulator per tile and d * inv is applied once: 2 (half)
//             or 3 VALU ops per weight pair instead of an fp32 fma per
//             sub-block, tile and output. (One tile keeps compute_v's
//             per-sub-block fp32 scaling, measured faster there.)
//  Q8_0: per-chunk fp32 scaling (compute_v).
template <int QT, bool SPLIT, int MT>
__device__ __forceinline__ void unit_vals(const Unit<QT> &r, const AReg<QT> (&a)[MT],
                                          const float (&inv)[MT][SPLIT ? 2 : 4], int g, bool live,
                                          float (&vals)[MT * (SPLIT ? 2 : 4)]) {
    constexpr int TPL = SPLIT ? 2 : 4;
    if constexpr (QT == QT_Q6_K && !SPLIT) {
        const float d = live ? half_bits(r.d) : 0.f;
        f4 c[MT];
        q6_mfma_folded<MT, false>(r, a, c);
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int k = 0; k < 4; k++) vals[mt * 4 + k] = (d * inv[mt][k]) * c[mt][k];
    } else if constexpr (QT == QT_Q6_K && SPLIT && MT >= 2) {
        // fp32-accurate with several tiles: the scales in the weight operand
        // as two exact fp16 terms (q6_mfma_folded); two packed ops per weight
        // pair replace an fp32 fma per sub-block, tile and output
        const float d = live ? half_bits(r.d) : 0.f;
        f4 c[MT];
        q6_mfma_folded<MT, true>(r, a, c);
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int k = 0; k < TPL; k++) vals[mt * TPL + k] = (d * inv[mt][k]) * (c[mt][2 * k] + c[mt][2 * k + 1]);
    } else if constexpr (QT == QT_Q4_K || QT == QT_Q5_K) {
        float d = half_bits(r.hdr.x), dmin = half_bits(r.hdr.x >> 16);
        if (!live) { d = 0.f; dmin = 0.f; }
        const KScales ks = k_scales<QT>(r.hdr, g);
        const uint32_t m_lo = ks.m_lo, m_hi = ks.m_hi;
        const h2 neg1024 = as_h2(0xE400E400u);  // (-1024, -1024)
        f4 c[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) c[mt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const h8 bf = k_frag<QT>(r, m, g, ks);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) c[mt] = mfma32(a[mt].f[m], bf, c[mt]);
        }
        const uint32_t mw = g == 0 ? m_lo : (g == 1 ? m_hi : 0u);
        const h2 p0 = as_h2(pair_lo(mw)) + neg1024, p1 = as_h2(pair_hi(mw)) + neg1024;
        h4 bm;
        bm[0] = p0[0]; bm[1] = p0[1]; bm[2] = p1[0]; bm[3] = p1[1];
        const float dm32 = -32.0f * dmin;
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const f4 cm = mfma16(a[mt].mins, bm, f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int k = 0; k < TPL; k++) {
                const float s = SPLIT ? c[mt][2 * k] + c[mt][2 * k + 1] : c[mt][k];
                const float sm = SPLIT ? cm[2 * k] + cm[2 * k + 1] : cm[k];
                vals[mt * TPL + k] = inv[mt][k] * __builtin_fmaf(dm32, sm, d * s);
            }
        }
    } else {
        f4 acc[MT], macc[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[mt] = macc[mt] = f4{0.f, 0.f, 0.f, 0.f};
        compute_v<QT, SPLIT, MT>(r, a, inv, g, live, acc, macc);
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int k = 0; k < TPL; k++) vals[mt * TPL + k] = SPLIT ? acc[mt][2 * k] + acc[mt][2 * k + 1] : acc[mt][k];
    }
}

// Most units (of 256 K) per wave of the one-tile streaming kernel that fit
// its registers without spilling: each unit of A operand is 32 VGPRs (one
// tile), and the larger Q5_K/Q6_K/Q8_0 items leave less room.
__host__ __device__ constexpr int stream_ups_cap(int qt, bool split) {
    return qt == QT_Q4_K ? (split ? 4 : 2) : qt == QT_Q5_K ? 2 : qt == QT_Q6_K ? (split ? 2 : 1) : 1;
}

// Waves per workgroup of the tall kernel: two per SIMD (8) where the A
// operand, the ring (4-deep, 2-deep for the larger Q5_K/Q6_K items at 4
// tiles, which Q6_K also prefers when it fits) and the rest fit in 256
// registers without spilling (two waves then
// overlap one's MFMAs with the other's dequantization), else one per SIMD
// (4) with the full register file. (fp32-accurate Q6_K fits since its scales
// go into the weight operand as two exact fp16 terms.) Independent of the
// weight layout, so packed and GGUF-layout weights sum the same K-slices in
// the same order.
__host__ __device__ constexpr int tall_waves(int qt, bool split, int mt) {
    return (qt == QT_Q4_K || qt == QT_Q5_K || qt == QT_Q6_K || (qt == QT_Q8_0 && mt <= 2)) ? 8 : 4;
}

// Several token tiles (M up to 32 fp32-accurate, 64 half): NW = 4 or 8
// waves (one or two per SIMD, tall_waves), each holding one 256-element
// unit of the A operand for all MT tiles in registers, so a dequantized
// weight fragment feeds MT MFMAs. A workgroup covers NW units (one K-slice,
// grid.y) of every G-th 16-row tile (grid.x). Per tile the waves' unit
// results meet in LDS (value-group major, so a group's 64 lanes hit
// distinct banks); they are gathered in batches of F tiles (4, or 2 with
// two waves per SIMD; double-buffered, one barrier per batch) and summed in
// wave order, the work spread evenly over the waves. Weight items stream
// through a register ring (8, 4 or 2 deep by register budget). Results go
// out with bounds-checked buffer stores, the same number on every path (no
// branches, no read-modify-write in the loop): to the K-slice's partials
// when part is set (the caller reduces or folds them), else to Y.
template <int QT, bool SPLIT, bool PK, int MT, int NW>
__global__ __launch_bounds__(NW * 64, 1)
void gemm_w_kernel(const uint8_t *__restrict__ W, float *__restrict__ Y, int M, int N, int K,
                   const uint8_t *__restrict__ afrag, const float *__restrict__ invs,
                   const uint8_t *__restrict__ mfrag, const float *__restrict__ ssq, float eps,
                   float *__restrict__ part) {
    using C = GemmCfg<QT>;
    static_assert(NW == 4 || NW == 8, "one or two waves per SIMD");
    constexpr int TOKT = SPLIT ? 8 : 16;
    constexpr int TOK = MT * TOKT;
    constexpr int TPL = SPLIT ? 2 : 4;
    constexpr int NV = MT * TPL;           // results per lane and tile
    constexpr int NVP = (NV + 3) & ~3;     // (padded to whole 16-byte LDS accesses)
    constexpr int UNIT_BYTES = (QT == QT_Q8_0) ? 8 * 34 : C::BB;
    // ring depth: 8 items where the registers allow it (Q8_0 items and the
    // fp32-accurate Q6_K operands are larger)
    // (two waves per SIMD: half the registers each, a 4-deep ring and
    // batches of 2 tiles, each tile summed by 4 waves a value group each)
    constexpr int R = (NW == 8 && MT == 4 && (QT == QT_Q5_K || QT == QT_Q6_K)) ? 2
                      : (NW == 8 || QT == QT_Q8_0 || (QT == QT_Q6_K && SPLIT)) ? 4 : 8;
    constexpr int F = NW == 8 ? 2 : 4;
    constexpr int WPT = NW / F;  // waves per tile in a batch's reduction
    static_assert(R % F == 0, "a ring pass holds whole reduction batches");
    // [batch half][tile][wave][value group][lane]: 16-byte lane stride, so
    // the 64 lanes' 16-byte accesses of a value group hit distinct banks
    __shared__ __align__(16) f4 red[2][F][NW][NVP / 4][64];
    __shared__ float rs[TOK];
    __shared__ float rsp[NW * 64];

    const int n_units = (K + UNIT - 1) / UNIT;
    const int n_tiles = (N + 15) / 16;
    const int G = gridDim.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n_in = lane & 15, g = lane >> 4;
    const int my_tiles = (n_tiles - 1 - (int)blockIdx.x) / G + 1;  // the plan keeps G <= n_tiles
    const int unit = (int)blockIdx.y * NW + wave;
    const bool live = unit < n_units;
    const int un = min(unit, n_units - 1);
    const size_t row_bytes = (size_t)(K / C::QK) * C::BB;
    const int tail_blk = (QT == QT_Q8_0 && (K % UNIT)) ? (K % UNIT) / 32 : 8;

    // 1. weight stream over this workgroup's tiles; past the last tile the
    //    loads repeat it so every ring step issues one item
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(W), (short)0, (int)(PK ? (uint32_t)n_tiles * n_units * Packed<QT>::CHUNK : 0u),
        0x00020000);
    auto load_item = [&](int j, Unit<QT> &b) {
        j = min(j, my_tiles - 1);
        if constexpr (PK) {
            const int tile = (int)blockIdx.x + G * j;
            if constexpr (QT == QT_Q6_K)
                load_unit_packed<QT>(W + ((size_t)tile * n_units + un) * Packed<QT>::CHUNK, lane, b);
            else
                load_unit_buf<QT>(wrs, (tile * n_units + un) * Packed<QT>::CHUNK, lane, b);
        } else {
            const int row = min(((int)blockIdx.x + G * j) * 16 + n_in, N - 1);
            load_unit<QT>(W + (size_t)row * row_bytes + (size_t)un * UNIT_BYTES, g, un == n_units - 1 ? tail_blk : 8,
                          b);
        }
    };

    // 2. loads. With two waves per SIMD (PEEL: the first ring pass is peeled
    //    below) in the order they are needed: the RMSNorm partial sums
    //    (waited for before the loop, so issued first), the first weight
    //    item, this wave's A operand chunk by chunk for all MT tiles (the
    //    MFMA lane layout: entry (chunk c, tile mt) at (c MT + mt) 64 + lane,
    //    so the first item's MFMAs start as their chunks land instead of
    //    after the whole 256-element unit), the inverse unit scales, then the
    //    rest of the ring (padding tokens' slots are read too: the input
    //    stage writes zero operands and unit scales for every token up to
    //    TOK). Without the peeled pass the loop's head is entered straight
    //    from here, so the A operand goes first, tile by tile, and is
    //    complete when the RMSNorm sums are (in-order completion): the
    //    need-ordered prologue there merged operand waits into every pass
    //    and drained the ring (the 4-tile fp32-accurate Q6_K kernel, 25 %
    //    slower).
    constexpr bool PEEL = NW == 8;  // (one wave per SIMD: the copies would no longer be inlined)
    AReg<QT> a[MT];
    float inv[MT][TPL];
    auto load_a = [&]() __attribute__((always_inline)) {
        const uint8_t *src = afrag + (size_t)un * UNIT_A1 * MT;
        if constexpr (QT == QT_Q6_K) {
#pragma unroll
            for (int c = 0; c < 16; c++)
#pragma unroll
                for (int mt = 0; mt < MT; mt++) a[mt].f[c] = *(const h4 *)(src + ((c * MT + mt) * 64 + lane) * 8);
        } else {
#pragma unroll
            for (int c = 0; c < 8; c++)
#pragma unroll
                for (int mt = 0; mt < MT; mt++) a[mt].f[c] = *(const h8 *)(src + ((c * MT + mt) * 64 + lane) * 16);
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            if constexpr (C::MINS) a[mt].mins = *(const h4 *)(mfrag + ((size_t)un * MT + mt) * 512 + lane * 8);
#pragma unroll
            for (int k = 0; k < TPL; k++) inv[mt][k] = invs[(size_t)un * TOK + lane_token<SPLIT>(mt, g, k)];
        }
    };
    RowScales<TOK, NW * 64> rsc;
    Unit<QT> buf[R];
    if constexpr (PEEL) {
        rsc.issue(ssq, n_units, tid);
        __builtin_amdgcn_sched_barrier(0);
        load_item(0, buf[0]);
        __builtin_amdgcn_sched_barrier(0);
        load_a();
        __builtin_amdgcn_sched_barrier(0);
    } else {
        // (tile by tile; slots of padding tokens are zero, not fetched)
        const uint8_t *src = afrag + (size_t)un * UNIT_A1 * MT;
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            if ((SPLIT ? (n_in >> 1) : n_in) + mt * TOKT < M) {
                if constexpr (QT == QT_Q6_K) {
#pragma unroll
                    for (int c = 0; c < 16; c++) a[mt].f[c] = *(const h4 *)(src + ((c * MT + mt) * 64 + lane) * 8);
                } else {
#pragma unroll
                    for (int c = 0; c < 8; c++) a[mt].f[c] = *(const h8 *)(src + ((c * MT + mt) * 64 + lane) * 16);
                }
                if constexpr (C::MINS) a[mt].mins = *(const h4 *)(mfrag + ((size_t)un * MT + mt) * 512 + lane * 8);
            } else {
                if constexpr (QT == QT_Q6_K) {
#pragma unroll
                    for (int c = 0; c < 16; c++) a[mt].f[c] = h4{};
                } else {
#pragma unroll
                    for (int c = 0; c < 8; c++) a[mt].f[c] = h8{};
                }
                if constexpr (C::MINS) a[mt].mins = h4{};
            }
#pragma unroll
            for (int k = 0; k < TPL; k++) inv[mt][k] = invs[(size_t)un * TOK + lane_token<SPLIT>(mt, g, k)];
        }
        rsc.issue(ssq, n_units, tid);
        __builtin_amdgcn_sched_barrier(0);
        load_item(0, buf[0]);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int p = 1; p < R - 1; p++) {
        load_item(p, buf[p]);
        __builtin_amdgcn_sched_barrier(0);  // ring slots fill in order
    }
    // output: element (t, r) at byte 4 (t N + r) of this K-slice's [M x N]
    // block, the token's tile part in the scalar offset, the lane part (row
    // r, token base tb) in the vector offset; tokens at or past M land at or
    // past the resource's size, and padding rows get an offset past it, so
    // those stores are dropped
    float *dst = part != nullptr ? part + (size_t)blockIdx.y * M * N : Y;
    const uint32_t out_bytes = (uint32_t)((size_t)M * N * 4);
    const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(dst, (short)0, (int)out_bytes, 0x00020000);
    const int tb = lane_token<SPLIT>(0, g, 0);
    rsc.finish(ssq, n_units, K, eps, tid, rsp, rs);
    // as many dropped stores (offset past the resource) as a flush issues,
    // behind the ring's prologue loads: the main loop is entered with the
    // same memory operations in flight as its back edge leaves, so the wait
    // at its head lets the ring's later items stay in flight
    constexpr int FLUSH_STORES = 4 * ((NVP / 4 + WPT - 1) / WPT);
#pragma unroll
    for (int i = 0; i < FLUSH_STORES; i++)
        __builtin_amdgcn_raw_buffer_store_b32(0u, ors, (int)0x80000000u, 4 * i, 0);  // (distinct: kept)

    // flush (a batch is complete): wave i sums tile i of the batch in wave
    // order and stores it
    auto consume = [&](int j, int jb, bool flush, Unit<QT> &b) __attribute__((always_inline)) {
        if constexpr (!PK) finish_unit<QT>(b);
        float vals[NVP];
        unit_vals<QT, SPLIT, MT>(b, a, inv, g, live, *(float(*)[NV])vals);
#pragma unroll
        for (int k = NV; k < NVP; k++) vals[k] = 0.f;
        const int hb = (j / F) & 1;
#pragma unroll
        for (int k = 0; k < NVP; k += 4) red[hb][jb][wave][k / 4][lane] = f4{vals[k], vals[k + 1], vals[k + 2], vals[k + 3]};
        if (flush) {
            __syncthreads();
            // Branch-free: every wave issues the same stores on every path
            // (a wave without a tile or value group stores past the
            // resource's end), so the wait counts the compiler places for
            // the ring's next items count these stores exactly instead of
            // draining the prefetched loads behind them.
            const int tl = wave / WPT, grp = wave % WPT;  // tile of the batch, first value group
            const bool tok = tl <= jb;
            const int tlc = tok ? tl : jb;
            const int r = ((int)blockIdx.x + G * (j - jb + tlc)) * 16 + n_in;
            const uint32_t voff = (tok && r < N) ? (uint32_t)(tb * N + r) * 4u : 0x80000000u;
            constexpr int QG = NVP / 4, QPW = (QG + WPT - 1) / WPT;  // value groups, per wave
#pragma unroll
            for (int i = 0; i < QPW; i++) {
                const int q0 = grp + WPT * i;
                const int q = q0 < QG ? q0 : QG - 1;
                // all waves' slices first (one LDS wait), then the sum in wave order
                f4 pv[NW];
#pragma unroll
                for (int w = 0; w < NW; w++) pv[w] = red[hb][tlc][w][q][lane];
                f4 sum = pv[0];
#pragma unroll
                for (int w = 1; w < NW; w++) sum += pv[w];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int k = min(4 * q + e, NV - 1);
                    const bool kok = q0 < QG && 4 * q + e < NV;
                    const int tk = lane_token<SPLIT>(k / TPL, 0, k % TPL);
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, sum[e] * rs[tb + tk]), ors,
                                                          kok ? (int)voff : (int)0x80000000u,
                                                          __builtin_amdgcn_readfirstlane(tk * N * 4), 0);
                }
            }
        }
    };
    // whole ring passes: every R-th item completes a batch at a fixed ring
    // position (straight-line code); the last partial pass checks the end.
    // With two waves per SIMD the first pass is peeled and the loop nested
    // under it: its memory waits follow the prologue's order (the first
    // item's MFMAs wait for the A operand chunk by chunk), and the loop is
    // entered only from a pass that leaves the same operations in flight as
    // its own back edge, so its waits stay exact.
    const int n_full = my_tiles - my_tiles % R;
    auto pass = [&](int ib) __attribute__((always_inline)) {
#pragma unroll
        for (int p = 0; p < R; p++) {
            load_item(ib + p + R - 1, buf[(p + R - 1) % R]);
            // (two waves per SIMD: the loads stay at the head of their step;
            // under that register budget the scheduler sinks them to the end
            // of the pass, next to their use, and the ring stops prefetching)
            if constexpr (NW == 8) __builtin_amdgcn_sched_barrier(0);
            consume(ib + p, p % F, p % F == F - 1, buf[p]);
        }
    };
    if constexpr (PEEL) {
        if (n_full > 0) {
            pass(0);
            for (int ib = R; ib < n_full; ib += R) pass(ib);
        }
    } else {
        for (int ib = 0; ib < n_full; ib += R) {
#pragma unroll
            for (int p = 0; p < R; p++) {
                load_item(ib + p + R - 1, buf[(p + R - 1) % R]);
                consume(ib + p, p % F, p % F == F - 1, buf[p]);
            }
        }
    }
#pragma unroll
    for (int p = 0; p < R - 1; p++)
        if (n_full + p < my_tiles) consume(n_full + p, p % F, p % F == F - 1 || n_full + p == my_tiles - 1, buf[p]);
}

// Prepared-activation workspace (shared by both kernels): the A operand,
// the Q4_K/Q5_K sub-block sums (LDS kernel) or min-term operand (streaming
// kernel), the inverse unit scales and the RMSNorm partial sums.
struct ActWs {
    uint8_t *afrag;
    float *xs, *inv;
    uint8_t *mfrag;
    float *ssq;
};

// Integer tuning override from the environment (read once per call site).
int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    return v ? atoi(v) : dflt;
}

// compact: the one-token-tile streaming kernel's operand layout (entry c,
// lane group G, slot s at (4 c + G) sl + s with sl = the slots of M tokens);
// otherwise 64 lanes per entry (the tall and LDS kernels).
template <int QT, int MT, bool SPLIT>
hipError_t launch_prep(const float *X, const ActIn &in, int M, int K, const ActWs &a, hipStream_t st,
                       bool compact = false) {
    using C = GemmCfg<QT>;
    constexpr int TOK = MT * (SPLIT ? 8 : 16);
    const int n_units = (K + UNIT - 1) / UNIT;
    constexpr int LK = QT == QT_Q6_K ? 1 : QT == QT_Q8_0 ? 2 : 0;
    // tokens per workgroup: 2 (one wave) spreads the stage over the most CUs
    // (measured: the verify step 1.1 % faster than 8 per workgroup; the
    // M = 64 tree forward unchanged); IHIP_PREP_TPW selects 4 or 8
    static const int tpw = env_int("IHIP_PREP_TPW", 2);
    // (sum_out: workgroups past the input's units fold and store its other columns)
    const int tail_units = (X == nullptr && in.sum_out != nullptr) ? (in.ldx - K + UNIT - 1) / UNIT : 0;
    float *xw = X != nullptr ? const_cast<float *>(X) : in.sum_out;
#define PREP(tp) prep_kernel<LK, MT, SPLIT, C::MINS, tp><<<dim3(n_units + tail_units, TOK / tp), 32 * tp, 0, st>>>( \
        X, in.ldx, M, K, in.op, in.norm_w, a.afrag, a.xs, a.inv, a.mfrag, a.ssq, in.add, in.n_add, in.add_stride, \
        xw, sl)
    const int sl = compact ? (SPLIT ? 2 * M : M) : 0;
    if (tpw == 2) PREP(2); else if (tpw == 4) PREP(4); else PREP(8);
#undef PREP
    return hipGetLastError();
}

// The store-only epilogue of an unchained call (rows of Y are N apart).
inline Chain plain_chain(int N) {
    Chain c{};
    c.epi = EPI_STORE;
    c.ldy = N;
    return c;
}

template <int QT, int NW, int UPS, bool SPLIT, bool PK, int MT>
hipError_t launch_v(const uint8_t *W, const float *X, const ActIn &in, float *Y, int M, int N, int K, int S, int G,
                    int accum, const ActWs &a, float *part, hipStream_t st, const Chain *chain = nullptr) {
    hipError_t e;
    if (!in.reuse && (e = launch_prep<QT, MT, SPLIT>(X, in, M, K, a, st, true)) != hipSuccess) return e;
    const int n_units = (K + UNIT - 1) / UNIT;
    // (a chained producer's epilogue is its own instantiation: classic calls keep their registers)
    const Chain c = chain != nullptr ? *chain : plain_chain(N);
    // (the chained calls' plans: 8 waves, or Q6_K's 4 waves of 3 units)
    if constexpr (SPLIT && MT == 1 && PK && (NW == 8 || (QT == QT_Q6_K && NW == 4 && UPS == 3))) {
        if (c.epi != EPI_STORE && S > 1) {  // (a chained epilogue sums its own K-slices)
            gemm_v_kernel<QT, NW, UPS, SPLIT, PK, MT, false, 3><<<dim3(G, S), NW * 64, 0, st>>>(
                W, a.afrag, a.mfrag, a.inv, M, N, K, G, 0, 0, Y, accum, in.op == ACT_RMSNORM ? a.ssq : nullptr,
                n_units, in.eps, part, c);
            return hipGetLastError();
        }
        if (c.epi != EPI_STORE) {
            gemm_v_kernel<QT, NW, UPS, SPLIT, PK, MT, false, 2><<<dim3(G, S), NW * 64, 0, st>>>(
                W, a.afrag, a.mfrag, a.inv, M, N, K, G, 0, 0, Y, accum, in.op == ACT_RMSNORM ? a.ssq : nullptr,
                n_units, in.eps, in.defer ? part : nullptr, c);
            return hipGetLastError();
        }
    }
    gemm_v_kernel<QT, NW, UPS, SPLIT, PK, MT, false, 0><<<dim3(G, S), NW * 64, 0, st>>>(
        W, a.afrag, a.mfrag, a.inv, M, N, K, G, 0, 0, Y, accum, in.op == ACT_RMSNORM ? a.ssq : nullptr, n_units,
        in.eps, (S > 1 || in.defer) ? part : nullptr, c);
    e = hipGetLastError();
    if (e != hipSuccess || S == 1 || in.defer) return e;
    const int64_t MN = (int64_t)M * N;
    reduce_kernel<<<(unsigned)((MN + 1023) / 1024), 256, 0, st>>>(part, Y, S, MN, accum);
    return hipGetLastError();
}

// A chained call whose input comes from a chained producer (XIN): no input
// stage; RMSNorm row scales from the producer's tile sums of squares.
template <int QT, int NW, int UPS>
hipError_t launch_vx(const uint8_t *W, float *Y, int M, int N, int K, int S, int G, int defer, const float *ssq,
                     int n_ssq, float eps, float *part, const Chain &ch, hipStream_t st) {
    // (the operand, its tile sums and their layout travel in the leading
    // arguments, which the hardware preloads into SGPRs)
    const uint8_t *xs = (const uint8_t *)ch.xsum;
    if (ch.epi != EPI_STORE && S > 1)  // (the last K-slice at a tile finishes it)
        gemm_v_kernel<QT, NW, UPS, true, true, 1, true, 3><<<dim3(G, S), NW * 64, 0, st>>>(
            W, ch.xop, xs, nullptr, M, N, K, G, ch.xsum_stride, ch.x_tiles_per_unit, Y, 0, ssq, n_ssq, eps, part, ch);
    else if (ch.epi != EPI_STORE)
        gemm_v_kernel<QT, NW, UPS, true, true, 1, true, 2><<<dim3(G, S), NW * 64, 0, st>>>(
            W, ch.xop, xs, nullptr, M, N, K, G, ch.xsum_stride, ch.x_tiles_per_unit, Y, 0, ssq, n_ssq, eps,
            (S > 1 || defer) ? part : nullptr, ch);
    else
        gemm_v_kernel<QT, NW, UPS, true, true, 1, true, 0><<<dim3(G, S), NW * 64, 0, st>>>(
            W, ch.xop, xs, nullptr, M, N, K, G, ch.xsum_stride, ch.x_tiles_per_unit, Y, 0, ssq, n_ssq, eps,
            (S > 1 || defer) ? part : nullptr, ch);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || S == 1 || defer || ch.epi != EPI_STORE) return e;
    const int64_t MN = (int64_t)M * N;
    reduce_kernel<<<(unsigned)((MN + 1023) / 1024), 256, 0, st>>>(part, Y, S, MN, 0);
    return hipGetLastError();
}

template <int QT, bool SPLIT, bool PK, int MT, int NW>
hipError_t launch_w(const uint8_t *W, const float *X, const ActIn &in, float *Y, int M, int N, int K, int S, int G,
                    int accum, const ActWs &a, float *part, hipStream_t st) {
    hipError_t e;
    if (!in.reuse && (e = launch_prep<QT, MT, SPLIT>(X, in, M, K, a, st)) != hipSuccess) return e;
    // several K-slices, accumulation and deferral all go through the
    // partials (the kernel itself never reads its output)
    const bool via_part = S > 1 || accum || in.defer;
    gemm_w_kernel<QT, SPLIT, PK, MT, NW><<<dim3(G, S), NW * 64, 0, st>>>(
        W, Y, M, N, K, a.afrag, a.inv, a.mfrag, in.op == ACT_RMSNORM ? a.ssq : nullptr, in.eps,
        via_part ? part : nullptr);
    e = hipGetLastError();
    if (e != hipSuccess || !via_part || in.defer) return e;
    const int64_t MN = (int64_t)M * N;
    reduce_kernel<<<(unsigned)((MN + 1023) / 1024), 256, 0, st>>>(part, Y, S, MN, accum);
    return hipGetLastError();
}

template <int QT, int MT, bool SPLIT, bool PK>
hipError_t launch_t(const uint8_t *W, const float *X, const ActIn &in, float *Y, int M, int N, int K, int ups, int S,
                    int G, int accum, const ActWs &a, float *part, hipStream_t st) {
    using C = GemmCfg<QT>;
    constexpr int TOK = MT * (SPLIT ? 8 : 16);
    hipError_t e;
    if (!in.reuse && (e = launch_prep<QT, MT, SPLIT>(X, in, M, K, a, st)) != hipSuccess) return e;
    const size_t lds = (size_t)ups * UNIT_A1 * MT + (C::MINS ? (size_t)ups * 8 * TOK * 4 : 0) + (size_t)ups * TOK * 4;
    if (lds > 65536) {
        e = hipFuncSetAttribute((const void *)gemm_q_kernel<QT, MT, SPLIT, PK>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    const bool reduce = S > 1 || accum;
    gemm_q_kernel<QT, MT, SPLIT, PK><<<dim3(G, S), WG_THREADS, lds, st>>>(
        W, Y, M, N, K, ups, S, a.afrag, a.xs, a.inv, in.op == ACT_RMSNORM ? a.ssq : nullptr, in.eps,
        (reduce || in.defer) ? part : nullptr);
    e = hipGetLastError();
    if (e != hipSuccess || !reduce || in.defer) return e;
    const int64_t MN = (int64_t)M * N;
    reduce_kernel<<<(unsigned)((MN + 1023) / 1024), 256, 0, st>>>(part, Y, S, MN, accum);
    return hipGetLastError();
}

}  // namespace

// ---------------------------------------------------------------- host plan
struct GemmPlan {
    bool split;      // fp32-accurate two-limb mode
    int MT;          // MFMA token tiles (16 slots each)
    bool stream;     // streaming kernel with register operands (else the LDS kernel)
    int NW, UPS;     // streaming kernel: waves per workgroup, units per wave
    int ups;         // LDS kernel: 256-element units per K-slice
    int S;           // K-slices (grid.y)
    int G;           // workgroups per K-slice (grid.x)
    size_t off_xs, off_inv, off_mfrag, off_ssq, off_part, off_cnt, ws_bytes;
};

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }


size_t packed_bytes(int qt, int N, int K);

static GemmPlan plan_gemm(int qt, int M, int N, int K, int flags) {
    GemmPlan p{};
    const bool force_f32 = flags & 1, force_half = flags & 2;
    p.split = force_f32 ? true : force_half ? false : (M < 16);
    p.MT = p.split ? (M + 7) / 8 : (M + 15) / 16;
    const int n_units = (K + UNIT - 1) / UNIT;
    const int TOK = p.MT * (p.split ? 8 : 16);
    const bool mins = (qt == QT_Q4_K || qt == QT_Q5_K);
    // tuning overrides: IHIP_GEMM_WGS (target workgroups), IHIP_GEMM_LDS_A
    // (A-operand bytes per workgroup, LDS kernel), IHIP_STREAM_UPS (streaming
    // kernel units per wave), IHIP_STREAM=0 (LDS kernel)
    static const int target = env_int("IHIP_GEMM_WGS", 1024);
    static const int lds_a = env_int("IHIP_GEMM_LDS_A", 32768);
    static const int use_stream = env_int("IHIP_STREAM", 1);
    static const int env_ups = env_int("IHIP_STREAM_UPS", 0);
    // (the streaming kernels address packed weights, and the tall kernel its
    // outputs, with 32-bit offsets: larger cases take the LDS kernel)
    static const int stream_mt = env_int("IHIP_STREAM_MT", 4);
    p.stream = use_stream && p.MT <= stream_mt && !((flags & 8) && packed_bytes(qt, N, K) >= ((size_t)1 << 31)) &&
               !(p.MT > 1 && (size_t)p.MT * 16 * N * 4 >= ((size_t)1 << 31));
    if (p.stream && p.MT > 1) {
        // several token tiles: their A operand fills the registers; 4 waves
        // (one per SIMD) or 8 (two per SIMD, IHIP_TALL_NW=8) of one unit
        // each per workgroup, one workgroup per CU
        // (IHIP_TALL_NW=4: one wave per SIMD throughout)
        static const int tall_nw = env_int("IHIP_TALL_NW", 0);
        p.NW = tall_nw != 4 ? tall_waves(qt, p.split, p.MT) : 4;
        p.UPS = 1;
        p.S = (n_units + p.NW - 1) / p.NW;
        const int n_tiles = (N + 15) / 16;
        const int g0 = std::max(1, std::min(n_tiles, 256 / p.S));
        const int per = (n_tiles + g0 - 1) / g0;
        p.G = (n_tiles + per - 1) / per;
    } else if (p.stream) {
        // K per workgroup NW*UPS units (UPS at most stream_ups_cap); prefer
        // one K-slice (no partials) with the fewest units per wave that still
        // covers K, else the largest chunk that divides K
        static const int env_nw = env_int("IHIP_STREAM_NW", 8);
        const int nw = env_nw == 8 ? 8 : 4;
        const int cap = stream_ups_cap(qt, p.split);
        int ups = cap;
        if (env_ups == 1 || env_ups == 2 || env_ups == 4) {
            ups = std::min(env_ups, cap);
        } else {
            for (int u : {1, 2, 4})
                if (u <= cap && nw * u >= n_units) { ups = u; break; }
            if (nw * ups < n_units)
                for (int u : {4, 2, 1})
                    if (u <= cap && n_units % (nw * u) == 0) { ups = u; break; }
        }
        p.NW = nw;
        p.UPS = ups;
        p.S = (n_units + nw * ups - 1) / (nw * ups);
        if (qt == QT_Q6_K && p.split && nw == 8 && env_ups == 0 && n_units % 12 == 0 && n_units >= 24) {
            // Q6_K past one 8 x 2-unit slice (down, 48 units): 4 waves of 3
            // units, one wave per SIMD with the full register file and a
            // 6-deep ring, 12-unit K-slices: 4 slices x 64 workgroups of 4
            // tiles fill all 256 CUs with 12 items per wave (the 8 x 2 plan:
            // 3 slices x 64 workgroups on 192 CUs; verify step 1.5 % faster)
            p.NW = 4;
            p.UPS = 3;
            p.S = n_units / 12;
        }
        // every workgroup resident at once (2 per CU at <= 256 VGPRs) and the
        // same number of tiles for each: no second dispatch wave, no tail
        // where half the workgroups idle
        static const int stream_target = env_int("IHIP_GEMM_WGS", 0);
        // workgroups the chip holds (4-wave ones two per CU at <= 256 VGPRs, one with 3 units)
        const int resident = (p.NW == 8 || p.UPS == 3) ? 256 : 512;
        const int target = stream_target > 0 ? stream_target : resident;
        const int n_tiles = (N + 15) / 16;
        const int g0 = std::max(1, std::min(n_tiles, target / p.S));
        const int per = (n_tiles + g0 - 1) / g0;
        p.G = (n_tiles + per - 1) / per;
    } else {
        const int rowgroups = (N + ROWS_PER_WG - 1) / ROWS_PER_WG;
        const int ups_max = std::max(1, lds_a / (UNIT_A1 * p.MT));
        p.S = (n_units + ups_max - 1) / ups_max;
        p.ups = (n_units + p.S - 1) / p.S;
        p.S = (n_units + p.ups - 1) / p.ups;
        p.G = std::max(1, std::min(rowgroups, (target + p.S - 1) / p.S));
    }
    size_t o = align256((size_t)n_units * UNIT_A1 * p.MT);
    p.off_xs = o;
    o += (mins && !p.stream) ? align256((size_t)n_units * 8 * TOK * 4) : 0;
    p.off_inv = o;
    o += align256((size_t)n_units * TOK * 4);
    p.off_mfrag = o;
    o += (mins && p.stream) ? align256((size_t)n_units * 512 * p.MT) : 0;
    p.off_ssq = o;
    o += align256((size_t)n_units * TOK * 4);
    p.off_part = o;
    // partials (split-K or accumulate; a K-split chained epilogue's
    // [tile][slice][64] float2), then that epilogue's per-tile slice counts
    const size_t tiles16 = (size_t)(N + 15) / 16;
    o += align256(std::max((size_t)p.S * M * N * 4, p.S > 1 ? (size_t)p.S * tiles16 * 512 : 0));
    p.off_cnt = o;
    o += align256(tiles16 * 4);
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

template <int QT, bool PK>
static hipError_t dispatch_mt(const GemmPlan &p, const uint8_t *W, const float *X, const ActIn &in, float *Y, int M,
                              int N, int K, int accum, uint8_t *ws, hipStream_t st) {
    // the sub-block sums feed only the LDS kernel, the min-term operand only
    // the streaming kernel (the other has no room for them in the workspace)
    const ActWs a{ws, p.stream ? nullptr : (float *)(ws + p.off_xs), (float *)(ws + p.off_inv),
                  p.stream ? ws + p.off_mfrag : nullptr, (float *)(ws + p.off_ssq)};
    float *part = (float *)(ws + p.off_part);
    if (p.stream && p.MT > 1) {
#define WM(mt, nw) return p.split ? launch_w<QT, true, PK, mt, nw>(W, X, in, Y, M, N, K, p.S, p.G, accum, a, part, st) \
                              : launch_w<QT, false, PK, mt, nw>(W, X, in, Y, M, N, K, p.S, p.G, accum, a, part, st)
        // (8 waves instantiated only where tall_waves allows two per SIMD)
        if (p.NW == 8) {
#define W8(sp, mt) if constexpr (tall_waves(QT, sp, mt) == 8) if (p.split == sp && p.MT == mt) \
    return launch_w<QT, sp, PK, mt, 8>(W, X, in, Y, M, N, K, p.S, p.G, accum, a, part, st)
            W8(true, 2); W8(true, 3); W8(true, 4); W8(false, 2); W8(false, 3); W8(false, 4);
#undef W8
            return hipErrorInvalidValue;  // (the plan picks 8 waves only where instantiated)
        }
        switch (p.MT) { case 2: WM(2, 4); case 3: WM(3, 4); default: WM(4, 4); }
#undef WM
    }
    if (p.stream) {
        // (instantiated up to the units per wave stream_ups_cap allows)
#define V(nw, u, sp) if constexpr (u <= stream_ups_cap(QT, sp)) if (p.NW == nw && p.UPS == u && p.split == sp) \
    return launch_v<QT, nw, u, sp, PK, 1>(W, X, in, Y, M, N, K, p.S, p.G, accum, a, part, st)
        V(8, 1, true); V(8, 2, true); V(8, 4, true); V(8, 1, false); V(8, 2, false); V(8, 4, false);
        if constexpr (QT == QT_Q6_K)
            if (p.NW == 4 && p.UPS == 3 && p.split)
                return launch_v<QT, 4, 3, true, PK, 1>(W, X, in, Y, M, N, K, p.S, p.G, accum, a, part, st);
        V(4, 1, true); V(4, 2, true); V(4, 4, true); V(4, 1, false); V(4, 2, false); V(4, 4, false);
#undef V
        return hipErrorInvalidValue;  // (the plan keeps UPS within the cap)
    }
#define L(mt, sp) return launch_t<QT, mt, sp, PK>(W, X, in, Y, M, N, K, p.ups, p.S, p.G, accum, a, part, st)
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

size_t packed_bytes(int qt, int N, int K) {
    const size_t tiles = (size_t)(N + 15) / 16, units = (size_t)(K + UNIT - 1) / UNIT;
    switch (qt) {
    case QT_Q4_K: return tiles * units * Packed<QT_Q4_K>::CHUNK;
    case QT_Q5_K: return tiles * units * Packed<QT_Q5_K>::CHUNK;
    case QT_Q6_K: return tiles * units * Packed<QT_Q6_K>::CHUNK;
    case QT_Q8_0: return tiles * units * Packed<QT_Q8_0>::CHUNK;
    }
    return 0;
}

// gated > 0: pack a [gate; up] matrix of N = 2 gated rows into tiles of 8
// gate rows and their up rows (gated a multiple of 8).
hipError_t launch_pack(int qt, const void *W, void *P, int N, int K, hipStream_t st, int gated) {
    const dim3 grid((K + UNIT - 1) / UNIT, (N + 15) / 16);
    const uint8_t *w = (const uint8_t *)W;
    uint8_t *p = (uint8_t *)P;
    switch (qt) {
    case QT_Q4_K: pack_kernel<QT_Q4_K><<<grid, 64, 0, st>>>(w, N, K, p, gated); break;
    case QT_Q5_K: pack_kernel<QT_Q5_K><<<grid, 64, 0, st>>>(w, N, K, p, gated); break;
    case QT_Q6_K: pack_kernel<QT_Q6_K><<<grid, 64, 0, st>>>(w, N, K, p, gated); break;
    case QT_Q8_0: pack_kernel<QT_Q8_0><<<grid, 64, 0, st>>>(w, N, K, p, gated); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

static hipError_t gemm_in(int qt, const void *W, const float *X, const ActIn &in, float *Y, int M, int N, int K,
                          int flags, void *ws, hipStream_t st) {
    const int m0 = launch_m(M, flags);
    if (m0 != M) {
        hipError_t e = gemm_in(qt, W, X, in, Y, m0, N, K, flags | 1, ws, st);
        if (e != hipSuccess) return e;
        ActIn in2 = in;
        if (in2.add != nullptr) in2.add += (size_t)m0 * (X != nullptr ? K : in.ldx);
        if (in2.sum_out != nullptr) in2.sum_out += (size_t)m0 * in.ldx;
        const float *X2 = X != nullptr ? X + (size_t)m0 * in.ldx : nullptr;  // (absent: the slices are the input)
        return gemm_in(qt, W, X2, in2, Y + (size_t)m0 * N, M - m0, N, K, flags | 1, ws, st);
    }
    const GemmPlan p = plan_gemm(qt, M, N, K, flags);
    const int accum = (flags & 4) ? 1 : 0;
    const bool pk = (flags & 8) != 0;
    const uint8_t *w = (const uint8_t *)W;
    uint8_t *wsp = (uint8_t *)ws;
#define D(q) return pk ? dispatch_mt<q, true>(p, w, X, in, Y, M, N, K, accum, wsp, st) \
                       : dispatch_mt<q, false>(p, w, X, in, Y, M, N, K, accum, wsp, st)
    switch (qt) {
    case QT_Q4_K: D(QT_Q4_K);
    case QT_Q5_K: D(QT_Q5_K);
    case QT_Q6_K: D(QT_Q6_K);
    case QT_Q8_0: D(QT_Q8_0);
    }
#undef D
    return hipErrorInvalidValue;
}

hipError_t launch_gemm(int qt, const void *W, const float *X, float *Y, int M, int N, int K, int flags, void *ws,
                       hipStream_t st) {
    const ActIn in{ACT_PLAIN, K, nullptr, 0.f, false, nullptr, 0, 0, false};
    return gemm_in(qt, W, X, in, Y, M, N, K, flags, ws, st);
}

// A chained fp32-accurate call on packed weights (one token tile, M <= 8):
// input either from the input stage (in != nullptr: prepared into ws as
// usual) or a chained producer's operand (in == nullptr: ch.xop, rescaled in
// registers), the RMSNorm row scales then from the producer's tile
// sums of squares (ssq_in, n_ssq_in parts; null = none); epilogue ch.epi
// (EPI_STORE with flags bit 32 leaves K-slice partials in ws; other
// epilogues of a K-split plan sum the slices per tile themselves, with the
// per-tile counts kept zero between calls in ws). Returns
// hipErrorInvalidValue where the plan is not the one-tile streaming kernel.
hipError_t launch_gemm_chain(int qt, const void *W, const ActIn *in, const float *X, const Chain &chain,
                             const float *ssq_in, int n_ssq_in, float eps, float *Y, int M, int N, int K, int flags,
                             void *ws, hipStream_t st) {
    const bool defer = (flags & 32) != 0;
    const int f = (flags & ~48) | 1 | 8;  // fp32-accurate, packed
    const GemmPlan p = plan_gemm(qt, M, N, K, f);
    if (!p.stream || p.MT != 1 || !p.split) return hipErrorInvalidValue;
    if (chain.epi != EPI_STORE && defer) return hipErrorInvalidValue;
    if (chain.epi != EPI_STORE && ((N + 15) / 16 + p.G - 1) / p.G > CHAIN_MAX_TILES) return hipErrorInvalidValue;
    uint8_t *wsp = (uint8_t *)ws;
    float *part = (float *)(wsp + p.off_part);
    Chain ch = chain;  // (a K-split epilogue's partials and counts live in ws)
    ch.tile_part = (float2 *)part;
    ch.tile_cnt = (int *)(wsp + p.off_cnt);
    const uint8_t *w = (const uint8_t *)W;
    // (chained calls: the 8-wave plans, and Q6_K's 4 x 3-unit one)
    const bool q6_43 = qt == QT_Q6_K && p.NW == 4 && p.UPS == 3;
    if (p.NW != 8 && !q6_43) return hipErrorInvalidValue;
    // (instantiated up to the units per wave stream_ups_cap allows)
#define CV(q, u) if constexpr (u <= stream_ups_cap(q, true)) if (qt == q && p.UPS == u) \
    return launch_v<q, 8, u, true, true, 1>(w, X, ai, Y, M, N, K, p.S, p.G, 0, a, part, st, &ch)
#define XV(q, u) if constexpr (u <= stream_ups_cap(q, true)) if (qt == q && p.UPS == u) \
    return launch_vx<q, 8, u>(w, Y, M, N, K, p.S, p.G, defer, ssq_in, n_ssq_in, eps, part, ch, st)
    if (in != nullptr) {
        const ActWs a{wsp, nullptr, (float *)(wsp + p.off_inv), wsp + p.off_mfrag, (float *)(wsp + p.off_ssq)};
        ActIn ai = *in;
        ai.defer = defer;
        CV(QT_Q4_K, 1); CV(QT_Q4_K, 2); CV(QT_Q4_K, 4); CV(QT_Q5_K, 1); CV(QT_Q5_K, 2);
        if (q6_43) return launch_v<QT_Q6_K, 4, 3, true, true, 1>(w, X, ai, Y, M, N, K, p.S, p.G, 0, a, part, st, &ch);
        CV(QT_Q6_K, 1); CV(QT_Q6_K, 2); CV(QT_Q8_0, 1);
        return hipErrorInvalidValue;
    }
    XV(QT_Q4_K, 1); XV(QT_Q4_K, 2); XV(QT_Q4_K, 4); XV(QT_Q5_K, 1); XV(QT_Q5_K, 2);
    if (q6_43) return launch_vx<QT_Q6_K, 4, 3>(w, Y, M, N, K, p.S, p.G, defer, ssq_in, n_ssq_in, eps, part, ch, st);
    XV(QT_Q6_K, 1); XV(QT_Q6_K, 2); XV(QT_Q8_0, 1);
#undef XV
#undef CV
    return hipErrorInvalidValue;
}

hipError_t launch_gemm_chain_ex(int qt, const void *W, const float *X, int ldx, int op, const float *norm_w,
                                float eps_in, const float *add, int n_add, int64_t add_stride, const Chain &ch,
                                const float *ssq_in, int n_ssq_in, float eps, float *Y, int M, int N, int K,
                                int flags, void *ws, hipStream_t st) {
    if (X == nullptr)
        return launch_gemm_chain(qt, W, nullptr, nullptr, ch, ssq_in, n_ssq_in, eps, Y, M, N, K, flags, ws, st);
    const ActIn in{op, ldx, norm_w, eps_in, false, add, n_add, add_stride, false};
    return launch_gemm_chain(qt, W, &in, X, ch, nullptr, 0, 0.f, Y, M, N, K, flags, ws, st);
}

// flags bit 16: reuse prepared activations; bit 32: defer (partials stay in
// the workspace). Splitting M > 32 (fp32-accurate) into two launches keeps
// only the second half prepared and its partials, so reuse and defer need
// M <= 32 there (checked by the caller).
hipError_t launch_gemm_ex(int qt, const void *W, const float *X, int ldx, int op, const float *norm_w, float eps,
                          const float *add, int n_add, int64_t add_stride, float *Y, int M, int N, int K, int flags,
                          void *ws, hipStream_t st) {
    // (flags 64: the slices are the input and their sum goes to X)
    const bool sum_out = (flags & 64) != 0;
    ActIn in{op, ldx, norm_w, eps, (flags & 16) != 0, add, n_add, add_stride, (flags & 32) != 0};
    in.sum_out = sum_out ? const_cast<float *>(X) : nullptr;
    return gemm_in(qt, W, sum_out ? nullptr : X, in, Y, M, N, K, flags & ~112, ws, st);
}

bool gemm_reuse_ok(int M, int flags) { return launch_m(M, flags) == M; }

// Where a deferred call left its K-slice partials: slices [S][M][N] at ws +
// offset.
void gemm_partials(int qt, int M, int N, int K, int flags, size_t *offset, int *n_slices) {
    const GemmPlan p = plan_gemm(qt, M, N, K, flags & ~48);
    *offset = p.off_part;
    *n_slices = p.S;
}
