// Bit-exact block dequantization (the dequantize_*_block! formulas of the
// reference, src/QuantsCPU.jl:491-658; same maths in src/Dequant.jl). Each
// multiply and subtract rounds separately, as Julia evaluates them, so
// contraction into FMA is switched off for this file.
#pragma clang fp contract(off)
#include "common.h"

namespace {

// 6-bit scale and min of sub-block s (src/QuantsCPU.jl:501-513).
__device__ __forceinline__ void scale_min_k4(const uint8_t *sc12, int s, uint32_t &sc, uint32_t &m) {
    if (s < 4) {
        sc = sc12[s] & 63;
        m = sc12[s + 4] & 63;
    } else {
        sc = (sc12[s + 4] & 0x0f) | ((sc12[s - 4] >> 6) << 4);
        m = (sc12[s + 4] >> 4) | ((sc12[s] >> 6) << 4);
    }
}

// Thread t of a block handles sub-block t/4 and 8 consecutive elements;
// 32 threads per 256-element block, 4 per 32-element Q8_0 block.
template <int QT>
__global__ void dequant_kernel(const uint8_t *__restrict__ w, float *__restrict__ out, int64_t n_blocks) {
    constexpr int BB = QTraits<QT>::BB;
    constexpr int TPB = QTraits<QT>::QK / 8;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t b = gid / TPB;
    if (b >= n_blocks) return;
    const int t = (int)(gid % TPB);
    const uint8_t *blk = w + b * BB;
    float *o = out + b * QTraits<QT>::QK;
    float v[8];
    int base;
    if constexpr (QT == QT_Q4_K || QT == QT_Q5_K) {
        const float d = f16_bits_to_f32(ld_u16(blk)), dmin = f16_bits_to_f32(ld_u16(blk + 2));
        const int s = t / 4;              // sub-block 0..7 (32 elements each)
        const int j = s / 2, hi = s & 1;  // pair j, high nibble for odd s
        const int l0 = (t % 4) * 8;       // element offset inside the sub-block
        uint32_t sc, m;
        scale_min_k4(blk + 4, s, sc, m);
        const float d1 = d * (float)sc, m1 = dmin * (float)m;
        const uint8_t *qs = blk + (QT == QT_Q4_K ? 16 : 48) + 32 * j;
        for (int e = 0; e < 8; e++) {
            const int l = l0 + e;
            const uint32_t q = hi ? (qs[l] >> 4) : (qs[l] & 0x0f);
            float qv = (float)q;
            if constexpr (QT == QT_Q5_K) {
                const uint32_t bit = (blk[16 + l] >> (2 * j + hi)) & 1;
                qv = qv + (bit ? 16.0f : 0.0f);
            }
            v[e] = d1 * qv - m1;
        }
        base = 64 * j + 32 * hi + l0;
    } else if constexpr (QT == QT_Q6_K) {
        const float d = f16_bits_to_f32(ld_u16(blk + 208));
        const int8_t *sc = (const int8_t *)(blk + 192);
        // element index e0 = 8t; half n, quarter qq, position l in 0..31
        const int e0 = 8 * t;
        const int n = e0 / 128, qq = (e0 % 128) / 32, l0 = e0 % 32;
        const uint8_t *ql = blk + 64 * n, *qh = blk + 128 + 32 * n;
        for (int e = 0; e < 8; e++) {
            const int l = l0 + e;
            const uint32_t h = qh[l];
            int q;
            switch (qq) {
            case 0: q = (int)((ql[l] & 0x0f) | ((h & 3) << 4)) - 32; break;
            case 1: q = (int)((ql[l + 32] & 0x0f) | (((h >> 2) & 3) << 4)) - 32; break;
            case 2: q = (int)((ql[l] >> 4) | (((h >> 4) & 3) << 4)) - 32; break;
            default: q = (int)((ql[l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32; break;
            }
            const float s = (float)sc[8 * n + 2 * qq + l / 16];
            v[e] = d * s * (float)q;
        }
        base = e0;
    } else {  // Q8_0
        const float d = f16_bits_to_f32(ld_u16(blk));
        for (int e = 0; e < 8; e++) v[e] = d * (float)(int8_t)blk[2 + 8 * t + e];
        base = 8 * t;
    }
    float4 *dst = (float4 *)(o + base);
    dst[0] = make_float4(v[0], v[1], v[2], v[3]);
    dst[1] = make_float4(v[4], v[5], v[6], v[7]);
}

}  // namespace

hipError_t launch_dequant(int qt, const void *w, float *out, int64_t n_blocks, hipStream_t st) {
    const int tpb = qt_block_elems(qt) / 8;
    const int64_t threads = n_blocks * tpb;
    const int bs = 256;
    const unsigned grid = (unsigned)((threads + bs - 1) / bs);
    if (grid == 0) return hipSuccess;
    const uint8_t *wp = (const uint8_t *)w;
    switch (qt) {
    case QT_Q4_K: dequant_kernel<QT_Q4_K><<<grid, bs, 0, st>>>(wp, out, n_blocks); break;
    case QT_Q5_K: dequant_kernel<QT_Q5_K><<<grid, bs, 0, st>>>(wp, out, n_blocks); break;
    case QT_Q6_K: dequant_kernel<QT_Q6_K><<<grid, bs, 0, st>>>(wp, out, n_blocks); break;
    case QT_Q8_0: dequant_kernel<QT_Q8_0><<<grid, bs, 0, st>>>(wp, out, n_blocks); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
