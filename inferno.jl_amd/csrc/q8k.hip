// The rest of QuantizedKernels' exports on gfx950: Q8_K activation
// quantization (quantize_row_q8_K) and the single-row K-quant x Q8_K dot
// products (vec_dot_q{4,5,6}_K_q8_K), src/kernels/quant_kernels.c:166-521,
// bound by src/QuantizedKernels.jl:149-175. The matmul path never uses them
// (it multiplies fp32 activations directly); they exist so that this library
// can stand in for libquant_kernels.so symbol for symbol.
//
// Results equal the reference's bit for bit: integer products and sums are
// exact in any order, and the float steps follow the reference's AVX2 lane
// structure. The 8-lane int32 accumulator lane t covers bytes 4t..4t+3 of
// every 32-byte slice and is folded into its own float lane with one fma per
// block; the lanes are summed as hsum_float_8 does, ((a0+a4)+(a2+a6)) +
// ((a1+a5)+(a3+a7)). Q4_K's mins use 4 float lanes (fma per block, summed
// (m0+m2)+(m1+m3)); Q5_K's one scalar (fma per block, as the reference's
// `summs += dmin * hsum` compiles with contraction).
#include "common.h"

namespace {

struct Q8K {  // block_q8_K (quant_kernels.c:52-56): 292 bytes, no padding
    float d;
    int8_t qs[256];
    int16_t bsums[16];
};
static_assert(sizeof(Q8K) == 292, "block_q8_K layout");

// One workgroup per 256-value block: amax, d = amax / 127, id = 1 / d
// (0 when d = 0), q = (int8) round-half-away(x * id), bsums of 16.
__global__ __launch_bounds__(256) void quantize_q8k_kernel(const float *__restrict__ x, uint8_t *__restrict__ y) {
    __shared__ float smax[4];
    const int b = blockIdx.x, j = threadIdx.x;
    const float v = x[(size_t)b * 256 + j];
    float m = wave_max(fabsf(v));
    if ((j & 63) == 0) smax[j >> 6] = m;
    __syncthreads();
    const float amax = fmaxf(fmaxf(smax[0], smax[1]), fmaxf(smax[2], smax[3]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const int q = (int)(int8_t)roundf(v * id);
    int s = q;  // sum over the 16 lanes of this value's group (an integer: exact in any order)
    for (int o = 8; o > 0; o >>= 1) s += __shfl_xor(s, o);
    Q8K *blk = (Q8K *)(y + (size_t)b * sizeof(Q8K));
    blk->qs[j] = (int8_t)q;
    if ((j & 15) == 0) blk->bsums[j >> 4] = (int16_t)s;
    if (j == 0) blk->d = d;
}

__device__ __forceinline__ float f16at(const uint8_t *p) { return f16_bits_to_f32(ld_u16(p)); }

__device__ __forceinline__ void sc_min(const uint8_t *s12, int s, int &sc, int &m) {
    if (s < 4) {
        sc = s12[s] & 63;
        m = s12[s + 4] & 63;
    } else {
        sc = (s12[s + 4] & 0x0f) | ((s12[s - 4] >> 6) << 4);
        m = (s12[s + 4] >> 4) | ((s12[s] >> 6) << 4);
    }
}

// Lane t of the int32 accumulator for one block (QT's bytes at x, Q8_K y).
template <int QT>
__device__ int lane_sum(const uint8_t *x, const Q8K &y, int t) {
    int sumi = 0;
    if constexpr (QT == QT_Q4_K || QT == QT_Q5_K) {
        const uint8_t *qh = x + 16, *q4 = x + (QT == QT_Q5_K ? 48 : 16);
        for (int j = 0; j < 4; j++) {
            int sc0, m0, sc1, m1;
            sc_min(x + 4, 2 * j, sc0, m0);
            sc_min(x + 4, 2 * j + 1, sc1, m1);
            int pl = 0, ph = 0;
            for (int b = 4 * t; b < 4 * t + 4; b++) {
                int lo = q4[32 * j + b] & 0xf, hi = q4[32 * j + b] >> 4;
                if constexpr (QT == QT_Q5_K) {
                    lo += ((qh[b] >> (2 * j)) & 1) << 4;
                    hi += ((qh[b] >> (2 * j + 1)) & 1) << 4;
                }
                pl += lo * y.qs[64 * j + b];
                ph += hi * y.qs[64 * j + 32 + b];
            }
            sumi += sc0 * pl + sc1 * ph;
        }
    } else {  // Q6_K: per 128-value half h and quarter i, lanes t < 4 use scale 8h + 2i, t >= 4 scale 8h + 2i + 1
        const int8_t *sc = (const int8_t *)(x + 192);
        for (int h = 0; h < 2; h++) {
            const uint8_t *ql = x + 64 * h, *qh = x + 128 + 32 * h;
            for (int i = 0; i < 4; i++) {
                int p = 0;
                for (int b = 4 * t; b < 4 * t + 4; b++) {
                    const int lo = (i & 1) ? ql[32 + b] : ql[b];
                    const int q = ((i >> 1) ? (lo >> 4) : (lo & 0xf)) | (((qh[b] >> (2 * i)) & 3) << 4);
                    p += (q - 32) * y.qs[128 * h + 32 * i + b];
                }
                sumi += sc[8 * h + 2 * i + (t >= 4 ? 1 : 0)] * p;
            }
        }
    }
    return sumi;
}

// One wave: lanes 0..7 are the float accumulator lanes; lane 0 folds them.
template <int QT>
__global__ __launch_bounds__(64) void vec_dot_kernel(const uint8_t *__restrict__ xw, const uint8_t *__restrict__ yq,
                                                     int nb, float *__restrict__ out) {
    constexpr int BB = QTraits<QT>::BB;
    __shared__ float lanes[8], mins[4];
    const int t = threadIdx.x;
    float acc = 0.f, accm = 0.f;
    for (int i = 0; i < nb; i++) {
        const uint8_t *x = xw + (size_t)i * BB;
        const Q8K &y = *(const Q8K *)(yq + (size_t)i * sizeof(Q8K));
        const float d = y.d * f16at(x + (QT == QT_Q6_K ? 208 : 0));
        if (t < 8) acc = __builtin_fmaf(d, (float)lane_sum<QT>(x, y, t), acc);
        if constexpr (QT == QT_Q4_K) {
            if (t < 4) {  // mins: lane t holds m_2t bsum-pairs + m_2t+1 ...
                const float dmin = -y.d * f16at(x + 2);
                int s0, m0, s1, m1;
                sc_min(x + 4, 2 * t, s0, m0);
                sc_min(x + 4, 2 * t + 1, s1, m1);
                const int prod = m0 * (y.bsums[4 * t] + y.bsums[4 * t + 1]) + m1 * (y.bsums[4 * t + 2] + y.bsums[4 * t + 3]);
                accm = __builtin_fmaf(dmin, (float)prod, accm);
            }
        } else if constexpr (QT == QT_Q5_K) {
            if (t == 0) {
                const float dmin = -y.d * f16at(x + 2);
                int hs = 0;
                for (int u = 0; u < 8; u++) {
                    int s, m;
                    sc_min(x + 4, u, s, m);
                    hs += m * (y.bsums[2 * u] + y.bsums[2 * u + 1]);
                }
                accm = __builtin_fmaf(dmin, (float)hs, accm);
            }
        }
    }
    if (t < 8) lanes[t] = acc;
    if (t < 4) mins[t] = accm;
    __syncthreads();
    if (t == 0) {
        const float h = ((lanes[0] + lanes[4]) + (lanes[2] + lanes[6])) + ((lanes[1] + lanes[5]) + (lanes[3] + lanes[7]));
        float r = h;
        if constexpr (QT == QT_Q4_K) r = h + ((mins[0] + mins[2]) + (mins[1] + mins[3]));
        if constexpr (QT == QT_Q5_K) r = h + mins[0];
        *out = r;
    }
}

}  // namespace

size_t q8k_block_bytes() { return sizeof(Q8K); }

hipError_t launch_quantize_q8k(const float *x, void *y, int64_t k, hipStream_t st) {
    if (k <= 0) return hipSuccess;
    quantize_q8k_kernel<<<(unsigned)(k / 256), 256, 0, st>>>(x, (uint8_t *)y);
    return hipGetLastError();
}

hipError_t launch_vec_dot_q8k(int qt, const void *x, const void *y, int nb, float *out, hipStream_t st) {
    const uint8_t *xw = (const uint8_t *)x, *yq = (const uint8_t *)y;
    switch (qt) {
    case QT_Q4_K: vec_dot_kernel<QT_Q4_K><<<1, 64, 0, st>>>(xw, yq, nb, out); break;
    case QT_Q5_K: vec_dot_kernel<QT_Q5_K><<<1, 64, 0, st>>>(xw, yq, nb, out); break;
    case QT_Q6_K: vec_dot_kernel<QT_Q6_K><<<1, 64, 0, st>>>(xw, yq, nb, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
