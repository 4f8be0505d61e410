// RMSNorm and the seeded synthetic-input generators.
#include "common.h"

namespace {

// One workgroup per row: out = x * (1 / sqrt(mean(x^2) + eps)) * w
// (src/ModelCPU.jl:110-122).
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                      float *__restrict__ out, int n, float eps) {
    __shared__ float sh[4];
    const float *xr = x + (size_t)blockIdx.x * n;
    float *orow = out + (size_t)blockIdx.x * n;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += 256) ss = __builtin_fmaf(xr[i], xr[i], ss);
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = (sh[0] + sh[1]) + (sh[2] + sh[3]);
    const float scale = 1.0f / sqrtf(tot / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += 256) orow[i] = xr[i] * scale * (w ? w[i] : 1.0f);
}

// ---- splitmix64 counter stream: word i = mix64(stream + (i + 1) * G) ----
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t word(uint64_t stream, uint64_t i) {
    return mix64(stream + (i + 1) * 0x9E3779B97F4A7C15ull);
}

// fp16(lo + u * span), u = top 24 bits / 2^24, multiply and add each rounded
// to fp32 (no contraction), then round-to-nearest-even to fp16.
__device__ __forceinline__ uint32_t fp16_field(uint64_t w, float lo, float span) {
    const float u = (float)(uint32_t)(w >> 40) * (1.0f / 16777216.0f);
    const float v = __fadd_rn(lo, __fmul_rn(u, span));
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v);
}

__device__ __forceinline__ void put_u16(uint8_t *p, uint32_t v) {
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
}
__device__ __forceinline__ void put_words(uint8_t *p, const uint64_t *w, int n) {
    for (int i = 0; i < n; i++)
        for (int b = 0; b < 8; b++) p[8 * i + b] = (uint8_t)(w[i] >> (8 * b));
}

// One thread per block; block b uses words [32b, 32b + 32) of the stream.
template <int QT>
__global__ void synth_kernel(uint64_t stream, int64_t first, int64_t nblk, uint8_t *__restrict__ out,
                             float lo_a, float span_a, float lo_b, float span_b) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk) return;
    const uint64_t b = (uint64_t)(first + i);
    uint64_t w[32];
    for (int j = 0; j < 28; j++) w[j] = word(stream, b * 32 + j);
    uint8_t *o = out + i * QTraits<QT>::BB;
    if constexpr (QT == QT_Q4_K || QT == QT_Q5_K) {
        put_u16(o, fp16_field(w[0], lo_a, span_a));
        put_u16(o + 2, fp16_field(w[1], lo_a, span_a));
        uint32_t sc[8], m[8];
        for (int j = 0; j < 8; j++) {
            sc[j] = (uint32_t)(w[2] >> (6 * j)) & 63;
            m[j] = (uint32_t)(w[3] >> (6 * j)) & 63;
        }
        for (int j = 0; j < 4; j++) {  // exact inverse of the 6-bit unpack
            o[4 + j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
            o[8 + j] = (uint8_t)(m[j] | ((m[j + 4] >> 4) << 6));
            o[12 + j] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
        }
        if constexpr (QT == QT_Q4_K) {
            put_words(o + 16, w + 4, 16);
        } else {
            put_words(o + 16, w + 20, 4);
            put_words(o + 48, w + 4, 16);
        }
    } else if constexpr (QT == QT_Q6_K) {
        put_words(o, w + 4, 16);
        put_words(o + 128, w + 20, 8);
        for (int j = 0; j < 16; j++) {
            const int v = (int)((w[2 + j / 8] >> (6 * (j % 8))) & 63) - 32;
            o[192 + j] = (uint8_t)(int8_t)v;
        }
        put_u16(o + 208, fp16_field(w[0], lo_a, span_a));
    } else {
        put_u16(o, fp16_field(w[0], lo_a, span_a));
        for (int j = 0; j < 32; j++) {
            const uint64_t piece = (w[1 + j / 4] >> (16 * (j % 4))) & 0xFFFF;
            const int q = (int)((piece * 255) >> 16) - 127;
            o[2 + j] = (uint8_t)(int8_t)q;
        }
    }
    (void)lo_b;
    (void)span_b;
}

__global__ void gaussian_kernel(uint64_t stream, int64_t n, float scale, const float *__restrict__ add,
                                float *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t a = word(stream, 2 * (uint64_t)i), b = word(stream, 2 * (uint64_t)i + 1);
    const double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);
    const double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
    const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
    out[i] = (float)z * scale + (add ? add[i] : 0.f);
}

// out[m, i] = silu(gu[m, i]) * gu[m, F + i] for rows of [gate | up]
// (mlp_forward, src/ModelCPU.jl:447-473); silu(g) = g / (1 + exp(-g)).
__global__ void silu_mul_kernel(const float *__restrict__ gu, int M, int F, float *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)M * F) return;
    const int64_t m = i / F, c = i % F;
    const float g = gu[m * 2 * F + c], u = gu[m * 2 * F + F + c];
    out[i] = g / (1.0f + expf(-g)) * u;
}

// y[i] += x[i] (residual add of the decoder layer, src/ModelCPU.jl:870-891)
__global__ void add_kernel(float *__restrict__ y, const float *__restrict__ x, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] += x[i];
}

// Read-bandwidth probe: every thread XORs the 16-byte words it streams (grid
// stride, four loads in flight) and each workgroup stores its XOR in its own
// word of out, so no load can be dropped, only one word per workgroup is
// written and no atomic serializes the tail.
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4 *__restrict__ src, int64_t n16,
                                                          uint32_t *__restrict__ out) {
    __shared__ uint32_t sh[4];
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    // (non-temporal loads, as the matmuls read their weights: the default
    // policy streams 10-15 % slower on this part; eight in flight per
    // thread)
    typedef unsigned int u4v __attribute__((ext_vector_type(4)));
    const u4v *s4 = (const u4v *)src;
    for (; i + 7 * stride < n16; i += 8 * stride) {
        u4v v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = __builtin_nontemporal_load(s4 + i + u * stride);
#pragma unroll
        for (int u = 0; u < 8; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += stride) {
        const uint4 a = src[i];
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    for (int o = 32; o > 0; o >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = sh[0] ^ sh[1] ^ sh[2] ^ sh[3];
}

}  // namespace

hipError_t launch_stream_read(const void *src, int64_t bytes, uint32_t *out, hipStream_t st) {
    const int64_t n16 = bytes / 16;
    if (n16 <= 0) return hipSuccess;
    // 8 workgroups of 256 threads per CU on 256 CUs (one output word each),
    // fewer for small buffers
    const int64_t want = (n16 + 1023) / 1024;
    const unsigned grid = (unsigned)(want < 2048 ? (want < 1 ? 1 : want) : 2048);
    stream_read_kernel<<<grid, 256, 0, st>>>((const uint4 *)src, n16, out);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const float *gu, int M, int F, float *out, hipStream_t st) {
    const int64_t n = (int64_t)M * F;
    if (n <= 0) return hipSuccess;
    silu_mul_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(gu, M, F, out);
    return hipGetLastError();
}

hipError_t launch_add(float *y, const float *x, int64_t n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    add_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(y, x, n);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const float *x, const float *w, float *out, int rows, int n, float eps, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    rmsnorm_kernel<<<rows, 256, 0, st>>>(x, w, out, n, eps);
    return hipGetLastError();
}

hipError_t launch_synth(int qt, uint64_t stream, int64_t first, int64_t nblk, void *out, hipStream_t st) {
    if (nblk <= 0) return hipSuccess;
    const unsigned grid = (unsigned)((nblk + 127) / 128);
    uint8_t *o = (uint8_t *)out;
    // field ranges: Q4_K/Q5_K d, dmin ~ U(0.001, 0.05); Q6_K, Q8_0 d ~ U(0.001, 0.02)
    const float lo = (float)0.001;
    const float span_k = (float)(0.05 - 0.001), span_s = (float)(0.02 - 0.001);
    switch (qt) {
    case QT_Q4_K: synth_kernel<QT_Q4_K><<<grid, 128, 0, st>>>(stream, first, nblk, o, lo, span_k, 0, 0); break;
    case QT_Q5_K: synth_kernel<QT_Q5_K><<<grid, 128, 0, st>>>(stream, first, nblk, o, lo, span_k, 0, 0); break;
    case QT_Q6_K: synth_kernel<QT_Q6_K><<<grid, 128, 0, st>>>(stream, first, nblk, o, lo, span_s, 0, 0); break;
    case QT_Q8_0: synth_kernel<QT_Q8_0><<<grid, 128, 0, st>>>(stream, first, nblk, o, lo, span_s, 0, 0); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gaussian(uint64_t stream, int64_t n, float scale, const float *add, float *out, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    gaussian_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(stream, n, scale, add, out);
    return hipGetLastError();
}
