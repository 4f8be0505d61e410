// Device helpers shared by the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define QT_Q8_0 8
#define QT_Q4_K 12
#define QT_Q5_K 13
#define QT_Q6_K 14

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

template <int QT> struct QTraits;
template <> struct QTraits<QT_Q4_K> { static constexpr int BB = 144, QK = 256; };
template <> struct QTraits<QT_Q5_K> { static constexpr int BB = 176, QK = 256; };
template <> struct QTraits<QT_Q6_K> { static constexpr int BB = 210, QK = 256; };
template <> struct QTraits<QT_Q8_0> { static constexpr int BB = 34, QK = 32; };

__host__ __device__ inline int qt_block_bytes(int qt) {
    return qt == QT_Q4_K ? 144 : qt == QT_Q5_K ? 176 : qt == QT_Q6_K ? 210 : qt == QT_Q8_0 ? 34 : -1;
}
__host__ __device__ inline int qt_block_elems(int qt) {
    return (qt == QT_Q4_K || qt == QT_Q5_K || qt == QT_Q6_K) ? 256 : qt == QT_Q8_0 ? 32 : -1;
}

// IEEE binary16 bits -> binary32, exact for every input including NaN
// payloads (integer-only, independent of the FP16 denorm mode).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
    uint32_t f;
    if (e == 0) {
        if (m == 0) {
            f = sign;
        } else {
            // subnormal m * 2^-24: shift the leading one up to bit 10
            const int sh = __clz(m) - 21;
            f = sign | ((uint32_t)(113 - sh) << 23) | (((m << sh) & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        f = sign | 0x7f800000u | (m << 13);
    } else {
        f = sign | ((e + 112) << 23) | (m << 13);
    }
    return __uint_as_float(f);
}

// Unaligned little-endian loads from global memory. gfx950 global loads
// accept any byte alignment (unaligned access mode), so these compile to
// plain dword / ushort loads.
__device__ __forceinline__ uint32_t ld_u32(const uint8_t *p) {
    uint32_t v;
    __builtin_memcpy(&v, p, 4);
    return v;
}
__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p) {
    uint16_t v;
    __builtin_memcpy(&v, p, 2);
    return v;
}

// Two bytes b0 (selector 4/6) and b1 (5/7) of x, each placed under the fp16
// exponent 0x64: returns the fp16 pair (1024 + b0, 1024 + b1) as bits.
// v_perm_b32: selector bytes 0-3 pick src1 bytes, 4-7 pick src0 bytes.
__device__ __forceinline__ uint32_t pair_lo(uint32_t x) {
    return __builtin_amdgcn_perm(x, 0x64646464u, 0x00050004u);
}
__device__ __forceinline__ uint32_t pair_hi(uint32_t x) {
    return __builtin_amdgcn_perm(x, 0x64646464u, 0x00070006u);
}

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }

// Exact fp16 pair of a small non-negative integer v (< 1024): (v, v).
__device__ __forceinline__ h2 h2_of_small(uint32_t v) {
    const uint32_t b = 0x6400u | v;
    return as_h2(b | (b << 16)) - as_h2(0x64006400u);
}

__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Wait until this wave's vector memory operations have completed (gfx9
// s_waitcnt encoding: vmcnt 0, expcnt and lgkmcnt left at their maxima, i.e.
// not waited for). A device-scope (agent) atomic store has completed when it
// has reached the device's coherence point, so a count published after this
// wait cannot be seen before the data it counts. A workgroup-scope fence
// emits no such wait on gfx950, and an agent-scope fence would also write
// back the whole L2.
__device__ __forceinline__ void wait_stores_done() { __builtin_amdgcn_s_waitcnt(0x0F70); }
