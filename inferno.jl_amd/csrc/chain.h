// Argument block of a chained fp32-accurate matmul (gemm.hip, capi.cpp):
// where the producer's epilogue leaves its output, the next matmul's operand
// and per-tile statistics, and where the consumer finds them. Field meanings
// are given with ihip_chain_in / ihip_chain_out in include/inferno_hip.h.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

enum { EPI_STORE = 0, EPI_STATS = 1, EPI_RESID = 2, EPI_GATE = 3 };

// Bytes of a chained operand for K inputs: per 256-element unit the split
// fp16 limbs in the one-tile input stage's layout (8192 bytes reserved; M
// tokens use entries of 4 lane groups x 2M slots), then per unit one
// exponent byte per lane entry (lane group G, slot s at (2M G + s) 16).
constexpr int CHAIN_UNIT_LIMBS = 8192;
constexpr int CHAIN_UNIT_EXPS = 1024;
inline int64_t chain_operand_bytes(int K) { return (int64_t)((K + 255) / 256) * (CHAIN_UNIT_LIMBS + CHAIN_UNIT_EXPS); }

struct Chain {
    // consumer side (operand from a chained producer)
    const uint8_t *xop;    // limbs [units][8192], then exponents [units][1024]
    const float *xsum;     // producer tile sums [token][xsum_stride] (min terms)
    int xsum_stride;
    int x_tiles_per_unit;  // 16 (16-row tiles) or 32 (8 gated channels per tile)
    // producer side (epilogue)
    int epi;
    int ldy;
    const float *yw;       // next RMSNorm weight, or null
    int op_lk;             // operand layout of the consumer: 0 Q4_K/Q5_K, 1 Q6_K, 2 Q8_0
    uint8_t *yop;          // the consumer's operand (chain_operand_bytes(width)), or null
    int y_units;           // units of the consumer's K (exponents follow the limbs)
    float *ysum;           // tile sums [token][ysum_stride], or null
    int ysum_stride;
    float *yssq;           // [tile][8], or null
    int stat_rows;         // statistics over rows < stat_rows (EPI_STATS)
    // a K-split producer's epilogue: per 16-row tile, the slices' partial
    // tiles ([tile][slice][64 lanes] float2) and the count of slices done
    // (0 between calls: the last slice to arrive resets it)
    float2 *tile_part;
    int *tile_cnt;
};
