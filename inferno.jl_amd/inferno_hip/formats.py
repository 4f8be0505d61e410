"""GGUF block formats on the hot path.

Type ids are GGML's (src/GGUF.jl:25-60); sizes follow the block structs of
src/kernels/quant_kernels.c:24-62 and src/QuantsCPU.jl:22-25.
"""
Q8_0 = 8
Q4_K = 12
Q5_K = 13
Q6_K = 14

QTYPES = (Q4_K, Q5_K, Q6_K, Q8_0)
NAMES = {Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", Q8_0: "Q8_0"}
BY_NAME = {v: k for k, v in NAMES.items()}

BLOCK_BYTES = {Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_0: 34}
BLOCK_ELEMS = {Q4_K: 256, Q5_K: 256, Q6_K: 256, Q8_0: 32}

# Q8_K activation block of the reference CPU path (quant_kernels.c:52-56):
# float d + int8 qs[256] + int16 bsums[16].
Q8_K_BLOCK_BYTES = 292


def row_bytes(qtype: int, k: int) -> int:
    be = BLOCK_ELEMS[qtype]
    if k % be:
        raise ValueError(f"inner_dim {k} is not a multiple of {be} for {NAMES[qtype]}")
    return (k // be) * BLOCK_BYTES[qtype]


def matrix_bytes(qtype: int, n: int, k: int) -> int:
    return n * row_bytes(qtype, k)
