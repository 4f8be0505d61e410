"""Seeded synthetic GGUF blocks and activations.

A counter-based splitmix64 stream: word i of stream s is mix64(s + (i+1)*G).
Every block b of a tensor uses words [32*b, 32*b + 32) of its stream, so any
block can be generated independently (the device generator in
csrc/synth.hip produces the same bytes; a GPU test checks that).

Block fields follow the GGUF layouts of the reference
(src/kernels/quant_kernels.c:24-62, src/QuantsCPU.jl:491-658):

* Q4_K: d, dmin ~ U(0.001, 0.05) as fp16; 8 scales and 8 mins ~ U{0..63}
  packed by the exact inverse of the 6-bit unpack (src/QuantsCPU.jl:501-513);
  128 bytes of nibbles ~ uniform.
* Q5_K: as Q4_K plus 32 bytes of high bits.
* Q6_K: 128 B low nibbles, 64 B high 2-bit pairs ~ uniform; 16 int8 scales
  ~ U{-32..31}; d ~ U(0.001, 0.02).
* Q8_0: 32 int8 ~ U{-127..127}; d ~ U(0.001, 0.02).

The fp16 fields are computed as fp16(lo + u*(hi-lo)) with u = top 24 bits /
2^24, the multiply and add each rounded to fp32, then round-to-nearest-even
to fp16 (numpy's float32 -> float16 cast).
"""
from __future__ import annotations

import numpy as np

from .formats import Q4_K, Q5_K, Q6_K, Q8_0, BLOCK_BYTES, BLOCK_ELEMS

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
WORDS_PER_BLOCK = 32


def _mix64(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def words(stream: int, start: int, count: int) -> np.ndarray:
    """Words [start, start+count) of a stream as uint64."""
    idx = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix64(np.uint64(stream & 0xFFFFFFFFFFFFFFFF) + idx * GOLDEN)


def stream_for(seed: int, name: str) -> int:
    """Substream id: seed xor an FNV-1a hash of the tensor name."""
    h = 0xCBF29CE484222325
    for ch in name.encode():
        h ^= ch
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return (seed ^ h) & 0xFFFFFFFFFFFFFFFF


def _u24(w: np.ndarray) -> np.ndarray:
    return ((w >> np.uint64(40)).astype(np.float32)) * np.float32(1.0 / 16777216.0)


def _fp16_field(w: np.ndarray, lo: float, hi: float) -> np.ndarray:
    u = _u24(w)
    v = np.float32(lo) + u * np.float32(hi - lo)   # two fp32 roundings, no fma
    return v.astype(np.float16).view(np.uint16)


def _bytes(ws: np.ndarray) -> np.ndarray:
    """[nb, n] uint64 words -> [nb, 8n] little-endian bytes."""
    return np.ascontiguousarray(ws.astype("<u8")).view(np.uint8).reshape(ws.shape[0], -1)


def pack_scales_k4(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Inverse of the Q4_K/Q5_K 6-bit unpack: [nb, 8] sc/m -> [nb, 12] bytes."""
    sc = sc.astype(np.uint8)
    m = m.astype(np.uint8)
    out = np.zeros((sc.shape[0], 12), dtype=np.uint8)
    for i in range(4):
        out[:, i] = sc[:, i] | ((sc[:, i + 4] >> 4) << 6)
        out[:, i + 4] = m[:, i] | ((m[:, i + 4] >> 4) << 6)
        out[:, i + 8] = (sc[:, i + 4] & 0xF) | ((m[:, i + 4] & 0xF) << 4)
    return out


def unpack_scales_k4(scales: np.ndarray):
    """6-bit unpack (src/QuantsCPU.jl:501-513): [nb, 12] -> sc, m [nb, 8]."""
    s = scales.astype(np.uint8)
    sc = np.zeros((s.shape[0], 8), dtype=np.uint8)
    m = np.zeros_like(sc)
    for j in range(8):
        if j < 4:
            sc[:, j] = s[:, j] & 63
            m[:, j] = s[:, j + 4] & 63
        else:
            sc[:, j] = (s[:, j + 4] & 0xF) | ((s[:, j - 4] >> 6) << 4)
            m[:, j] = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    return sc, m


def blocks(qtype: int, n_blocks: int, stream: int, first_block: int = 0) -> np.ndarray:
    """n_blocks synthetic blocks of qtype -> uint8 [n_blocks * block_bytes]."""
    bb = BLOCK_BYTES[qtype]
    if n_blocks == 0:
        return np.zeros(0, dtype=np.uint8)
    w = words(stream, first_block * WORDS_PER_BLOCK, n_blocks * WORDS_PER_BLOCK)
    w = w.reshape(n_blocks, WORDS_PER_BLOCK)
    out = np.zeros((n_blocks, bb), dtype=np.uint8)
    six = np.uint64(63)
    if qtype in (Q4_K, Q5_K):
        d = _fp16_field(w[:, 0], 0.001, 0.05)
        dmin = _fp16_field(w[:, 1], 0.001, 0.05)
        sc = np.stack([(w[:, 2] >> np.uint64(6 * i)) & six for i in range(8)], 1)
        m = np.stack([(w[:, 3] >> np.uint64(6 * i)) & six for i in range(8)], 1)
        out[:, 0:2] = d.reshape(-1, 1).view(np.uint8).reshape(-1, 2)
        out[:, 2:4] = dmin.reshape(-1, 1).view(np.uint8).reshape(-1, 2)
        out[:, 4:16] = pack_scales_k4(sc, m)
        if qtype == Q4_K:
            out[:, 16:144] = _bytes(w[:, 4:20])
        else:
            out[:, 16:48] = _bytes(w[:, 20:24])
            out[:, 48:176] = _bytes(w[:, 4:20])
    elif qtype == Q6_K:
        out[:, 0:128] = _bytes(w[:, 4:20])
        out[:, 128:192] = _bytes(w[:, 20:28])
        sc = np.stack([((w[:, 2 + i // 8] >> np.uint64(6 * (i % 8))) & six).astype(np.int16) - 32
                       for i in range(16)], 1)
        out[:, 192:208] = sc.astype(np.int8).view(np.uint8)
        d = _fp16_field(w[:, 0], 0.001, 0.02)
        out[:, 208:210] = d.reshape(-1, 1).view(np.uint8).reshape(-1, 2)
    elif qtype == Q8_0:
        d = _fp16_field(w[:, 0], 0.001, 0.02)
        out[:, 0:2] = d.reshape(-1, 1).view(np.uint8).reshape(-1, 2)
        pieces = np.stack([(w[:, 1 + i // 4] >> np.uint64(16 * (i % 4))) & np.uint64(0xFFFF)
                           for i in range(32)], 1)
        q = ((pieces * np.uint64(255)) >> np.uint64(16)).astype(np.int16) - 127
        out[:, 2:34] = q.astype(np.int8).view(np.uint8)
    else:
        raise ValueError(f"unsupported qtype {qtype}")
    return out.reshape(-1)


def matrix(qtype: int, n_rows: int, k: int, stream: int) -> np.ndarray:
    """A [n_rows x k] weight in GGUF row-major block layout (bytes)."""
    be = BLOCK_ELEMS[qtype]
    if k % be:
        raise ValueError(f"K={k} is not a multiple of {be}")
    return blocks(qtype, n_rows * (k // be), stream)


def gaussian(stream: int, n: int, first: int = 0) -> np.ndarray:
    """n fp32 samples of N(0,1): Box-Muller in fp64 from words 2i, 2i+1."""
    w = words(stream, 2 * first, 2 * n).reshape(n, 2)
    u1 = ((w[:, 0] >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
    u2 = (w[:, 1] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return z.astype(np.float32)


def uniform(stream: int, n: int, first: int = 0) -> np.ndarray:
    """n fp32 uniforms in [0, 1) with 24-bit resolution."""
    return _u24(words(stream, first, n))
