"""CPU checks of the packed layout's numpy statement: with no padding it is a
bit permutation of the GGUF matrix in which every quant, scale and d bit
appears exactly once (the formats other than Q6_K move whole bytes), and each
16-row tile of each 256-element unit stays in its own chunk."""
import numpy as np
import pytest

from _packref import pack_ref, unit_bytes
from inferno_hip import formats as F
from inferno_hip import synth


def _source_bits(qt, N, K):
    """For each bit of the packed matrix, the index of the GGUF bit it holds
    (bits little-endian within bytes): packing label j sets input bit b when
    bit j of b is set, so output bit o reads bit j of its source's index."""
    nbytes = N * K // F.BLOCK_ELEMS[qt] * F.BLOCK_BYTES[qt]
    nbits = 8 * nbytes
    idx = np.arange(nbits)
    src = None
    for j in range(int(nbits - 1).bit_length()):
        w = np.packbits(((idx >> j) & 1).astype(np.uint8), bitorder="little")
        out = np.unpackbits(pack_ref(qt, w, N, K), bitorder="little").astype(np.int64)
        src = out << j if src is None else src | (out << j)
    return src, nbits


@pytest.mark.parametrize("qt", F.QTYPES)
def test_pack_ref_is_a_permutation(qt):
    src, nbits = _source_bits(qt, 32, 512)
    assert src.size == nbits
    assert np.array_equal(np.sort(src), np.arange(nbits))


@pytest.mark.parametrize("qt", F.QTYPES)
def test_pack_ref_chunks_hold_their_tile(qt):
    N, K = 32, 512
    src, nbits = _source_bits(qt, N, K)
    row_bits = nbits // N
    ub = 8 * unit_bytes(qt)
    row, unit = src // row_bits, (src % row_bits) // ub
    chunk = np.arange(nbits) // (16 * ub)  # chunk = tile * n_units + unit, n_units = 2
    assert np.array_equal(row // 16, chunk // 2)
    assert np.array_equal(unit, chunk % 2)


@pytest.mark.parametrize("qt", [F.Q4_K, F.Q6_K])
def test_pack_ref_headers_whole_and_lanes_hold_their_row(qt):
    """Headers (Q4_K: d, dmin, scales; Q6_K: scales, d) are copied byte for
    byte; the quant bits of a 16-byte lane group stay in that lane's words."""
    src, nbits = _source_bits(qt, 16, 256)
    ub = 8 * unit_bytes(qt)
    hdr = slice(8 * 2048, 8 * 2304) if qt == F.Q4_K else slice(8 * 3072, 8 * 3360)
    o = np.arange(nbits)[hdr]
    assert np.array_equal(src[hdr] % 8, o % 8)  # whole bytes
    # quant words of lane l = n + 16 g come from row n
    q_end = 8 * (2048 if qt == F.Q4_K else 3072)
    lane = (np.arange(q_end) % (8 * 1024)) // 128
    assert np.array_equal(src[:q_end] // ub, lane & 15)


def test_pack_ref_zero_padding():
    qt = F.Q8_0
    N, K = 5, 96
    w = synth.matrix(qt, N, K, synth.stream_for(1, "pad"))
    packed = pack_ref(qt, w, N, K)
    assert packed.size == 1 * 1 * 16 * 272
    assert np.count_nonzero(packed) <= w.size
