"""CPU checks of the packed layout's numpy statement: with no padding it is a
byte permutation of the GGUF matrix in which every quant, scale and d byte
appears exactly once, and each 16-row tile of each 256-element unit stays in
its own chunk."""
import numpy as np
import pytest

from _packref import pack_ref, unit_bytes
from inferno_hip import formats as F
from inferno_hip import synth


@pytest.mark.parametrize("qt", F.QTYPES)
def test_pack_ref_is_a_permutation(qt):
    N, K = 32, 512
    # distinct labels per byte position: pack a matrix of byte indices mod 251
    # twice, with offsets, and check the position map is a bijection
    nbytes = N * K // F.BLOCK_ELEMS[qt] * F.BLOCK_BYTES[qt]
    idx = np.arange(nbytes)
    lo = pack_ref(qt, (idx % 256).astype(np.uint8), N, K).astype(np.int64)
    hi = pack_ref(qt, ((idx // 256) % 256).astype(np.uint8), N, K).astype(np.int64)
    hh = pack_ref(qt, (idx // 65536).astype(np.uint8), N, K).astype(np.int64)
    pos = lo + 256 * hi + 65536 * hh
    assert pos.size == nbytes
    assert np.array_equal(np.sort(pos), idx)


@pytest.mark.parametrize("qt", F.QTYPES)
def test_pack_ref_chunks_hold_their_tile(qt):
    N, K = 32, 512
    nbytes = N * K // F.BLOCK_ELEMS[qt] * F.BLOCK_BYTES[qt]
    row_bytes = nbytes // N
    idx = np.arange(nbytes)
    row = idx // row_bytes
    unit = (idx % row_bytes) // unit_bytes(qt)
    tag = (row // 16) * 4 + unit  # tile * n_units + unit, n_units = 2
    packed = pack_ref(qt, tag.astype(np.uint8), N, K)
    CH = 16 * unit_bytes(qt)
    for c in range(packed.size // CH):
        assert np.all(packed[c * CH:(c + 1) * CH] == (c // 2) * 4 + c % 2)


def test_pack_ref_zero_padding():
    qt = F.Q8_0
    N, K = 5, 96
    w = synth.matrix(qt, N, K, synth.stream_for(1, "pad"))
    packed = pack_ref(qt, w, N, K)
    assert packed.size == 1 * 1 * 16 * 272
    assert np.count_nonzero(packed) <= w.size
