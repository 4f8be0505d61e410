"""Host-side logic: block formats, the seeded generator, and the
speculative statistics of generate_speculative_cpu (no GPU)."""
import numpy as np

from inferno_hip import formats as F, synth
from inferno_hip.speculative import SpeculativeStats


def test_block_sizes_match_reference():
    # src/QuantsCPU.jl:22-25, src/kernels/quant_kernels.c:24-62
    assert F.BLOCK_BYTES == {F.Q4_K: 144, F.Q5_K: 176, F.Q6_K: 210, F.Q8_0: 34}
    assert F.row_bytes(F.Q4_K, 4096) == 16 * 144
    assert F.matrix_bytes(F.Q6_K, 151936, 2048) == 255252480


def test_generator_deterministic_and_independent_blocks():
    st = synth.stream_for(0x1F3E0001, "w")
    a = synth.blocks(F.Q4_K, 10, st)
    assert np.array_equal(a, synth.blocks(F.Q4_K, 10, st))
    # block b depends only on (stream, b)
    tail = synth.blocks(F.Q4_K, 4, st, first_block=6)
    assert np.array_equal(a[6 * 144:], tail)


def test_generator_field_ranges():
    st = synth.stream_for(9, "ranges")
    for qt in F.QTYPES:
        b = synth.blocks(qt, 2000, st).reshape(2000, F.BLOCK_BYTES[qt])
        off = 208 if qt == F.Q6_K else 0
        d = b[:, off:off + 2].copy().view(np.float16).astype(np.float32).ravel()
        hi = 0.05 if qt in (F.Q4_K, F.Q5_K) else 0.02
        assert d.min() >= 0.000999 and d.max() <= hi * 1.001
        if qt in (F.Q4_K, F.Q5_K):
            sc, m = synth.unpack_scales_k4(b[:, 4:16])
            assert sc.max() == 63 and sc.min() == 0 and m.max() == 63
        if qt == F.Q6_K:
            s = b[:, 192:208].view(np.int8)
            assert s.min() == -32 and s.max() == 31
        if qt == F.Q8_0:
            q = b[:, 2:].view(np.int8)
            assert q.min() == -127 and q.max() == 127


def test_gaussian_moments():
    z = synth.gaussian(synth.stream_for(1, "g"), 200000)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01


def test_speculative_stats_formula():
    # src/SpeculativeDecoding.jl:163-164
    s = SpeculativeStats(gamma=4, prompt_len=3)
    s.tokens_generated = 0
    for n_out in (5, 2, 1, 5):
        s.record(n_out)
    d = s.as_dict()
    assert d["draft_tokens_generated"] == 16 and d["tokens_accepted"] == 13
    assert d["acceptance_rate"] == 13 / 16
    assert d["speedup_estimate"] == (13 - 3) / (16 + 13) * 5
