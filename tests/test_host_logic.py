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


def test_speculative_stats_hand_trace():
    """generate_speculative_cpu's counters (src/SpeculativeDecoding.jl:114-172),
    worked by hand for gamma = 4, a 3-token prompt, max_tokens = 10 and steps
    returning 5 tokens (4 drafts + bonus), 2 (1 draft + residual), 5:
      after step 1: tokens_generated 5, total_draft_tokens 4, total_accepted 5
      after step 2: 7, 8, 7
      after step 3: 12 (the inner loop pushes every returned token), 12, 12,
      and 12 >= 10 ends the loop.
    acceptance_rate = 12 / 12 = 1.0 (:163, returned tokens over drafted ones);
    speedup_estimate = (12 - 3) / (12 + 12) * (1 + 4) = 1.875 (:164; the
    prompt length is subtracted although tokens_generated never counted it)."""
    s = SpeculativeStats(gamma=4, prompt_len=3)
    returned = iter((5, 2, 5, 5, 5))
    steps = 0
    while s.tokens_generated < 10:   # the loop condition of :142 (and the break of :158)
        s.record(next(returned))
        steps += 1
    d = s.as_dict()
    assert steps == 3
    assert d == {"acceptance_rate": 1.0, "draft_tokens_generated": 12, "tokens_accepted": 12,
                 "speedup_estimate": 1.875}
    # a run that rejects early: two steps of 1 token each (residual at position 0)
    s = SpeculativeStats(gamma=4, prompt_len=0)
    s.record(1)
    s.record(1)
    assert s.as_dict() == {"acceptance_rate": 0.25, "draft_tokens_generated": 8, "tokens_accepted": 2,
                           "speedup_estimate": 2 / 10 * 5}


def test_oracle_rmsnorm_closed_forms():
    """orc_rmsnorm (src/ModelCPU.jl:110-122: x / sqrt(mean(x^2) + eps) * w) on
    inputs whose result is known in closed form."""
    import oracle as O
    eps = 1e-6
    # constant vector c: mean square c^2, result c / sqrt(c^2 + eps) * w
    for c, n in ((3.0, 16), (-0.5, 7), (1e3, 4096)):
        x = np.full(n, c, np.float32)
        w = np.linspace(0.5, 2.0, n).astype(np.float32)
        want = c / np.sqrt(c * c + eps) * w.astype(np.float64)
        assert np.allclose(O.rmsnorm(x, eps, w), want, rtol=3e-7, atol=0)
    # [3, 4]: mean square 12.5
    got = O.rmsnorm(np.array([3.0, 4.0], np.float32), 0.0)
    assert np.allclose(got, [3 / np.sqrt(12.5), 4 / np.sqrt(12.5)], rtol=3e-7, atol=0)
    # one nonzero of n = 4: mean square a^2 / 4, result +-2 (eps negligible)
    got = O.rmsnorm(np.array([0.0, -7.0, 0.0, 0.0], np.float32), 0.0)
    assert got.tolist() == [0.0, -2.0, 0.0, 0.0]
    # all zeros: eps alone, result 0
    assert not O.rmsnorm(np.zeros(8, np.float32), eps).any()


def test_wrappers_reject_bad_tensors_before_the_library():
    """The Python wrappers validate every tensor (device, dtype, shape,
    layout) before a pointer reaches the C ABI, which cannot see sizes: host
    tensors, wrong dtypes and mis-shaped arguments raise ValueError."""
    import pytest
    import torch
    import inferno_hip as ih
    f32 = lambda *s: torch.zeros(*s, dtype=torch.float32)  # noqa: E731  (host tensors)
    i32 = lambda *s: torch.zeros(*s, dtype=torch.int32)  # noqa: E731
    with pytest.raises(ValueError, match="GPU"):
        ih.spec_accept(f32(2, 5, 64), f32(2, 4, 64), i32(2, 4), 0.8, f32(2, 4), f32(2), f32(2))
    with pytest.raises(ValueError, match="GPU"):
        ih.greedy_verify(f32(1, 5, 64), i32(1, 4))
    with pytest.raises(ValueError, match="GPU"):
        ih.tree_accept(f32(4, 64), f32(4, 64), i32(4), i32(4), 1.0, f32(4))
    with pytest.raises(ValueError, match="GPU"):
        ih.gemm_q(ih.formats.Q4_K, torch.zeros(144, dtype=torch.uint8), f32(1, 256), 1, 256)
    with pytest.raises(ValueError):
        ih.gemm_q_ex(ih.formats.Q4_K, torch.zeros(144, dtype=torch.uint8), f32(1, 256), 1, 256)
    with pytest.raises(ValueError, match="torch tensor"):
        ih.quantized_kernels.check_tensor(None, "x")
