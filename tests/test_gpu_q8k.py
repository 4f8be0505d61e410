"""GPU: the Q8_K exports (quantize_row_q8_K, vec_dot_q{4,5,6}_K_q8_K; the
remaining C symbols bound by src/QuantizedKernels.jl:149-175) called through
the C ABI with host pointers, bit for bit against the reference's own C
kernel built from src/kernels/quant_kernels.c into oracle/_ref (or, where
that build is absent, the oracle's restatement, which the CPU tests pin to
it bit for bit)."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from inferno_hip import formats as F
from inferno_hip import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import inferno_hip
    assert inferno_hip.quant_kernels_available(), inferno_hip._lib.last_error()
    return inferno_hip.load()


def _quantize(L, x):
    q8 = np.zeros((x.size // 256) * 292, dtype=np.uint8)
    L.quantize_row_q8_K(x.ctypes.data, q8.ctypes.data, x.size)
    assert L.ihip_last_status() == 0, L.ihip_last_error()
    return q8


def _want_quantize(x):
    return O.ref_quantize_q8_K(x) if O.ref_available() else O.quantize_q8_K(x)


def _want_dot(qt, w, q8, nb):
    return O.ref_vec_dot(qt, w, q8, nb) if O.ref_available() else O.vec_dot(qt, w, q8, nb)


def test_quantize_row_q8_K_bytes(L):
    rng = np.random.default_rng(8)
    cases = [rng.standard_normal(4096), rng.standard_normal(256) * 1e-3, rng.integers(-127, 128, 512),
             np.concatenate([np.zeros(256), rng.standard_normal(256) * 1e4]),   # an all-zero block (d = 0)
             (rng.integers(-3, 4, 1024) + 0.5)]                                 # halves: round away from zero
    for x in cases:
        x = np.ascontiguousarray(x, dtype=np.float32)
        got = _quantize(L, x)
        assert np.array_equal(got, _want_quantize(x)), x.size


@pytest.mark.parametrize("qt", [F.Q4_K, F.Q5_K, F.Q6_K])
def test_vec_dot_bits(L, qt):
    rng = np.random.default_rng(qt)
    for nb in (1, 4, 16):
        w = synth.blocks(qt, nb, synth.stream_for(qt, f"vd{nb}"))
        for scale in (1.0, 1e-3, 50.0):
            q8 = _quantize(L, (rng.standard_normal(256 * nb) * scale).astype(np.float32))
            got = np.float32(getattr(L, f"vec_dot_{F.NAMES[qt][:2].lower()}_K_q8_K")(w.ctypes.data, q8.ctypes.data, nb))
            want = np.float32(_want_dot(qt, w, q8, nb))
            assert got.view(np.uint32) == want.view(np.uint32), (nb, scale, got, want)
    # nb = 0: the empty sum
    assert getattr(L, f"vec_dot_{F.NAMES[qt][:2].lower()}_K_q8_K")(w.ctypes.data, q8.ctypes.data, 0) == 0.0
