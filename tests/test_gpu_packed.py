"""GPU: the packed weight layout. The device packer matches the layout's
numpy statement byte for byte (including zero padding of rows past N and
Q8_0 blocks past K), and the matmul over packed weights returns exactly the
bits of the matmul over the GGUF bytes, whose parity with the oracle the
other GPU tests pin."""
import numpy as np
import pytest

from _packref import pack_ref
from _util import rel_l2

import oracle as O
from inferno_hip import formats as F
from inferno_hip import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ih():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import inferno_hip
    assert inferno_hip.quant_kernels_available(), inferno_hip._lib.last_error()
    return inferno_hip


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


SHAPES = [(16, 256), (40, 512), (100, 1024), (33, 4096)]


# every format at whole units, and Q8_0 alone at K past the last whole unit
# (the K-quants need K % 256 == 0)
PACK_CASES = [(qt, N, K) for N, K in SHAPES for qt in F.QTYPES] + [(F.Q8_0, 24, 96), (F.Q8_0, 17, 288)]


@pytest.mark.parametrize("qt,N,K", PACK_CASES)
def test_pack_layout(ih, qt, N, K):
    w = synth.matrix(qt, N, K, synth.stream_for(N * 3 + K, f"pk{qt}"))
    got = ih.pack_weights(qt, _dev(w), N, K).cpu().numpy()
    assert got.size == ih.packed_bytes(qt, N, K)
    assert np.array_equal(got, pack_ref(qt, w, N, K))


@pytest.mark.parametrize("qt", F.QTYPES)
@pytest.mark.parametrize("N,K", SHAPES)
def test_packed_gemm_identical(ih, qt, N, K):
    import torch
    rng = np.random.default_rng(N + K + qt)
    w = synth.matrix(qt, N, K, synth.stream_for(N + 5 * K, f"pg{qt}"))
    wd = _dev(w)
    wp = ih.pack_weights(qt, wd, N, K)
    for M in (1, 4, 5, 8, 13, 24, 64):
        x = _dev(rng.standard_normal((M, K)).astype(np.float32))
        for flags in (ih.GEMM_F32, ih.GEMM_HALF, ih.GEMM_AUTO):
            if flags == ih.GEMM_F32 and M > 32:
                continue
            a = ih.gemm_q(qt, wd, x, N, K, flags=flags).cpu().numpy()
            b = ih.gemm_q(qt, wp, x, N, K, flags=flags | ih.GEMM_PACKED).cpu().numpy()
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (M, flags)
        if M <= 8:
            ref = O.gemv_f64(qt, w, x.cpu().numpy(), M, N, K)
            y0 = torch.randn(M, N, device="cuda")
            y = y0.clone()
            ih.gemm_q(qt, wp, x, N, K, flags=ih.GEMM_F32 | ih.GEMM_PACKED | ih.GEMM_ACCUM, out=y)
            assert rel_l2((y - y0).cpu().numpy(), ref) < 1e-5


def test_packed_q8_0_tail(ih):
    """Q8_0 with K % 256 != 0 (the last unit holds 5 of 8 blocks): the padded
    blocks of the packed layout and the short last unit of the GGUF layout
    add nothing, at one token tile and at several, fp32-accurate and half;
    both layouts agree bit for bit."""
    qt = F.Q8_0
    N, K = 48, 32 * 13
    rng = np.random.default_rng(9)
    w = synth.matrix(qt, N, K, synth.stream_for(77, "tail"))
    wd = _dev(w)
    wp = ih.pack_weights(qt, wd, N, K)
    for M in (1, 5, 16, 24, 37, 64):
        x = rng.standard_normal((M, K)).astype(np.float32)
        ref = O.gemv_f64(qt, w, x, M, N, K)
        for fl, bar in ((ih.GEMM_F32, 1e-5), (ih.GEMM_HALF, 2e-3)):
            got = ih.gemm_q(qt, wp, _dev(x), N, K, flags=fl | ih.GEMM_PACKED).cpu().numpy()
            raw = ih.gemm_q(qt, wd, _dev(x), N, K, flags=fl).cpu().numpy()
            assert rel_l2(got, ref) < bar, (M, fl)
            assert np.array_equal(got, raw), (M, fl)
