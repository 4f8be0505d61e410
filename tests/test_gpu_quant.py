"""GPU parity: dequant (bit-exact), device synthesis (byte-exact), fused
dequant-matmul (rel-L2 1e-5 fp32-accurate / 1e-2 half MFMA) and the host
drop-in q*_gemv entry points, all against the CPU oracle."""
import numpy as np
import pytest

from _util import rel_l2

import oracle as O
from inferno_hip import formats as F
from inferno_hip import synth

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-5   # north-star bar for the fp32-accumulate path
TOL_HALF = 1e-2  # north-star bar for the half-precision MFMA path


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


def _edge_blocks(qt):
    """Synthetic blocks plus hand-set edge cases of the fp16 scale fields."""
    bb = F.BLOCK_BYTES[qt]
    b = synth.blocks(qt, 24, synth.stream_for(7, f"edge{qt}")).reshape(24, bb).copy()
    d_off = 208 if qt == F.Q6_K else 0
    specials = [0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0xC000, 0x7C00, 0x7E00]
    for i, h in enumerate(specials):
        b[i, d_off:d_off + 2] = np.array([h & 0xFF, h >> 8], dtype=np.uint8)
        if qt in (F.Q4_K, F.Q5_K):  # dmin too
            b[i, 2:4] = np.array([specials[-1 - i] & 0xFF, specials[-1 - i] >> 8], dtype=np.uint8)
    return b.reshape(-1)


@pytest.mark.parametrize("qt", F.QTYPES)
def test_dequant_bit_exact(ih, qt):
    data = np.concatenate([_edge_blocks(qt), synth.blocks(qt, 1000, synth.stream_for(3, "dq"))])
    nblk = data.size // F.BLOCK_BYTES[qt]
    n = nblk * F.BLOCK_ELEMS[qt]
    ref = O.dequant(qt, data, nblk, F.BLOCK_ELEMS[qt])
    got = ih.dequant(qt, _dev(data), n).cpu().numpy()
    rb, gb = ref.view(np.uint32), got.view(np.uint32)
    both_nan = np.isnan(ref) & np.isnan(got)
    bad = (rb != gb) & ~both_nan
    assert not bad.any(), f"{F.NAMES[qt]}: {bad.sum()} mismatches, first at {np.argmax(bad)}"


@pytest.mark.parametrize("qt", F.QTYPES)
def test_device_synth_matches_host(ih, qt):
    st = synth.stream_for(11, "w")
    host = synth.blocks(qt, 777, st, first_block=5)
    dev = ih.quantized_kernels.synth_blocks(qt, st, 777, first_block=5).cpu().numpy()
    assert np.array_equal(host, dev)


SHAPES = [(40, 256), (128, 512), (200, 2048), (3072, 1024)]
MS = [1, 2, 3, 5, 8, 9, 16, 33, 64]


@pytest.mark.parametrize("qt", F.QTYPES)
@pytest.mark.parametrize("N,K", SHAPES)
def test_gemm_fp32_accurate(ih, qt, N, K):
    rng = np.random.default_rng(N * 7 + K + qt)
    w = synth.matrix(qt, N, K, synth.stream_for(N + K, f"gemm{qt}"))
    wd = _dev(w)
    for M in MS:
        x = rng.standard_normal((M, K)).astype(np.float32)
        ref = O.gemv_f64(qt, w, x, M, N, K)
        got = ih.gemm_q(qt, wd, _dev(x), N, K, flags=ih.GEMM_F32).cpu().numpy()
        err = rel_l2(got, ref)
        print(f"{F.NAMES[qt]} N={N} K={K} M={M} f32 rel-L2={err:.3e}", flush=True)
        assert err <= TOL_F32, (M, err)


@pytest.mark.parametrize("qt", F.QTYPES)
def test_gemm_half_mfma(ih, qt):
    N, K = 512, 2048
    rng = np.random.default_rng(qt)
    w = synth.matrix(qt, N, K, synth.stream_for(5, f"half{qt}"))
    wd = _dev(w)
    for M in (1, 7, 16, 17, 40, 64):
        x = rng.standard_normal((M, K)).astype(np.float32)
        ref = O.gemv_f64(qt, w, x, M, N, K)
        got = ih.gemm_q(qt, wd, _dev(x), N, K, flags=ih.GEMM_HALF).cpu().numpy()
        err = rel_l2(got, ref)
        print(f"{F.NAMES[qt]} M={M} half rel-L2={err:.3e}", flush=True)
        assert err <= TOL_HALF, (M, err)
        auto = ih.gemm_q(qt, wd, _dev(x), N, K).cpu().numpy()
        assert rel_l2(auto, ref) <= (TOL_F32 if M < 16 else TOL_HALF)


def test_gemm_invariants(ih):
    """Linearity, the M-row result equals M independent M=1 calls, the
    accumulate flag, and large-magnitude activations (per-token scaling)."""
    import torch
    qt, N, K = F.Q4_K, 256, 1024
    w = synth.matrix(qt, N, K, synth.stream_for(1, "inv"))
    wd = _dev(w)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, K)).astype(np.float32)
    y = ih.gemm_q(qt, wd, _dev(x), N, K, flags=ih.GEMM_F32).cpu().numpy().astype(np.float64)
    for m in range(5):
        y1 = ih.gemm_q(qt, wd, _dev(x[m:m + 1]), N, K, flags=ih.GEMM_F32).cpu().numpy()[0]
        assert rel_l2(y1, y[m]) <= 1e-6
    y2 = ih.gemm_q(qt, wd, _dev(2.0 * x[0:1] + x[1:2]), N, K, flags=ih.GEMM_F32).cpu().numpy()[0]
    assert rel_l2(y2, 2.0 * y[0] + y[1]) <= 1e-5
    acc = _dev(np.ones((5, N), dtype=np.float32))
    ih.gemm_q(qt, wd, _dev(x), N, K, flags=ih.GEMM_F32 | ih.GEMM_ACCUM, out=acc)
    assert rel_l2(acc.cpu().numpy(), y + 1.0) <= 1e-5
    big = (x * 3.0e4).astype(np.float32)  # beyond fp16 range before scaling
    ref = O.gemv_f64(qt, w, big, 5, N, K)
    got = ih.gemm_q(qt, wd, _dev(big), N, K, flags=ih.GEMM_F32).cpu().numpy()
    assert rel_l2(got, ref) <= TOL_F32
    tiny = (x * 1.0e-30).astype(np.float32)
    ref = O.gemv_f64(qt, w, tiny, 5, N, K)
    got = ih.gemm_q(qt, wd, _dev(tiny), N, K, flags=ih.GEMM_F32).cpu().numpy()
    assert rel_l2(got, ref) <= TOL_F32
    zero = torch.zeros((3, K), dtype=torch.float32, device="cuda")
    assert float(ih.gemm_q(qt, wd, zero, N, K).abs().max()) == 0.0


@pytest.mark.parametrize("qt", F.QTYPES)
def test_dropin_host_gemv(ih, qt):
    """The reference-named host entry points (quant_kernels.c:602-697)."""
    N, K = 300, 1024
    w = synth.matrix(qt, N, K, synth.stream_for(9, f"dropin{qt}"))
    x = np.random.default_rng(qt).standard_normal(K).astype(np.float32)
    out = np.zeros(N, dtype=np.float32)
    ih.quantized_kernels.GEMV_BY_QTYPE[qt](out, w, x, K, N)
    ref = O.gemv_f64(qt, w, x, 1, N, K)[0]
    assert rel_l2(out, ref) <= TOL_F32
    # second call hits the weight cache and must give the same answer
    out2 = np.zeros(N, dtype=np.float32)
    ih.quantized_kernels.GEMV_BY_QTYPE[qt](out2, w, x, K, N)
    assert np.array_equal(out, out2)


def test_dropin_cache_sees_reused_buffer(ih):
    """The drop-in weight cache is keyed by (pointer, bytes, type, N, K) with a
    fingerprint of sampled bytes: a host buffer overwritten in place (as a
    garbage-collected array's address reused by a new one of the same size)
    gives the new matrix's result, and the same bytes read as another type
    of equal byte size (Q4_K 272 x 1024 and Q8_0 288 x 512: 156672 bytes)
    give that type's result."""
    qk = ih.quantized_kernels
    N, K = 272, 1024
    buf = np.empty(N * (K // 256) * 144, dtype=np.uint8)
    x = np.random.default_rng(11).standard_normal(K).astype(np.float32)
    outs = []
    for tag in ("first", "second"):
        buf[:] = synth.matrix(F.Q4_K, N, K, synth.stream_for(12, f"reuse.{tag}"))
        out = np.zeros(N, dtype=np.float32)
        qk.q4_k_gemv_(out, buf, x, K, N)  # (np.ascontiguousarray keeps buf's address)
        assert rel_l2(out, O.gemv_f64(F.Q4_K, buf, x, 1, N, K)[0]) <= TOL_F32, tag
        outs.append(out)
    assert not np.array_equal(outs[0], outs[1])
    n8, k8 = 288, 512
    assert n8 * (k8 // 32) * 34 == buf.size
    xq = np.random.default_rng(12).standard_normal(k8).astype(np.float32)
    out8 = np.zeros(n8, dtype=np.float32)
    qk.q8_0_gemv_(out8, buf, xq, k8, n8)
    ref8 = O.gemv_f64(F.Q8_0, buf, xq, 1, n8, k8)[0]
    # (Q4_K bytes read as Q8_0 blocks: some fp16 d fields are NaN or Inf, and
    # those rows are NaN in both; the finite rows carry the comparison)
    assert np.array_equal(np.isnan(out8), np.isnan(ref8))
    fin = np.isfinite(ref8)
    assert fin.sum() > n8 // 4 and rel_l2(out8[fin], ref8[fin]) <= TOL_F32
    ih.load().ihip_weight_cache_clear()


def test_errors(ih):
    import torch
    from inferno_hip._lib import HipError
    wd = torch.zeros(144 * 4, dtype=torch.uint8, device="cuda")
    x = torch.zeros((1, 300), dtype=torch.float32, device="cuda")
    with pytest.raises(HipError) as e:
        ih.gemm_q(F.Q4_K, wd, x, 4, 300)
    assert e.value.status == -22
    x = torch.zeros((65, 256), dtype=torch.float32, device="cuda")
    with pytest.raises(HipError):
        ih.gemm_q(F.Q4_K, wd, x, 4, 256)
    L = ih.load()
    assert L.ihip_gemm_q(F.Q4_K, None, None, None, 1, 1, 256, 0, None, 0, None) == -14
    assert L.ihip_dequant(99, wd.data_ptr(), wd.data_ptr(), 256, None) == -22
