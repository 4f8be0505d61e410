"""GPU: ihip_gemm_q_ex, the matmul with its input transform fused (RMSNorm,
SiLU gating, row-strided input, reuse of prepared activations), against the
oracle's fp64 product of the transformed input (RMSNorm from the oracle's
rmsnorm, src/ModelCPU.jl:110-122; SiLU gating in float64)."""
import numpy as np
import pytest

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


def _rms_rows(x, w, eps):
    return np.stack([O.rmsnorm(r, eps, w) for r in x]).astype(np.float32)


@pytest.mark.parametrize("qt", F.QTYPES)
@pytest.mark.parametrize("packed", [False, True])
def test_rmsnorm_input(ih, qt, packed):
    N, K = 200, 1024
    rng = np.random.default_rng(qt + 3 * packed)
    w = synth.matrix(qt, N, K, synth.stream_for(N, f"rn{qt}"))
    wd = _dev(w)
    fl = ih.GEMM_F32
    if packed:
        wd = ih.pack_weights(qt, wd, N, K)
        fl |= ih.GEMM_PACKED
    nw = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    for M in (1, 5, 8, 24):
        x = (3.0 * rng.standard_normal((M, K))).astype(np.float32)
        for weight in (None, nw):
            ref = O.gemv_f64(qt, w, _rms_rows(x, weight, 1e-6), M, N, K)
            got = ih.gemm_q_ex(qt, wd, _dev(x), N, K, act=ih.ACT_RMSNORM,
                               norm_w=None if weight is None else _dev(weight), eps=1e-6, flags=fl).cpu().numpy()
            assert rel_l2(got, ref) < 1e-5, (M, weight is None)


@pytest.mark.parametrize("qt", [F.Q4_K, F.Q6_K])
def test_silu_mul_input_strided(ih, qt):
    N, K = 96, 512
    rng = np.random.default_rng(11)
    w = synth.matrix(qt, N, K, synth.stream_for(5, f"sl{qt}"))
    wp = ih.pack_weights(qt, _dev(w), N, K)
    for M in (1, 5, 8):
        gu = rng.standard_normal((M, 2 * K + 8)).astype(np.float32)  # ldx = 2K + 8
        g, u = gu[:, :K].astype(np.float64), gu[:, K:2 * K].astype(np.float64)
        a = (g / (1.0 + np.exp(-g)) * u).astype(np.float32)
        ref = O.gemv_f64(qt, w, a, M, N, K)
        got = ih.gemm_q_ex(qt, wp, _dev(gu), N, K, act=ih.ACT_SILU_MUL,
                           flags=ih.GEMM_F32 | ih.GEMM_PACKED).cpu().numpy()
        assert rel_l2(got, ref) < 1e-5, M


def test_strided_plain_and_reuse(ih):
    import torch
    qt = F.Q4_K
    K, N1, N2 = 1024, 160, 64
    rng = np.random.default_rng(12)
    w1 = synth.matrix(qt, N1, K, synth.stream_for(1, "r1"))
    w2 = synth.matrix(qt, N2, K, synth.stream_for(2, "r2"))
    p1, p2 = ih.pack_weights(qt, _dev(w1), N1, K), ih.pack_weights(qt, _dev(w2), N2, K)
    fl = ih.GEMM_F32 | ih.GEMM_PACKED
    for M in (1, 5, 8):
        big = _dev(rng.standard_normal((M, K + 64)).astype(np.float32))
        x = big[:, 32:32 + K]  # row-strided view
        xr = x.cpu().numpy()
        ws = torch.empty(ih.quantized_kernels.gemm_ws_bytes(qt, M, max(N1, N2), K, fl), dtype=torch.uint8,
                         device="cuda")
        y1 = ih.gemm_q_ex(qt, p1, x, N1, K, act=ih.ACT_RMSNORM, flags=fl, ws=ws)
        y2 = ih.gemm_q_ex(qt, p2, x, N2, K, act=ih.ACT_RMSNORM, flags=fl | ih.GEMM_REUSE, ws=ws)
        y2b = ih.gemm_q_ex(qt, p2, x, N2, K, act=ih.ACT_RMSNORM, flags=fl)
        assert torch.equal(y2, y2b)
        rr = _rms_rows(xr, None, 1e-6)
        assert rel_l2(y1.cpu().numpy(), O.gemv_f64(qt, w1, rr, M, N1, K)) < 1e-5
        y3 = ih.gemm_q_ex(qt, p1, x, N1, K, flags=fl)
        assert rel_l2(y3.cpu().numpy(), O.gemv_f64(qt, w1, xr, M, N1, K)) < 1e-5


def test_ex_errors(ih):
    import torch
    qt = F.Q4_K
    w = ih.pack_weights(qt, _dev(synth.matrix(qt, 16, 256, 1)), 16, 256)
    x = torch.zeros(40, 512, device="cuda")
    with pytest.raises(ValueError):  # rows narrower than 2K: the wrapper refuses before the C ABI
        ih.gemm_q_ex(qt, w, x[:, :256], 16, 256, act=ih.ACT_SILU_MUL)
    # the C ABI's own check of the same case (ldx < 2K)
    import ctypes as C
    ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    y = torch.empty(40, 16, device="cuda")
    gi = ih._lib.GemmInput(x.data_ptr(), 256, ih.ACT_SILU_MUL, None, 1e-6, None, 0, 0)
    assert ih.load().ihip_gemm_q_ex(qt, w.data_ptr(), C.byref(gi), y.data_ptr(), 40, 16, 256, ih.GEMM_PACKED,
                                    ws.data_ptr(), ws.numel(), None) == -22
    with pytest.raises(ih.HipError):  # reuse with M > 32 fp32-accurate
        ih.gemm_q_ex(qt, w, x[:, :256], 16, 256, flags=ih.GEMM_F32 | ih.GEMM_PACKED | ih.GEMM_REUSE)
    with pytest.raises(ih.HipError):
        ih.gemm_q_ex(qt, w, x[:5, :256], 16, 256, act=7)


@pytest.mark.parametrize("qt2", [F.Q4_K, F.Q6_K])
def test_defer_and_fold_residual(ih, qt2):
    """A deferred down projection (K split over slices) folded into the next
    matmul's input stage equals the accumulate-then-matmul sequence bit for
    bit: same slice order, same residual add."""
    import torch
    K1, H, N2 = 12288, 512, 96  # first matmul: [H x K1] (3 K-slices), second: [N2 x H]
    rng = np.random.default_rng(31)
    w1 = synth.matrix(F.Q6_K, H, K1, synth.stream_for(1, "d1"))
    w2 = synth.matrix(qt2, N2, H, synth.stream_for(2, "d2"))
    p1, p2 = ih.pack_weights(F.Q6_K, _dev(w1), H, K1), ih.pack_weights(qt2, _dev(w2), N2, H)
    fl = ih.GEMM_F32 | ih.GEMM_PACKED
    for M in (1, 5, 8):
        h = _dev(rng.standard_normal((M, K1)).astype(np.float32))
        x0 = _dev(rng.standard_normal((M, H)).astype(np.float32))
        # reference: x += W1 h (reduced), then y = W2 rmsnorm(x)
        xr = x0.clone()
        ih.gemm_q(F.Q6_K, p1, h, H, K1, flags=fl | ih.GEMM_ACCUM, out=xr)
        yr = ih.gemm_q_ex(qt2, p2, xr, N2, H, act=ih.ACT_RMSNORM, flags=fl)
        # fused: deferred partials, folded by the next input stage
        ws1 = torch.empty(ih.quantized_kernels.gemm_ws_bytes(F.Q6_K, M, H, K1, fl), dtype=torch.uint8, device="cuda")
        ih.gemm_q_ex(F.Q6_K, p1, h, H, K1, flags=fl | ih.GEMM_DEFER, ws=ws1)
        parts = ih.gemm_partials(F.Q6_K, M, H, K1, fl, ws1)
        assert parts[1] >= 2
        xf = x0.clone()
        yf = ih.gemm_q_ex(qt2, p2, xf, N2, H, act=ih.ACT_RMSNORM, flags=fl, add=parts)
        assert torch.equal(xf, xr), M
        assert torch.equal(yf, yr), M
        ref = O.gemv_f64(F.Q6_K, w1, h.cpu().numpy(), M, H, K1) + x0.cpu().numpy()
        assert rel_l2(xf.cpu().numpy(), ref) < 1e-5


@pytest.mark.parametrize("M,fl_prod,fl_cons", [(5, 1, 1), (24, 1, 1), (64, 2, 2), (40, 2, 1)])
def test_sum_out(ih, M, fl_prod, fl_cons):
    """GEMM_SUM_OUT: a deferred, possibly K-sliced product wider than the
    consumer's K ([q; k; v] feeding o) is summed by the consumer's input
    stage, which stores the whole sum (the columns past K by workgroups of
    their own) as the fp32 sum of the slices in slice order, and the
    consumer's product equals a plain call on that sum bit for bit. M = 40
    fp32-accurate runs as two launches over token halves."""
    import torch
    H, NQ, NKV, N2 = 4096, 512, 128, 256
    N1 = NQ + 2 * NKV
    rng = np.random.default_rng(M)
    w1 = synth.matrix(F.Q4_K, N1, H, synth.stream_for(3, "so1"))
    w2 = synth.matrix(F.Q4_K, N2, NQ, synth.stream_for(4, "so2"))
    p1, p2 = ih.pack_weights(F.Q4_K, _dev(w1), N1, H), ih.pack_weights(F.Q4_K, _dev(w2), N2, NQ)
    fp, fc = fl_prod | ih.GEMM_PACKED, fl_cons | ih.GEMM_PACKED
    x = _dev(rng.standard_normal((M, H)).astype(np.float32))
    ws1 = torch.empty(ih.quantized_kernels.gemm_ws_bytes(F.Q4_K, M, N1, H, fp), dtype=torch.uint8, device="cuda")
    ih.gemm_q_ex(F.Q4_K, p1, x, N1, H, flags=fp | ih.GEMM_DEFER, ws=ws1)
    parts = ih.gemm_partials(F.Q4_K, M, N1, H, fp, ws1)
    ptr, ns, stride = parts
    wf = ws1.view(torch.float32)
    off = (ptr - ws1.data_ptr()) // 4
    sl = wf[off:off + ns * stride].view(ns, stride)[:, :M * N1].reshape(ns, M, N1).cpu().numpy()
    ref = sl[0].copy()
    for j in range(1, ns):
        ref = (ref + sl[j]).astype(np.float32)
    qkv = torch.full((M, N1), float("nan"), device="cuda")
    y = ih.gemm_q_ex(F.Q4_K, p2, qkv, N2, NQ, flags=fc | ih.GEMM_SUM_OUT, add=parts)
    assert np.array_equal(qkv.cpu().numpy(), ref), (M, ns)
    y_plain = ih.gemm_q_ex(F.Q4_K, p2, qkv[:, :NQ], N2, NQ, flags=fc)
    assert torch.equal(y, y_plain), (M, ns)
    assert rel_l2(y.cpu().numpy(), O.gemv_f64(F.Q4_K, w2, ref[:, :NQ], M, N2, NQ)) < (1e-5 if fl_cons == 1 else 1e-2)


def test_sum_out_errors(ih):
    import ctypes as C
    import torch
    qt = F.Q4_K
    w = ih.pack_weights(qt, _dev(synth.matrix(qt, 16, 256, 1)), 16, 256)
    x = torch.zeros(5, 512, device="cuda")
    sl = torch.from_numpy(np.random.default_rng(7).standard_normal((2, 5, 512)).astype(np.float32)).cuda()
    with pytest.raises(ValueError):  # no add slices
        ih.gemm_q_ex(qt, w, x, 16, 256, flags=ih.GEMM_PACKED | ih.GEMM_SUM_OUT)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    y = torch.empty(5, 16, device="cuda")
    L = ih.load()

    def call(act, ldx, xp=x.data_ptr(), add=sl.data_ptr()):
        gi = ih._lib.GemmInput(xp, ldx, act, None, 1e-6, add, 2, 5 * 512)
        return L.ihip_gemm_q_ex(qt, w.data_ptr(), C.byref(gi), y.data_ptr(), 5, 16, 256,
                                ih.GEMM_PACKED | ih.GEMM_SUM_OUT, ws.data_ptr(), ws.numel(), None)
    assert call(ih.ACT_SILU_MUL, 512) == -22   # not with SiLU gating
    assert call(ih.ACT_PLAIN, 508) == -22      # ldx % 8
    assert call(ih.ACT_PLAIN, 512, xp=None) != 0  # x is the destination
    assert call(ih.ACT_PLAIN, 512) == 0
    torch.cuda.synchronize()
    assert torch.equal(x, sl[0] + sl[1])


@pytest.mark.parametrize("packed", [False, True])
def test_mlp_forward(ih, packed):
    """ihip_mlp_forward (the MLP half of a decoder layer, src/ModelCPU.jl:884-889
    with mlp_forward, :447-473) equals the two ihip_gemm_q_ex calls it stands
    for bit for bit, and the oracle's rmsnorm -> [gate; up] -> SiLU gating ->
    down -> residual add in float64 to 1e-5."""
    import torch
    H, FF = 512, 1024
    rng = np.random.default_rng(50 + packed)
    wgu = synth.matrix(F.Q4_K, 2 * FF, H, synth.stream_for(7, "mlp_gu"))
    wd = synth.matrix(F.Q6_K, H, FF, synth.stream_for(8, "mlp_down"))
    gu_d, d_d = _dev(wgu), _dev(wd)
    fl = ih.GEMM_F32
    if packed:
        gu_d, d_d = ih.pack_weights(F.Q4_K, gu_d, 2 * FF, H), ih.pack_weights(F.Q6_K, d_d, H, FF)
        fl |= ih.GEMM_PACKED
    nw = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    nw_d = _dev(nw)
    for M in (1, 5, 8, 20):
        x0 = (2.0 * rng.standard_normal((M, H))).astype(np.float32)
        x1 = _dev(x0)
        ih.mlp_forward_(F.Q4_K, gu_d, F.Q6_K, d_d, x1, H, FF, norm_w=nw_d, flags=fl)
        gu = ih.gemm_q_ex(F.Q4_K, gu_d, _dev(x0), 2 * FF, H, act=ih.ACT_RMSNORM, norm_w=nw_d, flags=fl)
        x2 = _dev(x0)
        ih.gemm_q_ex(F.Q6_K, d_d, gu, H, FF, act=ih.ACT_SILU_MUL, flags=fl | ih.GEMM_ACCUM, out=x2)
        assert torch.equal(x1, x2), M
        n = _rms_rows(x0, nw, 1e-6)
        gup = O.gemv_f64(F.Q4_K, wgu, n, M, 2 * FF, H)
        g, u = gup[:, :FF], gup[:, FF:]
        with np.errstate(over="ignore"):  # exp(-g) = inf for very negative g: silu -> 0
            h = (g / (1.0 + np.exp(-g)) * u).astype(np.float32)
        delta = O.gemv_f64(F.Q6_K, wd, h, M, H, FF)
        assert rel_l2(x1.cpu().numpy() - x0, delta) < 1e-5, M
