"""GPU: the several-token-tile matmul (M = 16..64 half precision, 9..32
fp32-accurate) against the oracle's fp64 product of the dequantized weights
(dequant formulas of src/QuantizedKernels.jl:55-190 for the K-quants and
Q8_0). Shapes hit the edges of that kernel: rows past N inside the last
16-row tile, tokens past M inside the last token tile, one K-slice and
several, accumulation and deferred partials (both through the K-slice
partial buffer), and the RMSNorm input stage."""
import numpy as np
import pytest

from _util import rel_l2

import oracle as O
from inferno_hip import formats as F
from inferno_hip import synth

pytestmark = pytest.mark.gpu

TOL_HALF = 1e-2  # north-star bar for the half-precision MFMA path
SANITY_HALF = 2e-3  # fp16 operands land near 4e-4; a dropped term or index lands far above
TOL_F32 = 1e-5


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


@pytest.mark.parametrize("qt", F.QTYPES)
@pytest.mark.parametrize("K", [768, 2560])  # 3 units (one K-slice), 10 units (three)
def test_tall_half(ih, qt, K):
    import torch
    N = 200  # 12.5 tiles: the last tile has 8 padding rows
    rng = np.random.default_rng(K + 11 * qt)
    w = synth.matrix(qt, N, K, synth.stream_for(N + K, f"tall{qt}"))
    wp = ih.pack_weights(qt, _dev(w), N, K)
    fl = ih.GEMM_HALF | ih.GEMM_PACKED
    for M in (16, 37, 64):
        x = rng.standard_normal((M, K)).astype(np.float32)
        ref = O.gemv_f64(qt, w, x, M, N, K)
        got = ih.gemm_q(qt, wp, _dev(x), N, K, flags=fl).cpu().numpy()
        err = rel_l2(got, ref)
        print(f"{F.NAMES[qt]} K={K} M={M} half rel-L2={err:.3e}", flush=True)
        assert err <= TOL_HALF and err <= SANITY_HALF, (M, err)
        y0 = torch.randn(M, N, device="cuda")
        y = y0.clone()
        ih.gemm_q(qt, wp, _dev(x), N, K, flags=fl | ih.GEMM_ACCUM, out=y)
        assert rel_l2((y - y0).cpu().numpy(), ref) <= SANITY_HALF, M


@pytest.mark.parametrize("qt", [F.Q4_K, F.Q6_K])
def test_tall_fp32_accurate(ih, qt):
    N, K = 144, 1536
    rng = np.random.default_rng(3 + qt)
    w = synth.matrix(qt, N, K, synth.stream_for(21, f"tallf{qt}"))
    wp = ih.pack_weights(qt, _dev(w), N, K)
    for M in (9, 24, 32):
        x = rng.standard_normal((M, K)).astype(np.float32)
        got = ih.gemm_q(qt, wp, _dev(x), N, K, flags=ih.GEMM_F32 | ih.GEMM_PACKED).cpu().numpy()
        err = rel_l2(got, O.gemv_f64(qt, w, x, M, N, K))
        print(f"{F.NAMES[qt]} M={M} f32 rel-L2={err:.3e}", flush=True)
        assert err <= TOL_F32, (M, err)


def test_tall_rmsnorm_and_fold(ih):
    """RMSNorm input stage at M = 64, and a deferred Q6_K down projection
    (4 K-slices) folded into the next matmul's input stage: equal bit for bit
    to accumulate-then-matmul, and to the oracle's float64 sequence."""
    import torch
    H, FF, N2, M = 512, 4096, 96, 64
    rng = np.random.default_rng(64)
    wd = synth.matrix(F.Q6_K, H, FF, synth.stream_for(3, "tall_down"))
    w2 = synth.matrix(F.Q4_K, N2, H, synth.stream_for(4, "tall_next"))
    pd, p2 = ih.pack_weights(F.Q6_K, _dev(wd), H, FF), ih.pack_weights(F.Q4_K, _dev(w2), N2, H)
    fl = ih.GEMM_HALF | ih.GEMM_PACKED
    nw = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    h = _dev(rng.standard_normal((M, FF)).astype(np.float32))
    x0 = _dev((2.0 * rng.standard_normal((M, H))).astype(np.float32))
    xr = x0.clone()
    ih.gemm_q(F.Q6_K, pd, h, H, FF, flags=fl | ih.GEMM_ACCUM, out=xr)
    yr = ih.gemm_q_ex(F.Q4_K, p2, xr, N2, H, act=ih.ACT_RMSNORM, norm_w=_dev(nw), flags=fl)
    ws = torch.empty(ih.quantized_kernels.gemm_ws_bytes(F.Q6_K, M, H, FF, fl), dtype=torch.uint8, device="cuda")
    ih.gemm_q_ex(F.Q6_K, pd, h, H, FF, flags=fl | ih.GEMM_DEFER, ws=ws)
    parts = ih.gemm_partials(F.Q6_K, M, H, FF, fl, ws)
    assert parts[1] >= 2
    xf = x0.clone()
    yf = ih.gemm_q_ex(F.Q4_K, p2, xf, N2, H, act=ih.ACT_RMSNORM, norm_w=_dev(nw), flags=fl, add=parts)
    assert torch.equal(xf, xr)
    assert torch.equal(yf, yr)
    xref = O.gemv_f64(F.Q6_K, wd, h.cpu().numpy(), M, H, FF) + x0.cpu().numpy()
    assert rel_l2(xf.cpu().numpy(), xref) <= SANITY_HALF
    n = np.stack([O.rmsnorm(r, 1e-6, nw) for r in xf.cpu().numpy()]).astype(np.float32)
    assert rel_l2(yf.cpu().numpy(), O.gemv_f64(F.Q4_K, w2, n, M, N2, H)) <= SANITY_HALF


@pytest.mark.parametrize("M", [5, 64])
def test_fold_gate_up_partials(ih, M):
    """[gate; up] deferred (K-sliced) and its partials summed by the down
    projection's SiLU-gating input stage (x absent) equal the reduce-then-
    matmul sequence bit for bit; o deferred and folded into the residual of
    the next RMSNorm input stage likewise."""
    import torch
    H, FF = 512, 1024
    rng = np.random.default_rng(70 + M)
    wgu = synth.matrix(F.Q4_K, 2 * FF, 4 * H, synth.stream_for(9, "fold_gu"))
    wd = synth.matrix(F.Q6_K, H, FF, synth.stream_for(10, "fold_down"))
    pgu, pd = ih.pack_weights(F.Q4_K, _dev(wgu), 2 * FF, 4 * H), ih.pack_weights(F.Q6_K, _dev(wd), H, FF)
    fl = (ih.GEMM_HALF if M > 16 else ih.GEMM_F32) | ih.GEMM_PACKED
    x = _dev(rng.standard_normal((M, 4 * H)).astype(np.float32))
    gu = ih.gemm_q(F.Q4_K, pgu, x, 2 * FF, 4 * H, flags=fl)
    yr = ih.gemm_q_ex(F.Q6_K, pd, gu, H, FF, act=ih.ACT_SILU_MUL, flags=fl)
    ws = torch.empty(ih.quantized_kernels.gemm_ws_bytes(F.Q4_K, M, 2 * FF, 4 * H, fl), dtype=torch.uint8,
                     device="cuda")
    ih.gemm_q_ex(F.Q4_K, pgu, x, 2 * FF, 4 * H, flags=fl | ih.GEMM_DEFER, ws=ws)
    parts = ih.gemm_partials(F.Q4_K, M, 2 * FF, 4 * H, fl, ws)
    yf = ih.gemm_q_ex(F.Q6_K, pd, None, H, FF, act=ih.ACT_SILU_MUL, flags=fl, add=parts, m=M, ldx=2 * FF)
    assert torch.equal(yf, yr)
    g, u = gu[:, :FF].double().cpu().numpy(), gu[:, FF:].double().cpu().numpy()
    with np.errstate(over="ignore"):
        h = (g / (1.0 + np.exp(-g)) * u).astype(np.float32)
    assert rel_l2(yf.cpu().numpy(), O.gemv_f64(F.Q6_K, wd, h, M, H, FF)) <= (SANITY_HALF if M > 16 else TOL_F32)


@pytest.mark.parametrize("qt", [F.Q4_K, F.Q6_K])
def test_fold_split_launch(ih, qt):
    """fp32-accurate M = 40 runs as two launches (32 + 8 tokens); slices given
    directly: the SiLU-gating input as the sum of two [M x 2K] slices (x
    absent) and a residual fold of two [M x K] slices both equal the
    explicit sum followed by the plain call, bit for bit."""
    import torch
    N, K, M = 96, 512, 40
    w = synth.matrix(qt, N, K, synth.stream_for(40, f"split{qt}"))
    wp = ih.pack_weights(qt, _dev(w), N, K)
    fl = ih.GEMM_F32 | ih.GEMM_PACKED
    g = torch.Generator(device="cpu").manual_seed(qt)
    sl = torch.randn(2, M, 2 * K, generator=g).cuda()
    y1 = ih.gemm_q_ex(qt, wp, None, N, K, act=ih.ACT_SILU_MUL, flags=fl,
                      add=(sl.data_ptr(), 2, M * 2 * K), m=M, ldx=2 * K)
    y2 = ih.gemm_q_ex(qt, wp, (sl[0] + sl[1]).contiguous(), N, K, act=ih.ACT_SILU_MUL, flags=fl)
    assert torch.equal(y1, y2)
    sr = torch.randn(2, M, K, generator=g).cuda()
    x0 = torch.randn(M, K, generator=g).cuda()
    xa = x0.clone()
    ya = ih.gemm_q_ex(qt, wp, xa, N, K, act=ih.ACT_RMSNORM, flags=fl, add=(sr.data_ptr(), 2, M * K))
    xb = x0 + (sr[0] + sr[1])
    yb = ih.gemm_q_ex(qt, wp, xb.clone(), N, K, act=ih.ACT_RMSNORM, flags=fl)
    assert torch.equal(xa, xb)
    assert torch.equal(ya, yb)
    n = np.stack([O.rmsnorm(r, 1e-6) for r in xb.cpu().numpy()]).astype(np.float32)
    assert rel_l2(ya.cpu().numpy(), O.gemv_f64(qt, w, n, M, N, K)) <= TOL_F32


@pytest.mark.parametrize("M", [5, 24])  # one token tile (fp32-accurate), several (half)
@pytest.mark.parametrize("n_add", [1, 3, 4, 5, 8, 9, 12])
def test_fold_slice_counts(ih, M, n_add):
    """The input stage folds any number of K-slice partials in slice order:
    up to 8 slices in one round of loads (gate and up columns together for
    the SiLU-gating input up to 4), more four at a time. A residual fold of
    n_add [M x K] slices and a SiLU-gating input given only as n_add [M x 2K]
    slices both equal the explicit left-to-right sum followed by the plain
    call, bit for bit, at every count across those paths."""
    import torch
    N, K = 64, 512
    qt = F.Q4_K
    w = synth.matrix(qt, N, K, synth.stream_for(41, "foldcount"))
    wp = ih.pack_weights(qt, _dev(w), N, K)
    fl = ih.GEMM_PACKED
    g = torch.Generator(device="cpu").manual_seed(100 * M + n_add)
    sr = torch.randn(n_add, M, K, generator=g).cuda()
    x0 = torch.randn(M, K, generator=g).cuda()
    acc = sr[0].clone()
    for i in range(1, n_add):
        acc = acc + sr[i]
    xa = x0.clone()
    ya = ih.gemm_q_ex(qt, wp, xa, N, K, act=ih.ACT_RMSNORM, flags=fl, add=(sr.data_ptr(), n_add, M * K))
    xb = x0 + acc
    yb = ih.gemm_q_ex(qt, wp, xb.clone(), N, K, act=ih.ACT_RMSNORM, flags=fl)
    assert torch.equal(xa, xb)
    assert torch.equal(ya, yb)
    sl = torch.randn(n_add, M, 2 * K, generator=g).cuda()
    acc2 = sl[0].clone()
    for i in range(1, n_add):
        acc2 = acc2 + sl[i]
    y1 = ih.gemm_q_ex(qt, wp, None, N, K, act=ih.ACT_SILU_MUL, flags=fl,
                      add=(sl.data_ptr(), n_add, M * 2 * K), m=M, ldx=2 * K)
    y2 = ih.gemm_q_ex(qt, wp, acc2.contiguous(), N, K, act=ih.ACT_SILU_MUL, flags=fl)
    assert torch.equal(y1, y2)
