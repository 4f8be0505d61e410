"""GPU: chained fp32-accurate matmuls (ihip_gemm_q_chain), the layer
composition without per-matmul input stages: a producer's epilogue writes
its fp32 output and the next matmul's split-fp16 operand at per-tile powers
of two (with tile sums and sums of squares); the consumer rescales that
operand per 256-element unit in registers.

Pinned three ways: (1) every product against the oracle's fp64 GEMV of the
dequantized weights on the GPU's own inputs (rel-L2 <= 1e-5, the north-star
bar); (2) a chained consumer's output against the classic call (input stage
+ matmul) on the same fp32 rows, to 1e-6: the rescaled limbs are the input
stage's wherever they stay normal fp16, so only sub-2^-24 parts of a unit's
scale and the order of the min-term sums differ; (3) the tile sums and sums
of squares against numpy over the GPU's outputs. A dynamic-range case spreads
the producer's tiles over 2^0 .. 2^-30 of a unit's largest value (exact,
subnormal and flushed rescales) and includes all-zero tiles and units. Layer
arithmetic: RMSNorm src/ModelCPU.jl:110-122, SiLU gating :447-473, residual
adds :870-891."""
import numpy as np
import pytest

from _util import rel_l2

import oracle as O
from inferno_hip import formats as F
from inferno_hip import synth

pytestmark = pytest.mark.gpu
EPS = 1e-6
FL = 1 | 8  # GEMM_F32 | GEMM_PACKED


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


def _h(t):
    return t.detach().cpu().numpy()


def _rms(x, w):
    x = np.asarray(x, np.float64)
    return (x / np.sqrt((x * x).mean(axis=1, keepdims=True) + EPS) * w).astype(np.float32)


def _sums_ok(got, v, M, tiles, rows=16):
    """Tile sums of v (fp32, any order) within the fp32 summation bound:
    n eps times the sum of the magnitudes (cancelling tiles need no more)."""
    a = v[:M, :tiles * rows].astype(np.float64).reshape(M, tiles, rows)
    bound = rows * 2.0 ** -23 * np.abs(a).sum(axis=2) + 1e-30
    return bool(np.all(np.abs(got[:M, :tiles] - a.sum(axis=2)) <= bound))


@pytest.mark.parametrize("qt2", F.QTYPES)
@pytest.mark.parametrize("M", [1, 5, 8])
def test_stats_producer_feeds_plain_consumer(ih, M, qt2):
    """[q; k; v]-shaped producer (RMSNorm input stage; operand and statistics
    of its first S rows) -> o-shaped consumer in each operand layout (Q4_K /
    Q5_K with the min-term operand, Q6_K, Q8_0)."""
    import torch
    N1, K1, S, N2 = 768, 1024, 512, 256
    w1 = synth.matrix(F.Q4_K, N1, K1, synth.stream_for(1, "ch.w1"))
    w2 = synth.matrix(qt2, N2, S, synth.stream_for(2, f"ch.w2.{qt2}"))
    p1, p2 = ih.pack_weights(F.Q4_K, _dev(w1), N1, K1), ih.pack_weights(qt2, _dev(w2), N2, S)
    rng = np.random.default_rng(M)
    x = (2.0 * rng.standard_normal((M, K1))).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(K1)).astype(np.float32)
    y1 = torch.zeros((M, N1), device="cuda")
    op, ts, _ = ih.chain_buffers(S)
    ih.gemm_q_chain(F.Q4_K, p1, N1, K1, M, x=_dev(x), act=ih.ACT_RMSNORM, norm_w=_dev(nw),
                    cout=ih.chain_out(ih.EPI_STATS, y1, qt2, op, ts, stat_rows=S))
    y2 = torch.zeros((M, N2), device="cuda")
    ih.gemm_q_chain(qt2, p2, N2, S, M, cin=ih.chain_in(op, ts, 16), cout=ih.chain_out(ih.EPI_STORE, y2))
    torch.cuda.synchronize()
    g1, g2 = _h(y1), _h(y2)
    assert rel_l2(g1, O.gemv_f64(F.Q4_K, w1, _rms(x, nw), M, N1, K1)) <= 1e-5
    assert rel_l2(g2, O.gemv_f64(qt2, w2, g1[:, :S], M, N2, S)) <= 1e-5
    assert _sums_ok(_h(ts), g1, M, S // 16)
    classic = ih.gemm_q_ex(qt2, p2, y1[:, :S], N2, S, flags=FL)
    assert rel_l2(g2, _h(classic)) <= 1e-6, (M, qt2)


@pytest.mark.parametrize("qd", F.QTYPES)
@pytest.mark.parametrize("M", [1, 5, 8])
def test_resid_gate_defer_chain(ih, M, qd):
    """o-shaped producer adding into the residual (operand of x w, tile sums
    of squares) -> [gate; up] consumer with RMSNorm from those statistics,
    producing h = silu(gate) up and the down operand in 8-channel tiles ->
    down-shaped consumer of h (each operand layout) left as K-slice partials:
    the MLP half of a layer with one input stage in total."""
    import torch
    q = ih.quantized_kernels
    H, NQ, FF = 512, 256, 1024
    wo = synth.matrix(F.Q4_K, H, NQ, synth.stream_for(3, "ch.o"))
    wgu = synth.matrix(F.Q4_K, 2 * FF, H, synth.stream_for(4, "ch.gu"))
    wd = synth.matrix(qd, H, FF, synth.stream_for(5, f"ch.down.{qd}"))
    po = ih.pack_weights(F.Q4_K, _dev(wo), H, NQ)
    pg = ih.pack_weights_gated(F.Q4_K, _dev(wgu), FF, H)
    pg_plain = ih.pack_weights(F.Q4_K, _dev(wgu), 2 * FF, H)
    pd = ih.pack_weights(qd, _dev(wd), H, FF)
    rng = np.random.default_rng(10 + M)
    qin = (3.0 * rng.standard_normal((M, NQ))).astype(np.float32)
    x0 = rng.standard_normal((M, H)).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    x = _dev(x0)
    op_x, ts_x, ssq_x = ih.chain_buffers(H, ssq=True)
    ih.gemm_q_chain(F.Q4_K, po, H, NQ, M, x=_dev(qin),
                    cout=ih.chain_out(ih.EPI_RESID, x, F.Q4_K, op_x, ts_x, norm_w=_dev(nw), tile_ssq=ssq_x))
    torch.cuda.synchronize()
    xn = _h(x)
    o_ref = O.gemv_f64(F.Q4_K, wo, qin, M, H, NQ)
    assert rel_l2(xn, x0.astype(np.float64) + o_ref) <= 1e-6
    assert _sums_ok(_h(ts_x), xn * nw, M, H // 16)
    sq = (xn.astype(np.float64) ** 2).reshape(M, H // 16, 16).sum(axis=2).T
    assert np.allclose(_h(ssq_x)[:, :M], sq, rtol=1e-6, atol=0)
    # [gate; up] from the chained residual: RMSNorm row scale from the tile sums of squares
    h = torch.zeros((M, FF), device="cuda")
    op_h, ts_h, _ = ih.chain_buffers(FF, tiles_per_unit=32)
    ih.gemm_q_chain(F.Q4_K, pg, 2 * FF, H, M, cin=ih.chain_in(op_x, ts_x, 16, tile_ssq=ssq_x, eps=EPS),
                    cout=ih.chain_out(ih.EPI_GATE, h, qd, op_h, ts_h))
    torch.cuda.synchronize()
    gh = _h(h)
    gu_ref = O.gemv_f64(F.Q4_K, wgu, _rms(xn, nw), M, 2 * FF, H)
    g, u = gu_ref[:, :FF], gu_ref[:, FF:]
    with np.errstate(over="ignore"):
        h_ref = g / (1.0 + np.exp(-g)) * u
    assert rel_l2(gh, h_ref) <= 1e-5
    assert _sums_ok(_h(ts_h), gh, M, FF // 8, rows=8)
    # the classic [gate; up] (plain packing, input stage) then SiLU gating: the same to rounding
    gu_c = ih.gemm_q_ex(F.Q4_K, pg_plain, x, 2 * FF, H, act=ih.ACT_RMSNORM, norm_w=_dev(nw), eps=EPS, flags=FL)
    assert rel_l2(gh, _h(q.silu_mul(gu_c, FF))) <= 1e-6
    # down from h's operand, deferred: partials against the oracle and the classic call on the same h
    ws = torch.empty(q.gemm_ws_bytes(qd, M, H, FF, FL), dtype=torch.uint8, device="cuda")
    ih.gemm_q_chain(qd, pd, H, FF, M, cin=ih.chain_in(op_h, ts_h, 32), flags=FL | ih.GEMM_DEFER, ws=ws)
    ptr, ns, stride = ih.gemm_partials(qd, M, H, FF, FL, ws)
    off = (ptr - ws.data_ptr()) // 4
    parts = ws.view(torch.float32)[off: off + ns * stride].view(ns, stride)[:, : M * H].reshape(ns, M, H).clone()
    ws2 = torch.empty_like(ws)
    ih.gemm_q_ex(qd, pd, h, H, FF, flags=FL | ih.GEMM_DEFER, ws=ws2)
    parts2 = ws2.view(torch.float32)[off: off + ns * stride].view(ns, stride)[:, : M * H].reshape(ns, M, H)
    d_chain = _h(parts).astype(np.float64).sum(axis=0)
    assert rel_l2(d_chain, O.gemv_f64(qd, wd, gh, M, H, FF)) <= 1e-5
    assert rel_l2(d_chain, _h(parts2).astype(np.float64).sum(axis=0)) <= 1e-6, (M, qd)


def _zero_rows(w, qt, rows, k):
    """Zero the scale fields (d, and dmin where present) of every block of the
    given rows: those rows dequantize to exactly 0."""
    w = w.copy()
    nb = k // F.BLOCK_ELEMS[qt]
    bb = F.BLOCK_BYTES[qt]
    for r in rows:
        for b in range(r * nb, (r + 1) * nb):
            if qt == F.Q6_K:
                w[b * bb + 208: b * bb + 210] = 0
            else:
                w[b * bb: b * bb + (4 if qt in (F.Q4_K, F.Q5_K) else 2)] = 0
    return w


@pytest.mark.parametrize("qt2", F.QTYPES)
def test_chain_dynamic_range(ih, qt2):
    """Residual tiles spread over 2^0 .. 2^-30 of their unit's largest value
    (the rescale exact, into fp16 subnormals, and flushed), one all-zero tile
    and one all-zero unit: the consumer against the oracle and the classic
    call."""
    import torch
    M, H, NQ, N2 = 5, 1024, 256, 128
    zero_rows = list(range(48, 64)) + list(range(512, 768))  # tile 3 of unit 0, all of unit 2
    wo = _zero_rows(synth.matrix(F.Q4_K, H, NQ, synth.stream_for(6, "dr.o")), F.Q4_K, zero_rows, NQ)
    w2 = synth.matrix(qt2, N2, H, synth.stream_for(7, f"dr.w2.{qt2}"))
    po, p2 = ih.pack_weights(F.Q4_K, _dev(wo), H, NQ), ih.pack_weights(qt2, _dev(w2), N2, H)
    rng = np.random.default_rng(20 + qt2)
    qin = (1e-3 * rng.standard_normal((M, NQ))).astype(np.float32)
    tile_mag = 2.0 ** (-2.0 * (np.arange(H // 16) % 16))  # 2^0 .. 2^-30 inside each unit
    x0 = (rng.standard_normal((M, H)) * np.repeat(tile_mag, 16)).astype(np.float32)
    x0[:, zero_rows] = 0.0
    nw = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    x = _dev(x0)
    op, ts, ssq = ih.chain_buffers(H, ssq=True)
    ih.gemm_q_chain(F.Q4_K, po, H, NQ, M, x=_dev(qin),
                    cout=ih.chain_out(ih.EPI_RESID, x, qt2, op, ts, norm_w=_dev(nw), tile_ssq=ssq))
    y = torch.zeros((M, N2), device="cuda")
    ih.gemm_q_chain(qt2, p2, N2, H, M, cin=ih.chain_in(op, ts, 16, tile_ssq=ssq, eps=EPS),
                    cout=ih.chain_out(ih.EPI_STORE, y))
    torch.cuda.synchronize()
    xn = _h(x)
    assert np.all(xn[:, zero_rows] == 0.0)
    got = _h(y)
    assert np.all(np.isfinite(got))
    assert rel_l2(got, O.gemv_f64(qt2, w2, _rms(xn, nw), M, N2, H)) <= 1e-5
    classic = ih.gemm_q_ex(qt2, p2, x, N2, H, act=ih.ACT_RMSNORM, norm_w=_dev(nw), eps=EPS, flags=FL)
    assert rel_l2(got, _h(classic)) <= 1e-6


def test_chain_argument_checks(ih):
    import torch
    L = ih.load()
    p = ih.pack_weights(F.Q4_K, _dev(synth.matrix(F.Q4_K, 256, 256, 9)), 256, 256)
    y = torch.zeros((9, 256), device="cuda")
    op, ts, _ = ih.chain_buffers(256)
    with pytest.raises(ih.HipError):  # M > 8
        ih.gemm_q_chain(F.Q4_K, p, 256, 256, 9, x=torch.zeros((9, 256), device="cuda"),
                        cout=ih.chain_out(ih.EPI_STATS, y, F.Q4_K, op, ts, stat_rows=256))
    with pytest.raises(ih.HipError):  # stat_rows not a multiple of 256
        ih.gemm_q_chain(F.Q4_K, p, 256, 256, 5, x=torch.zeros((5, 256), device="cuda"),
                        cout=ih.chain_out(ih.EPI_STATS, y, F.Q4_K, op, ts, stat_rows=128))
    with pytest.raises(ih.HipError):  # a Q4_K consumer needs the tile sums (min terms)
        ih.gemm_q_chain(F.Q4_K, p, 256, 256, 5, cin=ih.chain_in(op, None, 16), cout=ih.chain_out(ih.EPI_STORE, y))
    with pytest.raises(ih.HipError):  # unknown consumer layout
        ih.gemm_q_chain(F.Q4_K, p, 256, 256, 5, x=torch.zeros((5, 256), device="cuda"),
                        cout=ih.chain_out(ih.EPI_STATS, y, 99, op, ts, stat_rows=256))
    # buffers smaller than the call shape: the wrapper refuses before the C ABI
    x5 = torch.zeros((5, 256), device="cuda")
    with pytest.raises(ValueError, match="x must be"):
        ih.gemm_q_chain(F.Q4_K, p, 256, 256, 5, x=x5[:, :128], cout=ih.chain_out(ih.EPI_STORE, y))
    with pytest.raises(ValueError, match="cout y"):
        ih.gemm_q_chain(F.Q4_K, p, 256, 256, 5, x=x5, cout=ih.chain_out(ih.EPI_STORE, y[:5, :128]))
    with pytest.raises(ValueError, match="cin operand"):
        ih.gemm_q_chain(F.Q4_K, p, 256, 256, 5, cin=ih.chain_in(op[:64], ts, 16), cout=ih.chain_out(ih.EPI_STORE, y))
    with pytest.raises(ValueError, match="cin tile_sum"):
        ih.gemm_q_chain(F.Q4_K, p, 256, 256, 5, cin=ih.chain_in(op, ts[:, :4].contiguous(), 16),
                        cout=ih.chain_out(ih.EPI_STORE, y))
    with pytest.raises(ValueError, match="cout tile_ssq"):
        ih.gemm_q_chain(F.Q4_K, p, 256, 256, 5, x=x5,
                        cout=ih.chain_out(ih.EPI_STATS, y, F.Q4_K, op, ts, tile_ssq=torch.zeros(8, device="cuda"),
                                          stat_rows=256))
    with pytest.raises(ValueError, match="cout norm_w"):
        ih.gemm_q_chain(F.Q4_K, p, 256, 256, 5, x=x5,
                        cout=ih.chain_out(ih.EPI_STATS, y, F.Q4_K, op, ts, norm_w=torch.ones(128, device="cuda"),
                                          stat_rows=256))
    assert L.ihip_pack_weights_gated(F.Q4_K, p.data_ptr(), p.data_ptr(), 12, 256, None) == -22  # F % 8
    assert ih.chain_operand_bytes(4096) == 16 * (8192 + 1024)


@pytest.mark.parametrize("qt2", F.QTYPES)
@pytest.mark.parametrize("M", [3, 8])
def test_chain_ragged_rows(ih, M, qt2):
    """Row counts that end inside a 16-row tile and tile counts that do not
    divide over the workgroups: a STATS producer of 1000 rows (operand of
    its first 768) feeding consumers of 1000 and 200 rows (the last
    workgroups hold fewer tiles, the last tile 8 rows), against the oracle
    and the classic call on the same rows."""
    import torch
    N1, K1, S = 1000, 512, 768
    w1 = synth.matrix(F.Q4_K, N1, K1, synth.stream_for(6, "ch.rag1"))
    p1 = ih.pack_weights(F.Q4_K, _dev(w1), N1, K1)
    rng = np.random.default_rng(40 + M)
    x = rng.standard_normal((M, K1)).astype(np.float32)
    y1 = torch.zeros((M, N1), device="cuda")
    op, ts, _ = ih.chain_buffers(S)
    ih.gemm_q_chain(F.Q4_K, p1, N1, K1, M, x=_dev(x), cout=ih.chain_out(ih.EPI_STATS, y1, qt2, op, ts, stat_rows=S))
    torch.cuda.synchronize()
    g1 = _h(y1)
    assert rel_l2(g1, O.gemv_f64(F.Q4_K, w1, x, M, N1, K1)) <= 1e-5
    assert _sums_ok(_h(ts), g1, M, S // 16)
    for N2 in (1000, 200):
        w2 = synth.matrix(qt2, N2, S, synth.stream_for(7, f"ch.rag2.{qt2}.{N2}"))
        p2 = ih.pack_weights(qt2, _dev(w2), N2, S)
        y2 = torch.full((M, N2 + 8), 7.0, device="cuda")  # 8 columns past N2 must stay untouched
        ih.gemm_q_chain(qt2, p2, N2, S, M, cin=ih.chain_in(op, ts, 16),
                        cout=ih.chain_out(ih.EPI_STORE, y2[:, :N2]))
        torch.cuda.synchronize()
        g2 = _h(y2)
        assert np.all(g2[:, N2:] == 7.0), (M, qt2, N2)
        assert rel_l2(g2[:, :N2], O.gemv_f64(qt2, w2, g1[:, :S], M, N2, S)) <= 1e-5, (M, qt2, N2)
        classic = ih.gemm_q_ex(qt2, p2, y1[:, :S], N2, S, flags=FL)
        assert rel_l2(g2[:, :N2], _h(classic)) <= 1e-6, (M, qt2, N2)


@pytest.mark.parametrize("qt", [F.Q4_K, F.Q5_K])
@pytest.mark.parametrize("M,N", [(3, 4096 + 2048), (8, 4096 + 1000)])
def test_large_statistics_producer(ih, qt, M, N):
    """[q; k; v]-shaped statistics producers with more tiles than CUs (256
    statistics tiles and a tail of 128 or 63, the last one ragged; the
    output starts as NaN, so every row must be written): every row against
    the oracle and the classic call, the operand through an o-shaped
    consumer."""
    import torch
    K, S = 4096, 4096
    w = synth.matrix(qt, N, K, synth.stream_for(8, f"ch.split.{qt}.{N}"))
    p = ih.pack_weights(qt, _dev(w), N, K)
    rng = np.random.default_rng(60 + M)
    x = rng.standard_normal((M, K)).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    y = torch.full((M, N), float("nan"), device="cuda")
    op, ts, _ = ih.chain_buffers(S)
    ih.gemm_q_chain(qt, p, N, K, M, x=_dev(x), act=ih.ACT_RMSNORM, norm_w=_dev(nw), eps=EPS,
                    cout=ih.chain_out(ih.EPI_STATS, y, F.Q4_K, op, ts, stat_rows=S))
    torch.cuda.synchronize()
    gy = _h(y)
    assert np.all(np.isfinite(gy))
    ref = O.gemv_f64(qt, w, _rms(x, nw), M, N, K)
    assert rel_l2(gy, ref) <= 1e-5, (qt, M, N)
    assert rel_l2(gy[:, S:], ref[:, S:]) <= 1e-5, (qt, M, N)  # the split tail alone
    classic = ih.gemm_q_ex(qt, p, _dev(x), N, K, act=ih.ACT_RMSNORM, norm_w=_dev(nw), eps=EPS, flags=FL)
    assert rel_l2(gy, _h(classic)) <= 1e-6, (qt, M, N)
    assert _sums_ok(_h(ts), gy, M, S // 16)
    wo = synth.matrix(F.Q4_K, 512, S, synth.stream_for(9, "ch.split.o"))
    po = ih.pack_weights(F.Q4_K, _dev(wo), 512, S)
    yo = torch.zeros((M, 512), device="cuda")
    ih.gemm_q_chain(F.Q4_K, po, 512, S, M, cin=ih.chain_in(op, ts, 16), cout=ih.chain_out(ih.EPI_STORE, yo))
    torch.cuda.synchronize()
    assert rel_l2(_h(yo), O.gemv_f64(F.Q4_K, wo, gy[:, :S], M, 512, S)) <= 1e-5


@pytest.mark.parametrize("qt,N,K", [(F.Q6_K, 512, 6144), (F.Q6_K, 256, 12288), (F.Q4_K, 256, 12288)])
@pytest.mark.parametrize("M", [1, 5, 8])
def test_ksplit_chained_epilogue(ih, M, qt, N, K):
    """A chained producer split over K (2, 4 or 3 K-slices: the down
    projection's plan): each tile's slices are summed in slice order by the
    last slice to arrive, which runs the epilogue. EPI_RESID into the
    residual with the operand of x w for a Q4_K and a Q6_K consumer (the next
    [q; k; v], the head) and its tile sums of squares: x_new against x_old +
    the oracle's product (fp32 rounding of the residual), the statistics
    against numpy, each consumer against the classic call (input stage with
    the RMSNorm) on the same rows; EPI_STATS likewise. Two calls in a row
    give the same bits (the per-tile counts are zero again after each)."""
    import torch
    q = ih.quantized_kernels
    w = synth.matrix(qt, N, K, synth.stream_for(21, f"ks.{qt}.{N}.{K}"))
    pw = ih.pack_weights(qt, _dev(w), N, K)
    rng = np.random.default_rng(7 * M + K)
    xin = (2.0 * rng.standard_normal((M, K))).astype(np.float32)
    r0 = rng.standard_normal((M, N)).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(N)).astype(np.float32)
    ref = O.gemv_f64(qt, w, xin, M, N, K)
    ws = torch.zeros(q.gemm_ws_bytes(qt, M, N, K, FL), dtype=torch.uint8, device="cuda")
    outs = []
    for rep in range(2):
        x = _dev(r0)
        op, ts, ssq = ih.chain_buffers(N, ssq=True)
        ih.gemm_q_chain(qt, pw, N, K, M, x=_dev(xin), ws=ws,
                        cout=ih.chain_out(ih.EPI_RESID, x, F.Q4_K, op, ts, norm_w=_dev(nw), tile_ssq=ssq))
        torch.cuda.synchronize()
        outs.append((_h(x), _h(op), _h(ts), _h(ssq)))
    assert all(np.array_equal(a, b) for a, b in zip(outs[0], outs[1]))
    xn, _, tsn, ssqn = outs[0]
    assert rel_l2(xn, r0.astype(np.float64) + ref) <= 1e-6
    assert _sums_ok(tsn, xn * nw, M, N // 16)
    sq = (xn.astype(np.float64) ** 2).reshape(M, N // 16, 16).sum(axis=2).T
    assert np.allclose(ssqn[:, :M], sq, rtol=1e-6, atol=0)
    # consumers of the chained residual (RMSNorm row scale from the tile sums of squares)
    x = _dev(xn)
    for cq in (F.Q4_K, F.Q6_K):
        wc = synth.matrix(cq, 512, N, synth.stream_for(22, f"ks.c{cq}.{N}"))
        pc = ih.pack_weights(cq, _dev(wc), 512, N)
        op, ts, ssq = ih.chain_buffers(N, ssq=True)
        x2 = _dev(r0)
        ih.gemm_q_chain(qt, pw, N, K, M, x=_dev(xin), ws=ws,
                        cout=ih.chain_out(ih.EPI_RESID, x2, cq, op, ts if cq == F.Q4_K else None, norm_w=_dev(nw),
                                          tile_ssq=ssq))
        y = torch.zeros((M, 512), device="cuda")
        ih.gemm_q_chain(cq, pc, 512, N, M, cin=ih.chain_in(op, ts if cq == F.Q4_K else None, 16, tile_ssq=ssq, eps=EPS),
                        cout=ih.chain_out(ih.EPI_STORE, y))
        yc = ih.gemm_q_ex(cq, pc, x, 512, N, act=ih.ACT_RMSNORM, norm_w=_dev(nw), eps=EPS, flags=FL)
        torch.cuda.synchronize()
        assert rel_l2(_h(y), _h(yc)) <= 1e-6, cq
        assert rel_l2(_h(y), O.gemv_f64(cq, wc, _rms(xn, nw), M, 512, N)) <= 1e-5, cq
    # EPI_STATS on the K-split matmul: the product and the operand of all its rows
    y = torch.zeros((M, N), device="cuda")
    op, ts, _ = ih.chain_buffers(N)
    ih.gemm_q_chain(qt, pw, N, K, M, x=_dev(xin), ws=ws,
                    cout=ih.chain_out(ih.EPI_STATS, y, F.Q4_K, op, ts, stat_rows=N))
    torch.cuda.synchronize()
    assert rel_l2(_h(y), ref) <= 1e-5
    assert _sums_ok(_h(ts), _h(y), M, N // 16)
