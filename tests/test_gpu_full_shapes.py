"""GPU parity at the BASELINE configurations' full shapes, through the
benchmark's own composition (bench.py's Model / VerifyStep / TreeStep), every
operation compared with the CPU oracle on the same seeded inputs:

* config 2: the verify batch at hidden 2048 and M = 5 ([q; k; v], o,
  [gate; up], Q6_K down, Q8_0), as bench.config2 packs and runs it;
* config 3: the Q6_K lm_head 151936 x 2048 at M = 5 (one token tile) and in
  the 30-row fp32-accurate batch of six verify steps (several token tiles);
* config 4: the 9B-class verify step at hidden 4096 (two real layers and the
  Q6_K lm_head 151936 x 4096) at M = 1, 5, 8: each matmul against the
  oracle applied to the GPU's own inputs of that operation (deferred
  products read from their K-slice partials), each residual add within fp32
  rounding, then the k = M - 1 accept on the step's logits;
* config 5: the tree step at M = 64 (half-precision MFMA operands) with Q4_K
  and with Q5_K projections, per operation, then the tree walk at T = 1.0.

Reference formulas: the GGUF dequantization of src/QuantsCPU.jl:491-658 and
the product of src/ModelCPU.jl:284-378 (oracle fp64 GEMV), RMSNorm
src/ModelCPU.jl:110-122, SiLU gating and residual adds :447-473 / :870-891,
the accept rule src/SpeculativeDecoding.jl:37-107. Bars: rel-L2 <= 1e-5 per
fp32-accurate operation, <= 1e-2 per half-precision one (north star), accept
and tree outcomes identical on the same logits."""
import numpy as np
import pytest

from _util import rel_l2

import oracle as O
from inferno_hip import formats as F

pytestmark = pytest.mark.gpu

TOL_F32, TOL_HALF = 1e-5, 1e-2
TOL_FOLD = 1e-6  # a residual add: fp32 rounding of the sum
EPS = 1e-6


@pytest.fixture(scope="module")
def ih():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import inferno_hip
    assert inferno_hip.quant_kernels_available(), inferno_hip._lib.last_error()
    return inferno_hip


@pytest.fixture(scope="module")
def bench():
    import bench as B
    return B


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _h(t):
    return t.detach().cpu().numpy()


def _rms(x, w):
    x = np.asarray(x, np.float64)
    return (x / np.sqrt((x * x).mean(axis=1, keepdims=True) + EPS) * w).astype(np.float32)


def _silu_mul(gu, ff):
    g, u = gu[:, :ff].astype(np.float64), gu[:, ff:].astype(np.float64)
    with np.errstate(over="ignore"):
        return (g / (1.0 + np.exp(-g)) * u).astype(np.float32)


def _partials(ih, qt, m, n, k, flags, ws):
    """The K-slice partials [S, m, n] a GEMM_DEFER call left in ws."""
    import torch
    ptr, ns, stride = ih.gemm_partials(qt, m, n, k, flags, ws)
    off = (ptr - ws.data_ptr()) // 4
    wf = ws.view(torch.float32)
    return _h(wf[off: off + ns * stride].view(ns, stride)[:, : m * n].reshape(ns, m, n))


def _partials_sum(ih, qt, m, n, k, flags, ws):
    """Sum (fp64) of the K-slice partials a GEMM_DEFER call left in ws."""
    return _partials(ih, qt, m, n, k, flags, ws).astype(np.float64).sum(axis=0)


def _fp32_slice_order_sum(sl):
    s = sl[0].copy()
    for j in range(1, sl.shape[0]):
        s = (s + sl[j]).astype(np.float32)
    return s


class Checker:
    def __init__(self, tol, label):
        self.tol, self.label, self.errs = tol, label, {}

    def __call__(self, name, got, ref):
        e = rel_l2(got, ref)
        self.errs[name] = max(self.errs.get(name, 0.0), e)
        assert e <= self.tol, (self.label, name, e)

    def report(self):
        print(f"{self.label} per-operation max rel-L2: " + ", ".join(f"{k} {v:.2e}" for k, v in self.errs.items()),
              flush=True)


def _run_step_with_checks(ih, B, model, step, chk, fold_chk, prec_flags):
    """Runs step.forward with a probe that checks every operation of the
    bench's composition against the oracle on the GPU's own inputs. A
    deferred product (o, down, K-sliced [gate; up]) is read from its K-slice
    partials in the workspace before the next input stage folds it, and
    checked against the oracle (chk); each fold into the fp32 residual x is
    checked separately (fold_chk: x_new against x_old + the partials' sum,
    which only fp32 rounding of the residual separates). Differences of
    residuals are never used: the synthetic weights grow the residual to
    ~1e10 within a layer, so such a difference would lose the product's
    low bits."""
    import torch
    P, M = model.proj, step.M
    H, NQ, NKV, FF, V = B.H, B.NQ, B.NKV, B.FF, B.VOCAB
    hw = model.host_gguf
    st = {}
    fl = prec_flags | ih.GEMM_PACKED
    fold_gu = ih.gemm_partials(P, M, 2 * FF, H, fl, step.ws)[1] > 1
    fold_qkv = ih.gemm_partials(P, M, NQ + 2 * NKV, H, fl, step.ws)[1] > 1

    def down_check(i):
        d = _partials_sum(ih, F.Q6_K, M, H, FF, fl, step.ws_down)
        chk("down", d, O.gemv_f64(F.Q6_K, hw[i - 1]["down"], st["h"], M, H, FF))
        return d

    def probe(tag, i):
        torch.cuda.synchronize()
        x = _h(step.x).astype(np.float64)
        if tag == "pre":
            st["x_pre"] = x
            if i > 0:
                st["down"] = down_check(i)
        elif tag == "qkv":
            if i > 0:
                fold_chk("x += down", x, st["x_pre"] + st["down"])
            wq = np.concatenate([hw[i]["q"], hw[i]["kv"]])
            # (K-sliced: still partials, which o's input stage sums and stores)
            if fold_qkv:
                st["qkv_sl"] = _partials(ih, P, M, NQ + 2 * NKV, H, fl, step.ws)
            qkv = st["qkv_sl"].astype(np.float64).sum(axis=0) if fold_qkv else _h(step.qkv)
            chk("qkv", qkv, O.gemv_f64(P, wq, _rms(x, hw[i]["attn_norm"]), M, NQ + 2 * NKV, H))
            st["x_qkv"], st["qkv"] = x, qkv
        elif tag == "o":
            if fold_qkv:  # the stored sum: the partials' fp32 sum in slice order, every column
                assert np.array_equal(_h(step.qkv), _fp32_slice_order_sum(st["qkv_sl"])), "qkv stored by o's input"
            o = _partials_sum(ih, P, M, H, NQ, fl, step.ws_o)
            chk("o", o, O.gemv_f64(P, hw[i]["o"], st["qkv"][:, :NQ], M, H, NQ))
            st["o"] = o
        elif tag == "gu":
            fold_chk("x += o", x, st["x_qkv"] + st["o"])
            gu = _partials_sum(ih, P, M, 2 * FF, H, fl, step.ws) if fold_gu else _h(step.gu)
            chk("gate/up", gu, O.gemv_f64(P, hw[i]["gu"], _rms(x, hw[i]["ffn_norm"]), M, 2 * FF, H))
            st["h"] = _silu_mul(gu.astype(np.float32) if not fold_gu else gu, FF)
            st["x_gu"] = x
        elif tag == "head":
            d = down_check(i)
            fold_chk("x += down", x, st["x_gu"] + d)
            chk("lm_head", _h(step.logits), O.gemv_f64(F.Q6_K, model.host_lm, _rms(x, model.host_out_norm), M, V, H))
            print(f"{chk.label}: every layer and the head checked", flush=True)

    step.forward(probe=probe)
    torch.cuda.synchronize()


def _run_chain_step_with_checks(ih, B, model, step, chk, fold_chk):
    """The chained composition (bench.ChainStep) checked operation by
    operation: [q; k; v] and the tile sums of o's operand, o's product added
    into the residual (x_new against x_old + the oracle's o within fp32 rounding of
    the residual), h = silu(gate) up from [gate; up] on the RMSNorm'd
    residual, down's K-slice partials, the folds, the head."""
    import torch
    P, M = model.proj, step.M
    H, NQ, NKV, FF, V = B.H, B.NQ, B.NKV, B.FF, B.VOCAB
    hw = model.host_gguf
    st = {}
    fl = ih.GEMM_F32 | ih.GEMM_PACKED

    def down_check(i):
        d = _partials_sum(ih, F.Q6_K, M, H, FF, fl, step.ws_down)
        chk("down", d, O.gemv_f64(F.Q6_K, hw[i - 1]["down"], st["h"], M, H, FF))
        return d

    def probe(tag, i):
        torch.cuda.synchronize()
        x = _h(step.x).astype(np.float64)
        if tag == "pre":
            st["x_pre"] = x
            if i > 0:
                st["down"] = down_check(i)
        elif tag == "qkv":
            if i > 0:
                fold_chk("x += down", x, st["x_pre"] + st["down"])
            wq = np.concatenate([hw[i]["q"], hw[i]["kv"]])
            qkv = _h(step.qkv)
            chk("qkv", qkv, O.gemv_f64(P, wq, _rms(x, hw[i]["attn_norm"]), M, NQ + 2 * NKV, H))
            a = qkv[:, :NQ].astype(np.float64).reshape(M, NQ // 16, 16)
            bound = 16 * 2.0 ** -23 * np.abs(a).sum(axis=2) + 1e-30  # fp32 sums in any order
            assert np.all(np.abs(_h(step.ts_q)[:M, :NQ // 16] - a.sum(axis=2)) <= bound)
            st["x_qkv"], st["qkv"] = x, qkv
        elif tag == "o":
            fold_chk("x += o", x, st["x_qkv"] + O.gemv_f64(P, hw[i]["o"], st["qkv"][:, :NQ], M, H, NQ))
            st["x_o"] = x
        elif tag == "gu":
            g = O.gemv_f64(P, hw[i]["gu"], _rms(st["x_o"], hw[i]["ffn_norm"]), M, 2 * FF, H)
            with np.errstate(over="ignore"):
                h_ref = g[:, :FF] / (1.0 + np.exp(-g[:, :FF])) * g[:, FF:]
            st["h"] = _h(step.h)
            chk("h = silu(gate) up", st["h"], h_ref)
            st["x_gu"] = x
        elif tag == "head":
            d = down_check(i)
            fold_chk("x += down", x, st["x_gu"] + d)
            chk("lm_head", _h(step.logits), O.gemv_f64(F.Q6_K, model.host_lm, _rms(x, model.host_out_norm), M, V, H))
            print(f"{chk.label}: every layer and the head checked", flush=True)

    step.forward(probe=probe)
    torch.cuda.synchronize()
    # replayed: the same bits
    logits = step.logits.clone()
    step.forward()
    torch.cuda.synchronize()
    assert torch.equal(step.logits, logits)


@pytest.mark.parametrize("M", [1, 2, 4, 5, 8])  # the token counts of configs[3]
def test_config4_chained_step(ih, bench, M):
    """configs[3] through the chained composition the benchmark times
    (bench.ChainStep: one input stage per layer), two real layers and the
    151936 x 4096 head, every operation checked, then the accept on the
    step's logits against the oracle's."""
    import torch
    B = bench
    model = B.Model(ih, 2, keep_gguf=2, gated=True)
    k = max(M - 1, 1)
    step = B.ChainStep(ih, model, M, k, 0.8)
    chk = Checker(TOL_F32, f"config 4 chained (M = {M})")
    fold = Checker(TOL_FOLD, f"config 4 chained (M = {M}) residual folds")
    _run_chain_step_with_checks(ih, B, model, step, chk, fold)
    chk.report()
    fold.report()
    if M == 1:
        return
    step.accept()
    torch.cuda.synchronize()
    rt, rn = O.spec_accept(_h(step.logits), _h(step.drf), _h(step.draft)[0], 0.8, _h(step.u_acc)[0],
                           float(_h(step.u_res)[0]), float(_h(step.u_bonus)[0]), 0)
    n = int(step.out_n[0])
    assert n == rn and _h(step.out_tok)[0, : n + 1].tolist() == rt.tolist(), (n, rn)


# ----------------------------------------------------------------- config 2

def test_config2_verify_batch(ih):
    """the eight matrices at M = 5, hidden 2048, packed and
    called as bench.config2 calls them (the matrices that share an input as
    one packed matrix), fp32-accurate."""
    import torch
    q = ih.quantized_kernels
    st = ih.synth.stream_for
    M, Hd, Fd = 5, 2048, 6144
    mats = [("q", F.Q4_K, Hd, Hd), ("k", F.Q4_K, 512, Hd), ("v", F.Q4_K, 512, Hd), ("o", F.Q4_K, Hd, Hd),
            ("gate", F.Q4_K, Fd, Hd), ("up", F.Q4_K, Fd, Hd), ("down", F.Q6_K, Hd, Fd), ("q8", F.Q8_0, Hd, Hd)]
    g = {name: q.synth_blocks(qt, st(0x1F3E0002, f"full.c2.{name}"), n * k // F.BLOCK_ELEMS[qt])
         for name, qt, n, k in mats}
    host = {name: _h(t) for name, t in g.items()}
    P = {name: ih.pack_weights(qt, g[name], n, k) for name, qt, n, k in mats}
    W = {"qkv": torch.cat([P["q"], P["k"], P["v"]]), "o": P["o"], "gu": torch.cat([P["gate"], P["up"]]),
         "down": P["down"], "q8": P["q8"]}
    hostW = {"qkv": np.concatenate([host["q"], host["k"], host["v"]]), "o": host["o"],
             "gu": np.concatenate([host["gate"], host["up"]]), "down": host["down"], "q8": host["q8"]}
    calls = [("qkv", F.Q4_K, Hd + 1024, Hd), ("o", F.Q4_K, Hd, Hd), ("gu", F.Q4_K, 2 * Fd, Hd),
             ("down", F.Q6_K, Hd, Fd), ("q8", F.Q8_0, Hd, Hd)]
    x = q.synth_gaussian(st(0x1F3E0002, "full.c2.x"), M * Hd).view(M, Hd)
    xf = q.synth_gaussian(st(0x1F3E0002, "full.c2.xf"), M * Fd).view(M, Fd)
    fl = ih.GEMM_F32 | ih.GEMM_PACKED
    chk = Checker(TOL_F32, "config 2 (M = 5)")
    for name, qt, n, k in calls:
        xi = xf if name == "down" else x
        y = ih.gemm_q_ex(qt, W[name], xi, n, k, flags=fl)
        ref = O.gemv_f64(qt, hostW[name], _h(xi), M, n, k)
        chk(f"{name} {n}x{k}", _h(y), ref)
        # the GGUF-layout weights give the same bits as the packed ones
        if name in ("down", "q8", "o"):
            y2 = ih.gemm_q_ex(qt, g[name], xi, n, k, flags=ih.GEMM_F32)
            assert torch.equal(y, y2), name
    chk.report()


# ----------------------------------------------------------------- config 3

def test_config3_lm_head_shapes(ih):
    """configs[2]'s Q6_K lm_head 151936 x 2048: one verify step (M = 5, one
    token tile) and six steps in one 30-row call (fp32-accurate, several
    token tiles), as bench.config3 batches them."""
    q = ih.quantized_kernels
    st = ih.synth.stream_for
    V, Hd = 151936, 2048
    g = q.synth_blocks(F.Q6_K, st(0x1F3E0003, "full.c3.lm"), V * Hd // 256)
    hw = _h(g)
    lm = ih.pack_weights(F.Q6_K, g, V, Hd)
    chk = Checker(TOL_F32, "config 3 lm_head 151936x2048")
    for M in (5, 30):
        x = q.synth_gaussian(st(0x1F3E0003, f"full.c3.h{M}"), M * Hd).view(M, Hd)
        y = ih.gemm_q_ex(F.Q6_K, lm, x, V, Hd, flags=ih.GEMM_F32 | ih.GEMM_PACKED)
        chk(f"M={M}", _h(y), O.gemv_f64(F.Q6_K, hw, _h(x), M, V, Hd))
    chk.report()


# ----------------------------------------------------------------- config 4

@pytest.mark.parametrize("M", [1, 2, 4, 5, 8])  # the token counts of configs[3]
def test_config4_verify_step(ih, bench, M):
    """configs[3] at hidden 4096 with two real layers and the 151936 x 4096
    Q6_K head, composed by bench.VerifyStep (fp32-accurate), every operation
    checked; then the accept of the k = M - 1 drafts on the step's logits
    (the bench's own draws, and 64 more draws per mode against the batched
    oracle)."""
    import torch
    B = bench
    model = B.Model(ih, 2, keep_gguf=2)
    k = max(M - 1, 1)
    step = B.VerifyStep(ih, model, M, k, 0.8)
    chk = Checker(TOL_F32, f"config 4 (M = {M})")
    fold = Checker(TOL_FOLD, f"config 4 (M = {M}) residual folds")
    _run_step_with_checks(ih, B, model, step, chk, fold, ih.GEMM_F32)
    chk.report()
    fold.report()
    if M == 1:
        return
    Lt = _h(step.logits)
    Ld = _h(step.drf)
    step.accept()
    torch.cuda.synchronize()
    rt, rn = O.spec_accept(Lt, Ld, _h(step.draft)[0], 0.8, _h(step.u_acc)[0], float(_h(step.u_res)[0]),
                           float(_h(step.u_bonus)[0]), 0)
    n = int(step.out_n[0])
    assert n == rn and _h(step.out_tok)[0, : n + 1].tolist() == rt.tolist(), (n, rn)
    S = 64
    rng = np.random.default_rng(40 + M)
    z = Ld.astype(np.float64) / 0.8
    pz = np.exp(z - z.max(axis=1, keepdims=True))
    pz /= pz.sum(axis=1, keepdims=True)
    draft = np.stack([[rng.choice(B.VOCAB, p=pz[i]) for i in range(k)] for _ in range(S)]).astype(np.int32)
    ua = rng.random((S, k)).astype(np.float32)
    ur, ub = rng.random(S).astype(np.float32), rng.random(S).astype(np.float32)
    tgt = step.logits.unsqueeze(0).expand(S, M, B.VOCAB).contiguous()
    drf = step.drf.unsqueeze(0).expand(S, k, B.VOCAB).contiguous()
    for mode in (0, 1):
        tok, nn = ih.spec_accept(tgt, drf, _dev(draft), 0.8, _dev(ua), _dev(ur), _dev(ub), mode=mode)
        tok, nn = _h(tok), _h(nn)
        rtok, rnn = O.spec_accept_batch(np.broadcast_to(Lt, (S, M, B.VOCAB)), np.broadcast_to(Ld, (S, k, B.VOCAB)),
                                        draft, 0.8, ua, ur, ub, mode)
        assert np.array_equal(nn, rnn), (mode, nn, rnn)
        for s in range(S):
            nt = O.n_tokens(int(rnn[s]), k, mode)
            assert tok[s, :nt].tolist() == rtok[s, :nt].tolist(), (mode, s)
        print(f"config 4 (M = {M}) accept mode {mode}: lengths {np.bincount(nn, minlength=k + 1).tolist()}",
              flush=True)


# ----------------------------------------------------------------- config 5

@pytest.mark.parametrize("proj", ["Q4_K", "Q5_K"])
def test_config5_tree_step(ih, bench, proj):
    """the 64-node tree step at hidden 4096 (two real layers,
    the 151936 x 4096 Q6_K head) on the half-precision MFMA path with the
    projections in `proj`, composed by bench.TreeStep: every operation
    within 1e-2 (and near the fp16 rounding, <= 2e-3), then the tree walk at
    T = 1.0 identical to the oracle's on the GPU logits."""
    import torch
    B = bench
    model = B.Model(ih, 2, keep_gguf=2, proj=proj)
    step = B.TreeStep(ih, model)
    chk = Checker(TOL_HALF, f"config 5 (M = 64, {proj})")
    fold = Checker(TOL_FOLD, f"config 5 ({proj}) residual folds")
    _run_step_with_checks(ih, B, model, step, chk, fold, 0)
    chk.report()
    fold.report()
    assert max(chk.errs.values()) <= 2e-3, chk.errs
    step.accept()
    torch.cuda.synchronize()
    Lt, Ld = _h(step.logits), _h(step.drf_t)
    tok, par, u = _h(step.tok), _h(step.parent), _h(step.u)
    want = O.tree_accept(Lt, Ld, tok, par, 1.0, u)
    got = _h(step.path)[: int(step.plen[0])]
    assert got.tolist() == list(want), (got, want)
    lens = [len(want)]
    rng = np.random.default_rng(5)
    for _ in range(6):  # more uniform draws on the same tree
        u2 = rng.random(64).astype(np.float32)
        g2 = _h(ih.tree_accept(step.logits, step.drf_t, step.tok, step.parent, 1.0, _dev(u2)))
        w2 = O.tree_accept(Lt, Ld, tok, par, 1.0, u2)
        assert g2.tolist() == list(w2)
        lens.append(len(w2))
    print(f"config 5 ({proj}) tree path lengths: {lens}", flush=True)
