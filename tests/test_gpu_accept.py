"""GPU parity of the LM-head softmax statistics, rejection-sampling accept,
greedy verify and tree accept against the CPU oracle, with the same explicit
uniforms. Bars: accepted lengths identical on >= 99.9 % of steps, greedy
argmax identical (first index on ties), tree paths identical."""
import numpy as np
import pytest

from _util import rel_l2

import oracle as O
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


def _case(rng, S, k, V, noise=1.5, scale=3.0):
    Lt = (rng.standard_normal((S, k + 1, V)) * scale).astype(np.float32)
    Ld = (Lt[:, :k, :] + rng.standard_normal((S, k, V)) * noise).astype(np.float32)
    return Lt, Ld


def _draw(L, T, u):
    """Draft token ~ softmax(L/T) by inverse CDF in fp64 (test-side sampler)."""
    z = L.astype(np.float64) / T
    p = np.exp(z - z.max())
    c = np.cumsum(p)
    return int(min(np.searchsorted(c, u * c[-1]), L.size - 1))


def test_softmax_stats(ih):
    rng = np.random.default_rng(0)
    L = (rng.standard_normal((7, 151936)) * 4).astype(np.float32)
    L[3, :] = -2.0   # uniform row
    L[4, 17] = 80.0  # one dominant entry
    for T in (1.0, 0.8):
        zm, zs = ih.softmax_stats(_dev(L), T)
        zm, zs = zm.cpu().numpy(), zs.cpu().numpy()
        for r in range(L.shape[0]):
            m, s = O.softmax_stats(L[r], T)
            assert abs(zm[r] - m) <= 1e-6 * max(1.0, abs(m))
            assert abs(zs[r] - s) <= 2e-5 * s, (r, zs[r], s)


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("V,S,T", [(16, 2000, 0.8), (1000, 500, 1.0), (151936, 48, 0.8)])
def test_spec_accept_parity(ih, mode, V, S, T):
    k = 4
    rng = np.random.default_rng(V + S + mode)
    Lt, Ld = _case(rng, S, k, V, scale=3.0 if V > 100 else 1.0)
    ud = rng.random((S, k))
    draft = np.array([[_draw(Ld[s, i], T, ud[s, i]) for i in range(k)] for s in range(S)], dtype=np.int32)
    u_acc = rng.random((S, k)).astype(np.float32)
    u_res = rng.random(S).astype(np.float32)
    u_bon = rng.random(S).astype(np.float32)
    tok, n = ih.spec_accept(_dev(Lt), _dev(Ld), _dev(draft), T, _dev(u_acc), _dev(u_res), _dev(u_bon), mode=mode)
    tok, n = tok.cpu().numpy(), n.cpu().numpy()
    same_len = same_tok = 0
    for s in range(S):
        rt, rn = O.spec_accept(Lt[s], Ld[s], draft[s], T, u_acc[s], float(u_res[s]), float(u_bon[s]), mode)
        same_len += int(rn == n[s])
        same_tok += int(rn == n[s] and np.array_equal(rt, tok[s, : ih.n_tokens(int(n[s]), k, mode)]))
    print(f"mode={mode} V={V} S={S}: lengths {same_len}/{S}, tokens {same_tok}/{S}", flush=True)
    assert same_len >= 0.999 * S
    assert same_tok >= 0.999 * S


def test_spec_accept_special_cases(ih):
    V, k = 64, 4
    rng = np.random.default_rng(5)
    L = rng.standard_normal((1, k + 1, V)).astype(np.float32)
    draft = np.array([[3, 9, 27, 50]], dtype=np.int32)
    ones = np.full((1, k), 0.999, dtype=np.float32)
    u = np.array([0.5], dtype=np.float32)
    # q == p: every draft accepted whatever u < 1, then a bonus token
    tok, n = ih.spec_accept(_dev(L), _dev(L[:, :k].copy()), _dev(draft), 1.0, _dev(ones), _dev(u), _dev(u))
    assert int(n[0]) == k and tok[0, :k].cpu().numpy().tolist() == draft[0].tolist()
    # p[x_0] ~ 0: the first draft is rejected and the residual draw avoids x_0
    L2 = L.copy()
    L2[0, 0, 3] = -1e4
    zero = np.zeros((1, k), dtype=np.float32)
    tok, n = ih.spec_accept(_dev(L2), _dev(L[:, :k].copy()), _dev(draft), 1.0, _dev(zero), _dev(u), _dev(u))
    assert int(n[0]) == 0 and int(tok[0, 0]) != 3
    rt, rn = O.spec_accept(L2[0], L[0, :k], draft[0], 1.0, zero[0], 0.5, 0.5, 0)
    assert rn == 0 and int(rt[0]) == int(tok[0, 0])
    # k = 0: only a bonus token
    tok, n = ih.spec_accept(_dev(L[:, :1].copy()), _dev(np.zeros((1, 0, V), np.float32)),
                            _dev(np.zeros((1, 0), np.int32)), 0.7, _dev(np.zeros((1, 0), np.float32)), _dev(u),
                            _dev(u))
    rt, rn = O.spec_accept(L[0, :1], np.zeros((0, V), np.float32), np.zeros(0, np.int32), 0.7,
                           np.zeros(0, np.float32), 0.5, 0.5, 0)
    assert int(n[0]) == 0 and int(tok[0, 0]) == int(rt[0])


def test_reference_mode_bonus_after_last_rejection(ih):
    """Mode 1 reproduces src/SpeculativeDecoding.jl:100: a rejection of the
    last draft leaves length(accepted) == gamma, so a bonus token from target
    row k at T follows the residual; an earlier rejection has no bonus. The
    hand-worked two-draft case of the oracle tests at V = 3, and a batch at
    V = 151936 whose steps are forced to reject at every position."""
    Lt = np.log(np.array([[[0.5, 0.3, 0.2], [0.5, 0.3, 0.2], [0.1, 0.1, 0.8]]], np.float32)).repeat(3, 0)
    Ld = np.log(np.array([[[0.1, 0.6, 0.3], [0.1, 0.6, 0.3]]], np.float32)).repeat(3, 0)
    d = np.array([[1, 1]] * 3, np.int32)
    ua = np.array([[0.7, 0.1], [0.1, 0.7], [0.1, 0.2]], np.float32)
    ur = np.full(3, 0.5, np.float32)
    ub = np.array([0.9, 0.9, 0.15], np.float32)
    tok, n = ih.spec_accept(_dev(Lt), _dev(Ld), _dev(d), 1.0, _dev(ua), _dev(ur), _dev(ub), mode=1)
    tok, n = tok.cpu().numpy(), n.cpu().numpy()
    assert n.tolist() == [0, 1, 2]
    assert tok[0, :1].tolist() == [2] and tok[1].tolist() == [1, 2, 2] and tok[2].tolist() == [1, 1, 1]
    # V = 151936: draft i rejected by u_acc = 1 at position j = s % k (earlier ones accepted by u = 0)
    S, k, V = 16, 4, 151936
    rng = np.random.default_rng(9)
    Lt2, Ld2 = _case(rng, S, k, V)
    draft = np.array([[_draw(Ld2[s, i], 1.0, rng.random()) for i in range(k)] for s in range(S)], np.int32)
    ua2 = np.zeros((S, k), np.float32)
    for s in range(S):
        ua2[s, s % k] = 1.0
    ur2, ub2 = rng.random(S).astype(np.float32), rng.random(S).astype(np.float32)
    tok, n = ih.spec_accept(_dev(Lt2), _dev(Ld2), _dev(draft), 0.8, _dev(ua2), _dev(ur2), _dev(ub2), mode=1)
    tok, n = tok.cpu().numpy(), n.cpu().numpy()
    for s in range(S):
        rt, rn = O.spec_accept(Lt2[s], Ld2[s], draft[s], 0.8, ua2[s], float(ur2[s]), float(ub2[s]), 1)
        assert n[s] == rn == s % k
        assert len(rt) == ih.n_tokens(rn, k, 1) == (k + 1 if rn == k - 1 else rn + 1)
        assert tok[s, :len(rt)].tolist() == rt.tolist(), (s, tok[s], rt)


def test_greedy_verify(ih):
    rng = np.random.default_rng(3)
    S, k, V = 64, 4, 151936
    L = rng.standard_normal((S, k + 1, V)).astype(np.float32)
    am = L.argmax(-1)
    draft = am[:, :k].astype(np.int32).copy()
    for s in range(S):  # break the chain at a step-dependent position
        j = s % (k + 1)
        if j < k:
            draft[s, j] = (draft[s, j] + 1) % V
    # planted ties: equal maxima at two indices, the first must win
    L[0, 1, 5] = L[0, 1, 77] = 50.0
    L[1, 0, 151935] = L[1, 0, 4096] = 60.0
    n, a = ih.greedy_verify(_dev(L), _dev(draft))
    n, a = n.cpu().numpy(), a.cpu().numpy()
    for s in range(S):
        rn, ra = O.greedy_verify(L[s], draft[s])
        assert rn == n[s] and np.array_equal(ra, a[s]), s
    assert a[0, 1] == 5 and a[1, 0] == 4096


def test_greedy_verify_nonfinite_rows(ih):
    """Rows of -Inf, NaN and signed zeros follow Julia's argmax (isless
    order: the first NaN wins, +0.0 above -0.0, a row of -Inf gives its
    first index), never an index outside [0, V)."""
    k, V = 5, 151936
    L = np.random.default_rng(4).standard_normal((1, k + 1, V)).astype(np.float32)
    L[0, 0, :] = -np.inf                      # all -Inf
    L[0, 1, 70000] = np.nan                   # one NaN
    L[0, 1, 90000] = np.nan
    L[0, 2, :] = 0.0                          # -0.0 first, +0.0 later
    L[0, 2, :5000] = -0.0
    L[0, 3, :] = np.nan                       # all NaN
    L[0, 4, 4095] = L[0, 4, 4096] = np.inf    # +Inf tie across a chunk edge
    draft = np.array([[0, 70000, 5000, 0, 4095]], np.int32)
    n, a = ih.greedy_verify(_dev(L), _dev(draft))
    n, a = n.cpu().numpy(), a.cpu().numpy()
    rn, ra = O.greedy_verify(L[0], draft[0])
    assert a[0].tolist() == ra.tolist(), (a, ra)
    assert a[0, :5].tolist() == [0, 70000, 5000, 0, 4095] and rn == n[0] == 5


def _tree_parents(n, branching=(4, 4, 4)):
    par = [-1]
    frontier = [0]
    for b in branching:
        nxt = []
        for p in frontier:
            for _ in range(b):
                if len(par) < n:
                    par.append(p)
                    nxt.append(len(par) - 1)
        frontier = nxt
    while len(par) < n:
        par.append(frontier[(len(par)) % len(frontier)] if frontier else 0)
    par[0] = 0
    return np.array(par, dtype=np.int32)


@pytest.mark.parametrize("V", [32, 151936])
def test_tree_accept(ih, V):
    rng = np.random.default_rng(V)
    n = 64
    par = _tree_parents(n)
    trials = 8 if V > 1000 else 64
    for t in range(trials):
        Lt = (rng.standard_normal((n, V)) * 2).astype(np.float32)
        Ld = (Lt + rng.standard_normal((n, V)) * 0.7).astype(np.float32)
        tok = np.zeros(n, dtype=np.int32)
        for i in range(1, n):
            tok[i] = _draw(Ld[par[i]], 1.0, rng.random())
        u = rng.random(n).astype(np.float32) * 0.9
        path = ih.tree_accept(_dev(Lt), _dev(Ld), _dev(tok), _dev(par), 1.0, _dev(u)).cpu().numpy()
        ref = O.tree_accept(Lt, Ld, tok, par, 1.0, u)
        assert np.array_equal(path, ref), (t, path, ref)


def test_tree_accept_large_and_malformed(ih):
    """A tree larger than the walk's LDS capacity (its state then lives in the
    workspace), a chain (the walk reduces to the sequential accept), and a
    malformed parent array reported as an error."""
    rng = np.random.default_rng(5000)
    V = 32
    for n, chain in ((5000, False), (300, True)):
        par = np.array([0] + [i - 1 if chain else int(rng.integers(0, i)) for i in range(1, n)], dtype=np.int32)
        Lt = (rng.standard_normal((n, V)) * 1.5).astype(np.float32)
        Ld = (Lt + rng.standard_normal((n, V)) * 0.3).astype(np.float32)
        tok = np.zeros(n, dtype=np.int32)
        for i in range(1, n):
            tok[i] = _draw(Ld[par[i]], 1.0, rng.random())
        u = (rng.random(n) * 0.5).astype(np.float32)
        path = ih.tree_accept(_dev(Lt), _dev(Ld), _dev(tok), _dev(par), 1.0, _dev(u)).cpu().numpy()
        ref = O.tree_accept(Lt, Ld, tok, par, 1.0, u)
        assert np.array_equal(path, ref), (n, path[:8], ref[:8])
        assert len(path) > 3
    bad = _tree_parents(64)
    bad[7] = 9  # parent after its node
    Lt = np.zeros((64, V), dtype=np.float32)
    with pytest.raises(ValueError):
        ih.tree_accept(_dev(Lt), _dev(Lt), _dev(np.zeros(64, dtype=np.int32)), _dev(bad), 1.0,
                       _dev(np.zeros(64, dtype=np.float32)))


def test_rmsnorm(ih):
    x = np.random.default_rng(1).standard_normal((5, 4096)).astype(np.float32) * 3
    got = ih.rmsnorm(_dev(x)).cpu().numpy()
    ref = np.stack([O.rmsnorm(r) for r in x])
    assert rel_l2(got, ref) <= 1e-6


def test_commit_state_and_advance_len(ih):
    """The verify outcome applied on the device (no reference counterpart):
    state[s] = snapshot n of step s, len[s] += n + 1, nothing for n = -1;
    driven by a real accept's out_n inside a replayed HIP graph (no host
    round trip)."""
    import torch
    steps, k, shape = 3, 4, (7, 33)
    snaps = torch.randn(steps, k + 1, *shape, device="cuda")
    state = torch.zeros(steps, *shape, device="cuda")
    n = torch.tensor([2, -1, 4], dtype=torch.int32, device="cuda")
    ih.commit_state_(state, snaps, n)
    assert torch.equal(state[0], snaps[0, 2]) and torch.equal(state[2], snaps[2, 4])
    assert torch.count_nonzero(state[1]) == 0
    lens = torch.tensor([10, 20, 30], dtype=torch.int32, device="cuda")
    ih.advance_len_(lens, n)
    assert lens.tolist() == [13, 20, 35]
    # inside a graph after a real accept
    V = 1000
    rng = np.random.default_rng(77)
    Lt, Ld = _case(rng, steps, k, V, scale=3.0)
    draft = np.array([[_draw(Ld[s, i], 1.0, rng.random()) for i in range(k)] for s in range(steps)], dtype=np.int32)
    args = [_dev(Lt), _dev(Ld), _dev(draft), 1.0, _dev(rng.random((steps, k)).astype(np.float32)),
            _dev(rng.random(steps).astype(np.float32)), _dev(rng.random(steps).astype(np.float32))]
    out_tok = torch.zeros((steps, k + 1), dtype=torch.int32, device="cuda")
    out_n = torch.zeros(steps, dtype=torch.int32, device="cuda")
    state2 = torch.zeros_like(state)
    lens2 = torch.zeros(steps, dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())

    def step():
        ih.spec_accept(*args, out_tok=out_tok, out_n=out_n, stream=s)
        ih.commit_state_(state2, snaps, out_n, stream=s)
        ih.advance_len_(lens2, out_n, stream=s)
    with torch.cuda.stream(s):
        step()
    torch.cuda.synchronize()
    lens2.zero_()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step()
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
    nn = out_n.cpu().numpy()
    for i in range(steps):
        assert torch.equal(state2[i], snaps[i, nn[i]])
    assert lens2.cpu().tolist() == [3 * (int(x) + 1) for x in nn]
