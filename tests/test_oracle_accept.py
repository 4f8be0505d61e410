"""Pins of the CPU oracle's softmax statistics, speculative accept (both
modes), greedy verify and tree accept (no GPU). Beyond the committed
fixtures, each function is checked against an independent statement:
closed forms, brute-force path enumeration, and the defining property of
standard speculative sampling (the output token is distributed exactly as
the target distribution p)."""
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_v1.npz")


def softmax(L, T):
    z = L.astype(np.float64) / T
    e = np.exp(z - z.max())
    return e / e.sum()


def test_softmax_stats_closed_forms():
    for V in (1, 7, 1000):
        m, s = O.softmax_stats(np.full(V, -3.0, np.float32), 1.0)
        assert m == -3.0 and s == pytest.approx(V)
    L = np.zeros(10, np.float32)
    L[4] = 200.0
    m, s = O.softmax_stats(L, 0.5)
    assert m == 400.0 and s == pytest.approx(1.0)


def test_argmax_first_index():
    assert O.argmax_first(np.array([1, 5, 2, 5], np.float32)) == 1
    assert O.argmax_first(np.array([3, 3, 3], np.float32)) == 0
    assert O.argmax_first(np.array([42], np.float32)) == 0
    assert O.argmax_first(np.array([-10, -5, -1], np.float32)) == 2


def test_argmax_nan_and_inf_rows():
    """Julia's findmax order (argmax of mtp_verify_step!): isless, where NaN
    lies above every number (the first NaN wins) and -0.0 below +0.0; a row of
    -Inf returns its first index, as Julia's argmax returns 1 for a vector of
    -Inf. Cross-checked with numpy, whose argmax also returns the first NaN
    and the first of equal values (it differs only on signed zeros), and with
    a brute force over Python's sort by (isless key, index)."""
    inf, nan = np.inf, np.nan

    def key(v):  # Julia's isless as a sort key: NaN last, -0.0 before +0.0
        return (2, 0.0) if np.isnan(v) else (1, float(v), 0 if np.signbit(v) else 1)

    rows = ([-inf] * 5, [1.0, nan, 3.0, nan], [nan, 2.0], [-inf, -inf, 2.0, inf, inf], [0.0, -0.0, 0.0],
            [-inf, nan], [-0.0, 0.0], [-0.0, -0.0, 0.0, 0.0], [5.0, 5.0])
    for row in rows:
        a = np.array(row, np.float32)
        want = max(range(len(a)), key=lambda i: (key(a[i]), -i))
        assert O.argmax_first(a) == want, row
        if not (a == 0).any():
            assert O.argmax_first(a) == int(np.argmax(a)), row
    assert O.argmax_first(np.full(7, -inf, np.float32)) == 0
    assert O.argmax_first(np.array([1.0, nan, 3.0, nan], np.float32)) == 1
    assert O.argmax_first(np.array([-0.0, 0.0], np.float32)) == 1


def test_standard_accept_preserves_target_distribution():
    """Mode 0 with draft x ~ q and independent uniforms must output a token
    distributed as p (k = 1, first output token)."""
    rng = np.random.default_rng(7)
    V = 5
    Lt = rng.standard_normal((2, V)).astype(np.float32)
    Ld = rng.standard_normal((1, V)).astype(np.float32)
    T = 0.8
    p, q = softmax(Lt[0], T), softmax(Ld[0], T)
    n = 60000
    xs = rng.choice(V, size=n, p=q)
    ua, ur = rng.random(n).astype(np.float32), rng.random(n).astype(np.float32)
    counts = np.zeros(V)
    for i in range(n):
        tok, _ = O.spec_accept(Lt, Ld, np.array([xs[i]], np.int32), T, ua[i:i + 1], float(ur[i]), 0.5, 0)
        counts[tok[0]] += 1
    freq = counts / n
    sigma = np.sqrt(p * (1 - p) / n)
    assert np.all(np.abs(freq - p) < 5 * sigma + 1e-4), (freq, p)


def test_accept_special_cases():
    rng = np.random.default_rng(3)
    V, k = 12, 4
    Lt = rng.standard_normal((k + 1, V)).astype(np.float32)
    draft = np.array([0, 5, 7, 11], np.int32)
    # q == p: every draft accepted for any u < 1, then a bonus token
    tok, n = O.spec_accept(Lt, Lt[:k], draft, 1.0, np.full(k, 0.9999, np.float32), 0.3, 0.6, 0)
    assert n == k and tok[:k].tolist() == draft.tolist()
    pk = softmax(Lt[k], 1.0)
    assert tok[k] == int(np.searchsorted(np.cumsum(pk), 0.6 * pk.sum()))
    # p[x_0] = 0: rejected at 0, residual never returns x_0 for u > 0 (at
    # u = 0 the rule u*S <= C_j picks index 0 whatever its weight, as the
    # reference's `r <= cumsum` does, src/SpeculativeDecoding.jl:21-26)
    L2 = Lt.copy()
    L2[0, 0] = -1e30
    for u in np.linspace(0.001, 0.999, 21):
        tok, n = O.spec_accept(L2, Lt[:k], draft, 1.0, np.zeros(k, np.float32), float(u), 0.5, 0)
        assert n == 0 and tok[0] != 0
    # k = 0: a bonus token only
    tok, n = O.spec_accept(Lt[:1], np.zeros((0, V), np.float32), np.zeros(0, np.int32), 0.7,
                           np.zeros(0, np.float32), 0.1, 0.25, 0)
    p0 = softmax(Lt[0], 0.7)
    assert n == 0 and tok[0] == int(np.searchsorted(np.cumsum(p0), 0.25))


def test_reference_mode_hand_case():
    """Reference mode (src/SpeculativeDecoding.jl:75-97): T = 1 ratio with
    scalar q_i, residual max(p - q_i, 0) normalised, first j with u <= cumsum."""
    Lt = np.log(np.array([[0.5, 0.3, 0.2], [0.2, 0.2, 0.6]], np.float32))
    Ld = np.log(np.array([[0.1, 0.6, 0.3]], np.float32))
    # draft token 1: p = 0.3, q = 0.6 -> ratio 0.5
    tok, n = O.spec_accept(Lt, Ld, np.array([1], np.int32), 2.0, np.array([0.49], np.float32), 0.0, 0.0, 1)
    assert n == 1  # accepted, bonus drawn at T = 2
    # reject: residual max(p - 0.6, 0) = [0, 0, 0] -> all-zero -> last index;
    # with gamma = 1 the rejection leaves length(accepted) == gamma, so the
    # reference appends a bonus from target row 1 (:100): p1 = [0.2, 0.2, 0.6]
    # at T = 1, u_bonus 0.0 -> first index with 0 <= cumsum -> token 0
    tok, n = O.spec_accept(Lt, Ld, np.array([1], np.int32), 1.0, np.array([0.51], np.float32), 0.5, 0.0, 1)
    assert n == 0 and tok.tolist() == [2, 0]
    # the bonus row's inverse CDF: u_bonus 0.5 -> cumsum [0.2, 0.4, 1.0] -> token 2
    tok, n = O.spec_accept(Lt, Ld, np.array([1], np.int32), 1.0, np.array([0.51], np.float32), 0.5, 0.5, 1)
    assert n == 0 and tok.tolist() == [2, 2]
    # draft token 2: p = 0.2, q = 0.3; residual max(p - 0.3, 0) = [0.2, 0, 0] -> token 0, then the bonus
    # (u_bonus 0.3 -> cumsum 0.2 < 0.3 <= 0.4 -> token 1)
    tok, n = O.spec_accept(Lt, Ld, np.array([2], np.int32), 1.0, np.array([0.9], np.float32), 0.99, 0.3, 1)
    assert n == 0 and tok.tolist() == [0, 1]
    # standard mode on the same input: residual max(p - q, 0) = [0.4, 0, 0] -> token 0, no bonus
    tok, n = O.spec_accept(Lt, Ld, np.array([2], np.int32), 1.0, np.array([0.9], np.float32), 0.99, 0.3, 0)
    assert n == 0 and tok.tolist() == [0]


def test_reference_mode_bonus_only_after_last_draft():
    """src/SpeculativeDecoding.jl:100 appends the bonus iff length(accepted)
    == gamma: after all gamma drafts stand, or after a rejection of the last
    draft (gamma - 1 drafts + the residual); never after an earlier
    rejection. Two drafts over V = 3, hand-worked at T = 1."""
    Lt = np.log(np.array([[0.5, 0.3, 0.2], [0.5, 0.3, 0.2], [0.1, 0.1, 0.8]], np.float32))
    Ld = np.log(np.array([[0.1, 0.6, 0.3], [0.1, 0.6, 0.3]], np.float32))
    d = np.array([1, 1], np.int32)  # p = 0.3, q = 0.6 at both positions: ratio 0.5
    # reject at position 0: residual max(p - 0.6, 0) = 0 -> last index, no bonus (length 1 < 2)
    tok, n = O.spec_accept(Lt, Ld, d, 1.0, np.array([0.7, 0.1], np.float32), 0.5, 0.9, 1)
    assert n == 0 and tok.tolist() == [2]
    # accept position 0, reject position 1: [1, residual 2] has length gamma -> bonus from row 2
    # (u_bonus 0.9 -> cumsum [0.1, 0.2, 1.0] -> token 2; u_bonus 0.15 -> token 1)
    tok, n = O.spec_accept(Lt, Ld, d, 1.0, np.array([0.1, 0.7], np.float32), 0.5, 0.9, 1)
    assert n == 1 and tok.tolist() == [1, 2, 2]
    tok, n = O.spec_accept(Lt, Ld, d, 1.0, np.array([0.1, 0.7], np.float32), 0.5, 0.15, 1)
    assert n == 1 and tok.tolist() == [1, 2, 1]
    # both accepted: the ordinary bonus
    tok, n = O.spec_accept(Lt, Ld, d, 1.0, np.array([0.1, 0.2], np.float32), 0.5, 0.15, 1)
    assert n == 2 and tok.tolist() == [1, 1, 1]
    # the batched oracle returns the same rows, padded with -1
    Lb = np.stack([Lt] * 3)
    Db = np.stack([Ld] * 3)
    ua = np.array([[0.7, 0.1], [0.1, 0.7], [0.1, 0.2]], np.float32)
    out, ns = O.spec_accept_batch(Lb, Db, np.stack([d] * 3), 1.0, ua, np.full(3, 0.5, np.float32),
                                  np.array([0.9, 0.9, 0.15], np.float32), 1)
    assert ns.tolist() == [0, 1, 2]
    assert out.tolist() == [[2, -1, -1], [1, 2, 2], [1, 1, 1]]


def test_filtered_bonus_hand_cases():
    """speculate_and_verify passes top_p / top_k to the bonus draw only
    (src/SpeculativeDecoding.jl:100-104; the ratio tests and the residual
    use the unfiltered softmaxes, :79-93). Hand-worked on the two-draft
    V = 3 case above, bonus row p = [0.1, 0.1, 0.8] at T = 1:
    top_k = 1 keeps index 2 only (any u -> 2); top_k = 2 keeps {2, 0} (the
    stable descending order puts index 0 before the tied index 1) with
    probabilities [1/9, 0, 8/9]; top_p = 0.5 keeps index 2 only; min_p = 0.2
    drops p < 0.16: index 2 only."""
    Lt = np.log(np.array([[0.5, 0.3, 0.2], [0.5, 0.3, 0.2], [0.1, 0.1, 0.8]], np.float32))
    Ld = np.log(np.array([[0.1, 0.6, 0.3], [0.1, 0.6, 0.3]], np.float32))
    d = np.array([1, 1], np.int32)
    acc_all, rej_last = np.array([0.1, 0.2], np.float32), np.array([0.1, 0.7], np.float32)
    for mode, ua, want in ((1, acc_all, [1, 1]), (1, rej_last, [1, 2]), (0, acc_all, [1, 1])):
        for u in (0.05, 0.15, 0.5, 0.99):
            for kw in (dict(top_k=1), dict(top_p=0.5), dict(min_p=0.2), dict(top_k=1, top_p=0.3)):
                tok, n = O.spec_accept(Lt, Ld, d, 1.0, ua, 0.5, u, mode, **kw)
                assert tok.tolist() == want + [2], (mode, u, kw, tok)
            # top_k = 2: cumsum [1/9, 1/9, 1] -> u <= 1/9 gives 0, else 2 (never the dropped 1)
            tok, n = O.spec_accept(Lt, Ld, d, 1.0, ua, 0.5, u, mode, top_k=2)
            assert tok.tolist() == want + [0 if u <= 1 / 9 else 2], (mode, u, tok)
            # unfiltered: cumsum [0.1, 0.2, 1.0]
            tok, n = O.spec_accept(Lt, Ld, d, 1.0, ua, 0.5, u, mode, top_k=3, top_p=1.0)
            assert tok.tolist() == want + [0 if u <= 0.1 else 1 if u <= 0.2 else 2]
    # an earlier rejection draws no bonus: the filters change nothing
    tok, n = O.spec_accept(Lt, Ld, d, 1.0, np.array([0.7, 0.1], np.float32), 0.5, 0.05, 1, top_k=1)
    assert n == 0 and tok.tolist() == [2]
    # mode 0 rejection at the last draft: the residual only (no bonus), unfiltered
    tok, n = O.spec_accept(Lt, Ld, d, 1.0, rej_last, 0.01, 0.05, 0, top_k=1)
    assert n == 1 and tok.tolist() == [1, 0]
    # the batched oracle applies the same filters per step
    Lb, Db = np.stack([Lt] * 3), np.stack([Ld] * 3)
    ua = np.stack([acc_all, rej_last, np.array([0.7, 0.1], np.float32)])
    out, ns = O.spec_accept_batch(Lb, Db, np.stack([d] * 3), 1.0, ua, np.full(3, 0.5, np.float32),
                                  np.array([0.05, 0.05, 0.05], np.float32), 1, top_k=1)
    assert ns.tolist() == [2, 1, 0] and out.tolist() == [[1, 1, 2], [1, 2, 2], [2, -1, -1]]


def test_filtered_bonus_matches_sampler_oracle():
    """At a larger V the filtered bonus equals softmax_sample on the bonus
    row (itself pinned by test_oracle_sampler), and with filters that keep
    every entry the accept is unchanged."""
    rng = np.random.default_rng(11)
    k, V = 3, 512
    Lt = (rng.standard_normal((k + 1, V)) * 2).astype(np.float32)
    Ld = (Lt[:k] + rng.standard_normal((k, V))).astype(np.float32)
    d = np.array([int(np.argmax(Ld[i])) for i in range(k)], np.int32)
    for u in rng.random(20):
        for kw in (dict(top_k=7), dict(top_p=0.6), dict(top_k=50, top_p=0.8, min_p=0.02)):
            tok, n = O.spec_accept(Lt, Ld, d, 0.7, np.zeros(k, np.float32), 0.5, float(u), 0, **kw)
            assert n == k and tok[k] == O.softmax_sample(Lt[k], float(u), 0.7, **kw)
        a = O.spec_accept(Lt, Ld, d, 0.7, np.zeros(k, np.float32), 0.5, float(u), 1)
        b = O.spec_accept(Lt, Ld, d, 0.7, np.zeros(k, np.float32), 0.5, float(u), 1, top_k=V, top_p=1.0)
        assert a[1] == b[1] and a[0].tolist() == b[0].tolist()


def test_accept_fixtures():
    g = np.load(GOLD, allow_pickle=False)
    for mode in (0, 1):
        for s in range(g["accept_Lt"].shape[0]):
            tok, n = O.spec_accept(g["accept_Lt"][s], g["accept_Ld"][s], g["accept_draft"][s], 0.8,
                                   g["accept_ua"][s], float(g["accept_ur"][s]), float(g["accept_ub"][s]), mode)
            assert n == g[f"accept_mode{mode}_n"][s]
            want = g[f"accept_mode{mode}_tok"][s]
            assert tok.tolist() == want[: len(tok)].tolist() and (want[len(tok):] == -1).all()


def test_greedy_verify():
    rng = np.random.default_rng(4)
    L = rng.standard_normal((5, 30)).astype(np.float32)
    am = L.argmax(-1)
    n, a = O.greedy_verify(L, am[:4].astype(np.int32))
    assert n == 4 and a.tolist() == am.tolist()
    d = am[:4].astype(np.int32).copy()
    d[2] = (d[2] + 1) % 30
    assert O.greedy_verify(L, d)[0] == 2
    L[0, 3] = L[0, 9] = 99.0
    assert O.greedy_verify(L, np.array([3, 0, 0, 0], np.int32))[0] == 1


def _brute_tree(Lt, Ld, tok, par, T, u):
    """Independent statement: enumerate every node, accept it iff every edge
    on its root path passes its ratio test; deepest, then smallest index."""
    n = len(par)
    ok = []
    for i in range(n):
        path, v = [], i
        while v != 0:
            path.append(v)
            v = par[v]
        good = True
        for v in path:
            p, q = softmax(Lt[par[v]], T)[tok[v]], softmax(Ld[par[v]], T)[tok[v]]
            good &= bool(u[v] < min(1.0, p / q))
        ok.append((len(path), -i) if good else (-1, 0))
    best = max(range(n), key=lambda i: ok[i])
    path, v = [best], best
    while v != 0:
        v = par[v]
        path.append(v)
    return path[::-1]


def test_tree_accept_brute_force():
    rng = np.random.default_rng(5)
    for trial in range(200):
        n = int(rng.integers(1, 9))
        V = int(rng.integers(2, 7))
        par = np.array([0] + [int(rng.integers(0, i)) for i in range(1, n)], np.int32)
        Lt = rng.standard_normal((n, V)).astype(np.float32)
        Ld = (Lt + rng.standard_normal((n, V))).astype(np.float32)
        tok = rng.integers(0, V, n).astype(np.int32)
        u = rng.random(n).astype(np.float32)
        got = O.tree_accept(Lt, Ld, tok, par, 1.0, u)
        assert got.tolist() == _brute_tree(Lt, Ld, tok, par, 1.0, u), trial


def test_chain_tree_equals_spec_accept():
    rng = np.random.default_rng(6)
    V, k = 20, 6
    for trial in range(50):
        Lt = rng.standard_normal((k + 1, V)).astype(np.float32)
        Ld = (Lt[:k] + rng.standard_normal((k, V))).astype(np.float32)
        draft = rng.integers(0, V, k).astype(np.int32)
        u = rng.random(k).astype(np.float32)
        _, n = O.spec_accept(Lt, Ld, draft, 1.0, u, 0.5, 0.5, 0)
        # tree node i+1 carries draft i, judged at row i of its parent i
        par = np.arange(-1, k, dtype=np.int32)
        par[0] = 0
        tok = np.concatenate([[0], draft]).astype(np.int32)
        tLt = np.concatenate([Lt[:k], Lt[k:]], 0)
        tLd = np.concatenate([Ld, np.zeros((1, V), np.float32)], 0)
        uu = np.concatenate([[0.0], u]).astype(np.float32)
        path = O.tree_accept(tLt, tLd, tok, par, 1.0, uu)
        assert len(path) - 1 == n
