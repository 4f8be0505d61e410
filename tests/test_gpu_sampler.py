"""GPU: the draft-side sampler (ihip_sample: softmax_sample,
src/ModelCPU.jl:1123-1200) and the logit penalties (ihip_apply_penalties:
src/ModelCPU.jl:1202-1225) against the oracle. Known answers are exact; at
V = 151936 the GPU's tree sums may move a draw only where u lies within
rounding of a step of the oracle's cumulative distribution (or the nucleus
edge within rounding of top_p), and at most one draw per setting may do so.
Penalties are bit-exact."""
import math

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

VOCAB = 151936


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
    return torch.from_numpy(np.array(a, order="C")).cuda()  # (a writable copy: some inputs are read-only views)


def _pad4(L):
    L = np.asarray(L, np.float32)
    n = (-L.size) % 4
    return np.concatenate([L, np.full(n, -np.inf, np.float32)])


def _draw(ih, L, us, **kw):
    L = np.asarray(L, np.float32)
    rows = L if L.ndim == 2 else np.broadcast_to(L, (len(us), L.size))
    return ih.softmax_sample(_dev(np.ascontiguousarray(rows)), _dev(np.asarray(us, np.float32)), **kw).cpu().numpy()


def test_known_answers(ih):
    LOG = lambda ps: np.log(np.asarray(ps, np.float64)).astype(np.float32)
    L = _pad4(LOG([0.25, 0.75]))
    assert list(_draw(ih, L, [0.2, 0.25, 0.3, 0.9999])) == [0, 0, 1, 1]
    U = np.zeros(8, np.float32)
    rs = [0.01, 0.124, 0.126, 0.3, 0.5, 0.99]
    assert list(_draw(ih, U, rs)) == [math.ceil(8 * r) - 1 for r in rs]
    P = LOG([0.1, 0.2, 0.3, 0.4])
    assert list(_draw(ih, P, [0.42, 0.43], top_p=0.5)) == [2, 3]
    Q = _pad4(LOG([0.1, 0.3, 0.6]))
    assert list(_draw(ih, Q, [0.3, 0.34], min_p=0.5)) == [1, 2]
    assert list(_draw(ih, _pad4(LOG([1e-3, 1.0])), [0.0, 0.5], top_k=1)) == [0, 1]  # r = 0 -> first index
    E = np.array([1.0, 5.0, 2.0, 4.0], np.float32)
    rng = np.random.default_rng(5)
    us = rng.random(64).astype(np.float32)
    assert set(_draw(ih, E, us, temperature=0.7, top_k=2)) <= {1, 3}
    assert set(_draw(ih, E, us, temperature=0.7, top_k=1)) == {1}
    assert set(_draw(ih, E, us, temperature=0.5, top_p=0.01)) == {1}
    ties = np.array([2.0, 3.0, 3.0, 1.0, 3.0, 0.0, 0.0, 0.0], np.float32)
    assert list(_draw(ih, ties, [0.5], temperature=0.0)) == [1]
    assert set(_draw(ih, ties, np.linspace(0.01, 0.99, 50), top_k=2)) == {1, 2}


def test_greedy_julia_order(ih):
    """T = 0 is Julia's argmax (src/ModelCPU.jl:1125-1127, findmax order):
    the first NaN above every number, +0.0 above -0.0, the first of equals,
    index 0 for a row of -Inf; rows of one and of several rounds, against
    the oracle's argmax_first."""
    nan, inf = np.nan, np.inf
    rows = [[1.0, nan, 3.0, nan], [-0.0, 0.0, -0.0, 0.0], [0.0, -0.0, 0.0, 0.0], [-inf] * 4, [-inf, 2.0, inf, inf],
            [nan, 2.0, 5.0, 1.0], [5.0, 5.0, 1.0, 5.0]]
    for row in rows:
        L = np.array(row, np.float32)
        for spread in (True, False):
            assert list(_draw(ih, L, [0.5], temperature=0.0, spread=spread)) == [O.argmax_first(L)], (row, spread)
    rng = np.random.default_rng(31)
    big = rng.standard_normal((6, 3 * 4096 + 8)).astype(np.float32)
    big[1, [5000, 9001]] = nan
    big[2, 4097] = 100.0
    big[2, 12000] = 100.0
    big[3, :] = -0.0
    big[3, 8193] = 0.0
    big[4, :] = -inf
    big[5, 7] = inf
    big[5, 11000] = nan
    want = [O.argmax_first(big[r]) for r in range(6)]
    for spread in (True, False):  # spread: each chunk's first argmax, then the row's
        assert list(_draw(ih, big, np.full(6, 0.5, np.float32), temperature=0.0, spread=spread)) == want, spread


def _near_boundary(row, u, g, o, kw):
    p = O.sample_dist(row, **kw).astype(np.float64)
    c = np.cumsum(p)
    lo, hi = min(g, o), max(g, o)
    if abs(u - c[lo]) < 1e-5 or abs(u - c[hi - 1]) < 1e-5:
        return True
    if kw.get("top_p", 1.0) < 1.0:  # nucleus edge within rounding of top_p
        q = O.sample_dist(row, temperature=kw.get("temperature", 1.0), top_k=kw.get("top_k", 0)).astype(np.float64)
        cs = np.cumsum(np.sort(q)[::-1])
        if np.min(np.abs(cs - kw["top_p"])) < 1e-5:
            return True
    return False


SETTINGS = [dict(temperature=1.0), dict(temperature=0.8, top_p=0.9), dict(temperature=0.8, top_k=40),
            dict(temperature=0.7, top_k=50, top_p=0.95), dict(temperature=1.0, min_p=0.05),
            dict(temperature=0.8, top_p=0.9, min_p=0.02), dict(temperature=1.0, top_k=4096, top_p=0.9),
            dict(temperature=0.0)]


@pytest.mark.parametrize("kw", SETTINGS, ids=lambda kw: ",".join(f"{k}={v}" for k, v in kw.items()))
def test_parity_full_vocab(ih, kw):
    rows = 48
    rng = np.random.default_rng(hash(tuple(sorted(kw.items()))) % 2**32)
    L = (3.0 * rng.standard_normal((rows, VOCAB))).astype(np.float32)
    us = rng.random(rows).astype(np.float32)
    got = _draw(ih, L, us, **kw)
    bad = 0
    for r in range(rows):
        want = O.softmax_sample(L[r], float(us[r]), **kw)
        if got[r] != want:
            assert kw.get("temperature", 1.0) != 0.0, (r, got[r], want)
            assert _near_boundary(L[r], float(us[r]), int(got[r]), want, kw), (r, got[r], want)
            bad += 1
    assert bad <= 1


def test_plain_draw_paths(ih):
    """Plain draws (no top-p, no min-p), both ways: spread over workgroups
    of 4096 logits (ihip_sample_ex), and in one workgroup per row, which
    takes its rounds' sums from per-wave parts of the statistics pass up to
    V = 262144 and the online pass beyond it or when the row has no finite
    maximum or sum: rows that are all -Inf or hold a NaN or +Inf (the
    reference's V - 1), two finite entries among -Inf, u = 0, and Gaussian
    rows at V = 262144, 300000 and 151936."""
    V = 4096
    a = np.full(V, -np.inf, np.float32)
    b = np.zeros(V, np.float32)
    b[7] = np.nan
    c = np.full(V, -np.inf, np.float32)
    c[100] = c[3000] = 1.0
    d = np.zeros(V, np.float32)
    d[5] = np.inf
    us = [0.1, 0.5, 0.9]
    rng = np.random.default_rng(11)
    big = [((3.0 * rng.standard_normal((8, Vb))).astype(np.float32), rng.random(8).astype(np.float32))
           for Vb in (262144, 300000)]
    # spread: ihip_sample_ex (rows over workgroups of 4096 logits); else one workgroup per row
    for spread in (True, False):
        assert list(_draw(ih, a, us, spread=spread)) == [V - 1] * 3
        assert list(_draw(ih, b, us, spread=spread)) == [V - 1] * 3
        assert list(_draw(ih, c, us, spread=spread)) == [100, 100, 3000]
        assert list(_draw(ih, d, us, spread=spread)) == [V - 1] * 3
        assert list(_draw(ih, c, [0.0], spread=spread)) == [0]  # r = 0: the first index
        for L, u8 in big:
            got = _draw(ih, L, u8, temperature=0.9, spread=spread)
            for r in range(8):
                want = O.softmax_sample(L[r], float(u8[r]), temperature=0.9)
                assert got[r] == want or _near_boundary(L[r], float(u8[r]), int(got[r]), want,
                                                        dict(temperature=0.9)), (spread, L.shape, r, got[r], want)
    # the one-workgroup plain path at full vocabulary (the parity tests take the spread one)
    L = (3.0 * rng.standard_normal((48, VOCAB))).astype(np.float32)
    u48 = rng.random(48).astype(np.float32)
    got = _draw(ih, L, u48, spread=False)
    bad = 0
    for r in range(48):
        want = O.softmax_sample(L[r], float(u48[r]))
        if got[r] != want:
            assert _near_boundary(L[r], float(u48[r]), int(got[r]), want, {}), (r, got[r], want)
            bad += 1
    assert bad <= 1


def test_topk_spread_matches_one_workgroup(ih):
    """Top-k draws with 1 <= k <= 64 over at most 64 chunks of 4096 logits
    spread over workgroups (each chunk's top-k, then the row's among them)
    give the one-workgroup kernel's tokens bit for bit: Gaussian and
    quantized (tied) rows at V = 151936, 262144 and 4100, rows all -Inf or
    holding NaN or +Inf (V - 1 on both), u = 0, with top-p and min-p after
    the cut. (Larger
    k, and V above 262144, take the threshold kernels by count: tested
    against the oracle below.)"""
    rng = np.random.default_rng(17)
    cases = []
    for V in (151936, 262144, 4100):
        G = (3.0 * rng.standard_normal((24, V))).astype(np.float32)
        Qz = rng.integers(0, 3, size=(8, V)).astype(np.float32)
        X = np.concatenate([G, Qz])
        X[24, :] = -np.inf
        X[25, 11] = np.nan
        X[26, V - 3] = np.inf
        cases.append(X)
    settings = [dict(temperature=0.8, top_k=40), dict(temperature=1.0, top_k=1), dict(temperature=0.7, top_k=64),
                dict(temperature=0.7, top_k=50, top_p=0.95), dict(temperature=1.1, top_k=7, min_p=0.1),
                dict(temperature=0.9, top_k=37, top_p=0.6, min_p=0.02)]
    for L in cases:
        us = rng.random(L.shape[0]).astype(np.float32)
        us[1] = 0.0
        for kw in settings:
            a = _draw(ih, L, us, spread=True, **kw)
            b = _draw(ih, L, us, spread=False, **kw)
            assert np.array_equal(a, b), (L.shape, kw, np.nonzero(a != b)[0][:8])
    # against the oracle at k = 40 (V = 151936, quantized ties)
    L = cases[0][24:]
    us = rng.random(L.shape[0]).astype(np.float32)
    got = _draw(ih, L, us, temperature=0.9, top_k=40)
    for r in range(3, L.shape[0]):
        want = O.softmax_sample(L[r], float(us[r]), temperature=0.9, top_k=40)
        assert got[r] == want or _near_boundary(L[r], float(us[r]), int(got[r]), want,
                                                dict(temperature=0.9, top_k=40)), r


def test_topp_minp_spread(ih):
    """Top-p and min-p (each alone and together), spread over workgroups of
    4096 logits (ihip_sample_ex: threshold histograms, the bucket's gather,
    key passes, kept sums per stage) and in one workgroup per row, against
    the oracle: Gaussian
    rows at V = 151936 and 300000, quantized rows whose threshold bucket
    holds ties (gathered at V = 8192, over the row at V = 16384), a flat row
    (every logit tied: the first n kept), rows all -Inf or holding NaN or
    +Inf (V - 1), and u = 0 (the first index)."""
    rng = np.random.default_rng(23)
    cases = [(3.0 * rng.standard_normal((16, VOCAB))).astype(np.float32),
             (3.0 * rng.standard_normal((4, 300000))).astype(np.float32),
             rng.integers(0, 3, size=(16, 8192)).astype(np.float32),
             rng.integers(0, 3, size=(8, 16384)).astype(np.float32)]
    settings = [dict(temperature=0.8, top_p=0.9), dict(temperature=1.0, top_p=0.5), dict(temperature=0.7, top_p=0.0),
                dict(temperature=1.0, min_p=0.05), dict(temperature=0.9, min_p=0.3),
                dict(temperature=0.8, top_p=0.9, min_p=0.02), dict(temperature=1.0, top_p=0.5, min_p=0.3)]
    for L in cases:
        us = rng.random(L.shape[0]).astype(np.float32)
        for kw in settings:
            want = [O.softmax_sample(L[r], float(us[r]), **kw) for r in range(L.shape[0])]
            for spread in (True, False):
                got = _draw(ih, L, us, spread=spread, **kw)
                bad = 0
                for r in range(L.shape[0]):
                    if got[r] != want[r]:
                        assert _near_boundary(L[r], float(us[r]), int(got[r]), want[r], kw), \
                            (spread, L.shape, kw, r, got[r], want[r])
                        bad += 1
                assert bad <= 1, (spread, L.shape, kw)
    flat = np.zeros(8192, np.float32)
    uf = np.array([0.01, 0.3, 0.49, 0.77, 0.999], np.float32)
    V = 4096
    a = np.full(V, -np.inf, np.float32)
    b = np.zeros(V, np.float32)
    b[7] = np.nan
    d = np.zeros(V, np.float32)
    d[5] = np.inf
    for spread in (True, False):
        assert list(_draw(ih, flat, uf, top_p=0.5, spread=spread)) == [math.ceil(4096 * u) - 1 for u in uf]
        assert list(_draw(ih, flat, uf, min_p=0.5, spread=spread)) == [math.ceil(8192 * u) - 1 for u in uf]
        assert list(_draw(ih, flat, uf, top_p=0.5, min_p=0.5, spread=spread)) == [math.ceil(4096 * u) - 1 for u in uf]
        for kw in (dict(top_p=0.9), dict(min_p=0.05), dict(top_p=0.9, min_p=0.05)):
            for x in (a, b, d):
                assert list(_draw(ih, x, [0.1, 0.9], spread=spread, **kw)) == [V - 1] * 2, (spread, kw)
            assert list(_draw(ih, flat, [0.0], spread=spread, **kw)) == [0]


def test_topk_large_spread(ih):
    """Top-k above 64 (or at V above 262144), with or without top-p and
    min-p, spread over workgroups of 4096 logits (the k-th element's bucket
    and key by count from the chunks' histograms, the kept entries compacted
    in index order, the one-row kernel's candidate draw over them) give the
    one-workgroup kernel's tokens bit for bit, and match the oracle:
    Gaussian rows at V = 151936 and 300000, quantized rows (ties at the
    threshold, gathered and over the row), a flat row (the first k), rows
    all -Inf or +Inf (V - 1) and a row holding a NaN (the reference's top-k
    keeps it, first in its descending sortperm, and every probability is
    then NaN: V - 1; also through the k <= 64 candidate path)."""
    rng = np.random.default_rng(29)
    cases = [(3.0 * rng.standard_normal((12, VOCAB))).astype(np.float32),
             (3.0 * rng.standard_normal((4, 300000))).astype(np.float32),
             rng.integers(0, 3, size=(12, 8192)).astype(np.float32),
             rng.integers(0, 3, size=(6, 16384)).astype(np.float32)]
    settings = [dict(temperature=0.8, top_k=100), dict(temperature=1.0, top_k=1000), dict(temperature=0.7, top_k=4000),
                dict(temperature=0.9, top_k=100, min_p=0.05), dict(temperature=0.8, top_k=40),
                dict(temperature=0.8, top_k=1000, top_p=0.9), dict(temperature=1.0, top_k=300, top_p=0.5, min_p=0.05)]
    for L in cases:
        us = rng.random(L.shape[0]).astype(np.float32)
        for kw in settings:
            want = [O.softmax_sample(L[r], float(us[r]), **kw) for r in range(L.shape[0])]
            got = _draw(ih, L, us, spread=False, **kw)
            assert np.array_equal(_draw(ih, L, us, spread=True, **kw), got), (L.shape, kw)
            bad = 0
            for r in range(L.shape[0]):
                if got[r] != want[r]:
                    assert _near_boundary(L[r], float(us[r]), int(got[r]), want[r], kw), \
                        (L.shape, kw, r, got[r], want[r])
                    bad += 1
            assert bad <= 1, (L.shape, kw)
    flat = np.zeros(8192, np.float32)
    uf = np.array([0.013, 0.303, 0.487, 0.771, 0.9985], np.float32)
    V = 4096
    a = np.full(V, -np.inf, np.float32)
    d = np.zeros(V, np.float32)
    d[5] = np.inf
    b = np.zeros(V, np.float32)
    b[7] = np.nan
    for spread in (True, False):
        assert list(_draw(ih, flat, uf, top_k=100, spread=spread)) == [math.ceil(100 * float(u)) - 1 for u in uf]
        for kw in (dict(top_k=100), dict(top_k=100, min_p=0.05), dict(top_k=40), dict(top_k=40, top_p=0.9),
                   dict(top_k=100, top_p=0.9)):
            for x in (a, d):
                assert list(_draw(ih, x, [0.1, 0.9], spread=spread, **kw)) == [V - 1] * 2, (spread, kw)
            ub = [0.013, 0.303, 0.777]
            assert list(_draw(ih, b, ub, spread=spread, **kw)) == [O.softmax_sample(b, u, **kw) for u in ub]
            assert list(_draw(ih, flat, [0.0], spread=spread, **kw)) == [0]


def test_topk_ties_exact(ih):
    # all equal: top_k = 5 keeps indices 0..4, token = ceil(5 u) - 1
    Z = np.zeros(4096, np.float32)
    us = np.array([0.03, 0.19, 0.21, 0.5, 0.77, 0.97], np.float32)
    assert list(_draw(ih, Z, us, top_k=5)) == [math.ceil(5 * u) - 1 for u in us]
    # quantized logits: ties straddle the k-th place; kept = all 2s, then 1s by index
    rng = np.random.default_rng(9)
    L = rng.integers(0, 3, size=(16, 8192)).astype(np.float32)
    us = rng.random(16).astype(np.float32)
    for k in (1, 37, 100, 4000):
        got = _draw(ih, L, us, top_k=k, temperature=0.9)
        for r in range(16):
            want = O.softmax_sample(L[r], float(us[r]), temperature=0.9, top_k=k)
            assert got[r] == want or _near_boundary(L[r], float(us[r]), int(got[r]), want,
                                                    dict(temperature=0.9, top_k=k)), (k, r)


def test_penalties_exact(ih):
    import torch
    rng = np.random.default_rng(13)
    L = (2.0 * rng.standard_normal((3, 1000))).astype(np.float32)
    ids = np.array([5, 17, 17, 999, 1000, -3, 0, 42, 5], np.int32)  # repeats and out-of-range ids
    d = _dev(L)
    ih.apply_penalties_(d, torch.from_numpy(ids), presence=0.4, repetition=1.3)
    want = np.stack([O.apply_penalties(L[r], ids, 0.4, 1.3) for r in range(3)])
    np.testing.assert_array_equal(d.cpu().numpy(), want)
    per_row = rng.integers(-5, 1005, size=(3, 64)).astype(np.int32)
    d2 = _dev(L)
    ih.apply_penalties_(d2, torch.from_numpy(per_row), presence=-0.25, repetition=0.8)
    want2 = np.stack([O.apply_penalties(L[r], per_row[r], -0.25, 0.8) for r in range(3)])
    np.testing.assert_array_equal(d2.cpu().numpy(), want2)
    d3 = _dev(L)
    ih.apply_penalties_(d3, torch.from_numpy(ids))  # presence 0, repetition 1: untouched
    np.testing.assert_array_equal(d3.cpu().numpy(), L)


DEGENERATE_SETTINGS = [dict(), dict(temperature=0.8, top_k=40), dict(temperature=0.8, top_k=1000),
                       dict(temperature=0.8, top_k=10000), dict(top_p=0.9), dict(min_p=0.05),
                       dict(top_k=100, top_p=0.9, min_p=0.05), dict(top_k=6000, top_p=0.9)]


def test_degenerate_rows_before_u0(ih):
    """A row whose reference probabilities are all NaN (all -Inf, a +Inf, a
    NaN anywhere: kept by top-k too) draws the last index whatever u is,
    u <= 0 included (the reference's r <= cumsum is false against NaN);
    a finite row draws index 0 at u <= 0. Every setting and both entry
    points, one and several rounds, against the oracle."""
    for V in (4096, 3 * 4096 + 5):
        a = np.full(V, -np.inf, np.float32)
        d = np.zeros(V, np.float32)
        d[V - 2] = np.inf
        b = np.zeros(V, np.float32)
        b[V // 2] = np.nan
        c = np.full(V, -np.inf, np.float32)
        c[0] = np.nan  # a NaN among -Inf (the round's maximum is -Inf)
        c[V - 1] = 1.0
        f = np.linspace(-1, 1, V).astype(np.float32)
        for kw in DEGENERATE_SETTINGS:
            for x in (a, d, b, c, f):
                us = [0.0, -0.5, 0.37]
                want = [O.softmax_sample(x, u, **kw) for u in us]
                for spread in (True, False):
                    got = list(_draw(ih, x, us, spread=spread, **kw))
                    assert got == want, (V, kw, spread, got, want)


ODD_SETTINGS = [dict(temperature=1.0), dict(temperature=0.8, top_p=0.9), dict(temperature=0.8, top_k=40),
                dict(temperature=0.7, top_k=50, top_p=0.95), dict(temperature=1.0, min_p=0.05),
                dict(temperature=0.9, top_k=1000, top_p=0.9), dict(temperature=1.0, top_k=10000),
                dict(temperature=0.0)]


@pytest.mark.parametrize("kw", ODD_SETTINGS, ids=lambda kw: ",".join(f"{k}={v}" for k, v in kw.items()))
def test_any_vocabulary_size(ih, kw):
    """Vocabularies that are not a multiple of 4 (rows then start at any
    4-byte address): V = 151937 against the oracle on both entry points, and
    tiny V = 1, 2, 3, 5, 4099 exactly."""
    rng = np.random.default_rng(41)
    rows, V = 24, 151937
    L = (3.0 * rng.standard_normal((rows, V))).astype(np.float32)
    us = rng.random(rows).astype(np.float32)
    want = [O.softmax_sample(L[r], float(us[r]), **kw) for r in range(rows)]
    for spread in (True, False):
        got = _draw(ih, L, us, spread=spread, **kw)
        bad = 0
        for r in range(rows):
            if got[r] != want[r]:
                assert kw.get("temperature", 1.0) != 0.0, (r, got[r], want[r])
                assert _near_boundary(L[r], float(us[r]), int(got[r]), want[r], kw), (spread, r, got[r], want[r])
                bad += 1
        assert bad <= 1, (spread, kw)
    for Vs in (1, 2, 3, 5, 4099):
        X = np.round(2.0 * rng.standard_normal((6, Vs))).astype(np.float32)
        u6 = rng.random(6).astype(np.float32)
        want = [O.softmax_sample(X[r], float(u6[r]), **kw) for r in range(6)]
        for spread in (True, False):
            got = list(_draw(ih, X, u6, spread=spread, **kw))
            assert got == want, (Vs, spread, got, want)


@pytest.mark.parametrize("kw", [dict(temperature=0.8, top_k=10000), dict(temperature=1.0, top_k=5000, top_p=0.9),
                                dict(temperature=0.9, top_k=20000, min_p=0.01),
                                dict(temperature=0.7, top_k=150000, top_p=0.8, min_p=0.02)],
                         ids=lambda kw: ",".join(f"{k}={v}" for k, v in kw.items()))
def test_topk_above_4096(ih, kw):
    """top_k from 4097 up to V - 1 (the k-th element's threshold by count,
    the softmax over the kept entries, then top-p / min-p on it) against the
    oracle at V = 151936, Gaussian and quantized (tied) rows, both entry
    points; a flat row keeps its first k."""
    rng = np.random.default_rng(43)
    L = np.concatenate([(3.0 * rng.standard_normal((16, VOCAB))).astype(np.float32),
                        rng.integers(0, 4, size=(8, VOCAB)).astype(np.float32)])
    us = rng.random(L.shape[0]).astype(np.float32)
    want = [O.softmax_sample(L[r], float(us[r]), **kw) for r in range(L.shape[0])]
    for spread in (True, False):
        got = _draw(ih, L, us, spread=spread, **kw)
        bad = 0
        for r in range(L.shape[0]):
            if got[r] != want[r]:
                assert _near_boundary(L[r], float(us[r]), int(got[r]), want[r], kw), (spread, r, got[r], want[r])
                bad += 1
        assert bad <= 1, (spread, kw)
    k = kw["top_k"]
    flat = np.zeros(VOCAB, np.float32)
    js = [0, 37, 500, 4000, k - 1]
    uf = ((np.array(js) + 0.5) / k).astype(np.float32)  # mid-step: token j
    if kw.get("top_p", 1.0) >= 1.0:
        for spread in (True, False):
            assert list(_draw(ih, flat, uf, spread=spread, **kw)) == js


def test_penalties_beyond_262144(ih):
    """Penalties over a vocabulary of 300000 (the LDS bitmap taken in two
    windows): ids on both sides of 262144, repeats, out-of-range ids; one
    list for every row and one per row, bit-exact against the oracle."""
    import torch
    rng = np.random.default_rng(47)
    V = 300000
    L = (2.0 * rng.standard_normal((3, V))).astype(np.float32)
    ids = np.array([5, 262143, 262144, 262144, 299999, 300000, -1, 150000, 5, 280001], np.int32)
    d = _dev(L)
    ih.apply_penalties_(d, torch.from_numpy(ids), presence=0.4, repetition=1.3)
    want = np.stack([O.apply_penalties(L[r], ids, 0.4, 1.3) for r in range(3)])
    np.testing.assert_array_equal(d.cpu().numpy(), want)
    per_row = rng.integers(-5, V + 5, size=(3, 2000)).astype(np.int32)
    d2 = _dev(L)
    ih.apply_penalties_(d2, torch.from_numpy(per_row), presence=-0.25, repetition=0.8)
    want2 = np.stack([O.apply_penalties(L[r], per_row[r], -0.25, 0.8) for r in range(3)])
    np.testing.assert_array_equal(d2.cpu().numpy(), want2)
