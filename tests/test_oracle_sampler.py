"""The oracle's draft-side sampler (softmax_sample, src/ModelCPU.jl:1123-1200;
penalties :1202-1225) pinned by closed forms, by the properties the
reference's own sampler tests assert (tests/unit/test_engine.jl:45-125: T = 0
is the first argmax, top-k = 1 always the max, top-k = 2 only the two
largest, a tiny top-p only the max) and by an independent brute force of the
nucleus on small vocabularies (Python sorted() and math.fsum, not numpy)."""
import math

import numpy as np
import pytest

import oracle as O

LOG = lambda ps: np.log(np.asarray(ps, dtype=np.float64)).astype(np.float32)


def test_closed_forms():
    L = LOG([0.25, 0.75])  # softmax = [0.25, 0.75]
    assert O.softmax_sample(L, 0.2) == 0 and O.softmax_sample(L, 0.25) == 0 and O.softmax_sample(L, 0.3) == 1
    assert O.softmax_sample(L, 0.9999) == 1
    # uniform logits: token = ceil(8 r) - 1
    U = np.zeros(8, np.float32)
    for r in (0.01, 0.124, 0.126, 0.3, 0.5, 0.99):
        assert O.softmax_sample(U, r) == math.ceil(8 * r) - 1, r
    # top-p 0.5 on [0.1 0.2 0.3 0.4]: keep {3, 2} -> [0, 0, 3/7, 4/7]
    P = LOG([0.1, 0.2, 0.3, 0.4])
    assert O.softmax_sample(P, 0.42, top_p=0.5) == 2 and O.softmax_sample(P, 0.43, top_p=0.5) == 3
    np.testing.assert_allclose(O.sample_dist(P, top_p=0.5), [0, 0, 3 / 7, 4 / 7], rtol=1e-6)
    # min-p 0.5 on [0.1 0.3 0.6]: keep p >= 0.3 -> [0, 1/3, 2/3]
    Q = LOG([0.1, 0.3, 0.6])
    np.testing.assert_allclose(O.sample_dist(Q, min_p=0.5), [0, 1 / 3, 2 / 3], rtol=1e-6)
    assert O.softmax_sample(Q, 0.3, min_p=0.5) == 1 and O.softmax_sample(Q, 0.34, min_p=0.5) == 2
    # temperature divides the logits: T = 0.5 squares the odds
    np.testing.assert_allclose(O.sample_dist(L, temperature=0.5), [0.1, 0.9], rtol=1e-6)
    # r = 0 returns the first index even at zero probability (the loop's r <= cumsum_1)
    assert O.softmax_sample(LOG([1e-3, 1.0]), 0.0, top_k=1) == 0
    # r above every cumsum returns the last index
    assert O.softmax_sample(L, 1.5) == 1


def test_reference_test_engine_properties():
    rng = np.random.default_rng(3)
    L = np.array([1.0, 5.0, 2.0, 4.0], np.float32)
    for r in rng.random(200):
        assert O.softmax_sample(L, r, temperature=0.7, top_k=2) in (1, 3)
        assert O.softmax_sample(L, r, temperature=0.7, top_k=1) == 1
        assert O.softmax_sample(L, r, temperature=0.5, top_p=0.01) == 1
        assert 0 <= O.softmax_sample(L, r, temperature=0.7) < 4
    ties = np.array([2.0, 3.0, 3.0, 1.0, 3.0], np.float32)
    assert O.softmax_sample(ties, 0.5, temperature=0.0) == 1  # first argmax
    # T = 0 is Julia's argmax (findmax order): the first NaN wins, +0.0 beats -0.0, -Inf rows give index 0
    nan, inf = np.nan, np.inf
    for row, want in (([1.0, nan, 3.0, nan], 1), ([-0.0, 0.0], 1), ([0.0, -0.0, 0.0], 0), ([-inf] * 3, 0),
                      ([-inf, 2.0, inf, inf], 2), ([nan, 2.0], 0)):
        assert O.softmax_sample(np.array(row, np.float32), 0.5, temperature=0.0) == want, row
    # top-k ties keep the lowest indices: k = 2 of three 3.0s -> {1, 2}
    assert {O.softmax_sample(ties, r, top_k=2) for r in np.linspace(0.01, 0.99, 50)} == {1, 2}


def _nucleus_brute(L, T, top_p):
    z = [float(np.float32(x) / np.float32(T)) for x in L]
    m = max(z)
    e = [math.exp(v - m) for v in z]
    s = math.fsum(e)
    p = [v / s for v in e]
    order = sorted(range(len(p)), key=lambda i: (-p[i], i))
    keep, cum = [], 0.0
    for i in order:
        keep.append(i)
        cum += p[i]
        if cum >= top_p:
            break
    return set(keep), p


@pytest.mark.parametrize("seed", range(6))
def test_nucleus_and_topk_sets_brute_force(seed):
    rng = np.random.default_rng(seed)
    V = 40
    L = (2.0 * rng.standard_normal(V)).astype(np.float32)
    T, top_p = 0.8, 0.7
    want, pb = _nucleus_brute(L, T, top_p)
    got = set(np.nonzero(O.sample_dist(L, temperature=T, top_p=top_p))[0].tolist())
    # equal unless the brute-force cumsum sits within float32 rounding of top_p
    cums = np.cumsum(sorted(pb, reverse=True))
    if np.min(np.abs(cums - top_p)) > 1e-6:
        assert got == want
    k = 7
    topk = set(sorted(range(V), key=lambda i: (-float(L[i]), i))[:k])
    assert set(np.nonzero(O.sample_dist(L, temperature=T, top_k=k))[0].tolist()) == topk
    # inverse CDF: monotone in r, every drawn token has mass, frequencies ~ p
    rs = (np.arange(20000) + 0.5) / 20000
    toks = np.array([O.softmax_sample(L, r, temperature=T, top_p=top_p) for r in rs[::40]])
    assert np.all(np.diff(toks) >= 0)
    p = O.sample_dist(L, temperature=T, top_p=top_p)
    assert all(p[t] > 0 for t in toks)
    c = np.cumsum(p, dtype=np.float64)
    idx = np.searchsorted(c, rs)
    freq = np.bincount(idx, minlength=V) / rs.size
    np.testing.assert_allclose(freq, p, atol=2e-4)


def test_penalties_closed_form():
    L = np.array([2.0, -2.0, 0.5, -0.5, 3.0], np.float32)
    out = O.apply_penalties(L, [1, 2, 2, 9, -1], presence=0.5, repetition=2.0)
    # id 1: -2 - 0.5 = -2.5 -> * 2 = -5; id 2: 0.5 - 0.5 = 0 -> not > 0 -> * 2 = 0
    np.testing.assert_array_equal(out, np.array([2.0, -5.0, 0.0, -0.5, 3.0], np.float32))
    out2 = O.apply_penalties(L, [0, 3], repetition=1.5)
    np.testing.assert_array_equal(out2, np.array([2.0 / np.float32(1.5), -2.0, 0.5, -0.5 * np.float32(1.5), 3.0],
                                                 np.float32))
    np.testing.assert_array_equal(O.apply_penalties(L, [0, 1]), L)  # presence 0, repetition 1: no-op


def test_julia_descending_order_and_nan_rows():
    """julia_desc_order is sortperm(L, rev=true): Julia's isless reversed and
    stable (brute force over Python's sort by (isless key, index)): NaN
    first, +0.0 before -0.0, equals by index. With a NaN kept by top-k the
    reference's maximum and probabilities are NaN and the draw returns the
    last index for every r, r <= 0 included; a finite row returns the first
    index at r <= 0 whatever the filters."""
    nan, inf = np.nan, np.inf

    def key(v):  # Julia's isless as a sort key: NaN largest, -0.0 below +0.0
        return (2, 0.0, 0) if np.isnan(v) else (1, float(v), 0 if np.signbit(v) else 1)

    rng = np.random.default_rng(3)
    pool = np.array([nan, inf, -inf, 0.0, -0.0, 1.5, -2.0, 1.5], np.float32)
    for _ in range(200):
        L = rng.choice(pool, size=int(rng.integers(1, 12))).astype(np.float32)
        want = sorted(range(L.size), key=lambda i: (tuple(-x for x in key(L[i])), i))
        assert O.julia_desc_order(L).tolist() == want, L
    V = 50
    x = np.linspace(-2, 2, V).astype(np.float32)
    y = x.copy()
    y[17] = nan
    for kw in (dict(top_k=5), dict(top_k=1), dict(top_k=5, top_p=0.5), dict(top_k=5, min_p=0.1), dict()):
        for r in (0.0, -1.0, 0.3, 0.999):
            assert O.softmax_sample(y, r, **kw) == V - 1, (kw, r)
            if r <= 0:
                assert O.softmax_sample(x, r, **kw) == 0, (kw, r)
    assert set(np.nonzero(O.sample_dist(x, top_k=3))[0].tolist()) == {47, 48, 49}


def test_top_p_is_float32():
    """softmax_sample's top_p is a Float32 (src/ModelCPU.jl:1123): 0.9 is
    0.899999976..., so 4500 of 5000 equal probabilities fl32(1/5000)
    (exact sum 0.8999999773) reach it where a float64 0.9 would need 4501."""
    L = np.zeros(5000, np.float32)
    p = O.sample_dist(L, top_p=0.9)
    assert int((p > 0).sum()) == 4500
    assert 4500 * float(np.float32(1 / 5000)) >= float(np.float32(0.9)) > 0.8999999
