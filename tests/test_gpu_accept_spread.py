"""GPU parity of the accept at the real vocabulary (V = 151936) on spread,
non-one-hot distributions, and of the filtered bonus draw.

* 4096 verify steps per mode: target logits N(0, sd^2) with sd cycling
  through 1, 2, 3 per batch of 256 steps, draft logits = target +
  N(0, 1.5^2), k = 4 drafts drawn from the draft softmax, T = 0.8 (the last
  batch at T = 1.0), explicit uniforms; every step through ihip_spec_accept
  against the oracle's accept (src/SpeculativeDecoding.jl:20-30,75-104).
  Most steps end in the residual draw over all 151936 entries, the rest in
  the bonus draw. Bar (north star): accepted lengths identical on >= 99.9 %
  of steps; the drawn tokens are held to the same bar.
* speculate_and_verify's top_k / top_p (src/SpeculativeDecoding.jl:44-45):
  the bonus token is softmax_sample(target row k; T, top_p, top_k)
  (:100-104, src/ModelCPU.jl:1134-1173). ihip_spec_accept_ex against the
  oracle's accept with the filtered bonus, mode 1 at top_k = 40 and at
  top_p = 0.9 (>= 1000 bonus draws each), both filters with min_p, and
  mode 0; drafts drawn by the filtered sampler as the reference draws them
  (:58). Same bar on the tokens.
Logits are generated on the device in batches of 256 steps (1.4 GB) and
streamed to the host for the oracle."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

V, K = 151936, 4
BATCH = 256


@pytest.fixture(scope="module")
def ih():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import inferno_hip
    assert inferno_hip.quant_kernels_available(), inferno_hip._lib.last_error()
    return inferno_hip


def _batch(g, S, sd, T):
    """Device tensors of S steps: target [S, K+1, V] ~ N(0, sd^2), draft
    [S, K, V] = target + N(0, 1.5^2), drafts ~ softmax(draft / T)."""
    import torch
    Lt = torch.randn((S, K + 1, V), generator=g, device="cuda") * sd
    Ld = Lt[:, :K] + torch.randn((S, K, V), generator=g, device="cuda") * 1.5
    p = torch.softmax(Ld.reshape(-1, V).double() / T, -1)
    draft = torch.multinomial(p, 1, generator=g).view(S, K).to(torch.int32)
    del p
    return Lt, Ld.contiguous(), draft


def _oracle_batch(Lt, Ld, draft, T, ua, ur, ub, mode, **filters):
    return O.spec_accept_batch(Lt, Ld, draft, T, ua, ur, ub, mode, **filters)


def _compare(tok, n, rtok, rn, mode):
    same_len = same_tok = 0
    for s in range(len(rn)):
        nt = O.n_tokens(int(rn[s]), K, mode)
        ok_len = int(n[s]) == int(rn[s])
        same_len += ok_len
        same_tok += ok_len and tok[s, :nt].tolist() == rtok[s, :nt].tolist()
    return same_len, same_tok


def test_spread_distributions_4096_steps(ih):
    import torch
    g = torch.Generator(device="cuda").manual_seed(0x1F3E0003 + 77)
    steps = 16 * BATCH
    stats = {m: {"len": 0, "tok": 0, "residual": 0, "bonus": 0, "hist": np.zeros(K + 1, np.int64)} for m in (0, 1)}
    pmax_mean = []
    for b in range(steps // BATCH):
        sd = (1.0, 2.0, 3.0)[b % 3]
        T = 1.0 if b == steps // BATCH - 1 else 0.8
        Lt, Ld, draft = _batch(g, BATCH, sd, T)
        ua = torch.rand((BATCH, K), generator=g, device="cuda")
        ur = torch.rand(BATCH, generator=g, device="cuda")
        ub = torch.rand(BATCH, generator=g, device="cuda")
        pmax_mean.append(float(torch.softmax(Lt[:, 0] / T, -1).max(-1).values.mean()))
        res = {m: ih.spec_accept(Lt, Ld, draft, T, ua, ur, ub, mode=m) for m in (0, 1)}
        h = [t.cpu().numpy() for t in (Lt, Ld, draft, ua, ur, ub)]
        for m in (0, 1):
            tok, n = (t.cpu().numpy() for t in res[m])
            rtok, rn = _oracle_batch(*h[:3], T, *h[3:], m)
            sl, st = _compare(tok, n, rtok, rn, m)
            a = stats[m]
            a["len"] += sl
            a["tok"] += st
            a["residual"] += int((rn < K).sum())
            a["bonus"] += int((rn == K).sum())
            a["hist"] += np.bincount(rn[rn >= 0], minlength=K + 1)
        print(f"batch {b} (sd {sd}, T {T}): mode 0 lengths {stats[0]['len']}, tokens {stats[0]['tok']}; "
              f"mode 1 lengths {stats[1]['len']}, tokens {stats[1]['tok']} of {(b + 1) * BATCH}", flush=True)
        del Lt, Ld, draft, res
    print(f"mean largest target probability per row: {np.mean(pmax_mean):.4f}", flush=True)
    for m in (0, 1):
        a = stats[m]
        print(f"mode {m}: lengths identical {a['len']}/{steps}, tokens {a['tok']}/{steps}; residual draws "
              f"{a['residual']}, bonus draws {a['bonus']}; length histogram {a['hist'].tolist()}", flush=True)
        assert a["len"] >= 0.999 * steps
        assert a["tok"] >= 0.999 * steps
        assert a["residual"] + a["bonus"] == steps and a["residual"] >= steps // 4


def _filtered_case(ih, g, S, T, mode, top_k, top_p, min_p):
    """S steps at sd 2 whose drafts come from the filtered draft softmax;
    u_acc forces most steps to a bonus draw: all accepted (u = 0), the last
    draft rejected (u = 1 there: mode 1's bonus after the residual), one
    step in eight with random uniforms."""
    import torch
    Lt, Ld, _ = _batch(g, S, 2.0, T)
    ud = torch.rand(S * K, generator=g, device="cuda")
    draft = ih.softmax_sample(Ld.view(-1, V), ud, T, top_p=top_p, top_k=top_k, min_p=min_p).view(S, K)
    ua = torch.zeros((S, K), device="cuda")
    sel = torch.arange(S, device="cuda")
    ua[sel % 8 == 7, K - 1] = 1.0
    rnd = sel % 8 == 6
    ua[rnd] = torch.rand((int(rnd.sum()), K), generator=g, device="cuda")
    ur = torch.rand(S, generator=g, device="cuda")
    ub = torch.rand(S, generator=g, device="cuda")
    return Lt, Ld, draft.contiguous(), ua, ur, ub


@pytest.mark.parametrize("mode,top_k,top_p,min_p,steps", [
    (1, 40, 1.0, 0.0, 1152),
    (1, 0, 0.9, 0.0, 1152),
    (1, 1000, 0.9, 0.05, 256),
    (0, 40, 0.9, 0.0, 256),
])
def test_filtered_bonus(ih, mode, top_k, top_p, min_p, steps):
    import torch
    g = torch.Generator(device="cuda").manual_seed(0x1F3E0003 + 1000 * top_k + int(100 * top_p) + mode)
    T = 0.8
    filt = dict(top_k=top_k, top_p=top_p, min_p=min_p)
    same_len = same_tok = bonus = 0
    for s0 in range(0, steps, 192):
        S = min(192, steps - s0)
        Lt, Ld, draft, ua, ur, ub = _filtered_case(ih, g, S, T, mode, **filt)
        tok, n = (t.cpu().numpy() for t in ih.spec_accept(Lt, Ld, draft, T, ua, ur, ub, mode=mode, **filt))
        h = [t.cpu().numpy() for t in (Lt, Ld, draft, ua, ur, ub)]
        rtok, rn = _oracle_batch(*h[:3], T, *h[3:], mode, **filt)
        sl, st = _compare(tok, n, rtok, rn, mode)
        same_len += sl
        same_tok += st
        bonus += int(sum(O._bonus_slot(int(x), K, mode) >= 0 for x in rn))
        # the filtered bonus keeps to the filter: with top_k its token is among the row's top_k
        if top_k:
            for s in range(S):
                b = O._bonus_slot(int(rn[s]), K, mode)
                if b >= 0:
                    row = h[0][s, K] / np.float32(T)
                    assert row[tok[s, b]] >= np.partition(row, V - top_k)[V - top_k], (s, tok[s, b])
        del Lt, Ld, draft
    print(f"mode {mode} top_k {top_k} top_p {top_p} min_p {min_p}: lengths {same_len}/{steps}, tokens "
          f"{same_tok}/{steps}, filtered bonus draws {bonus}", flush=True)
    assert same_len >= 0.999 * steps and same_tok >= 0.999 * steps
    assert bonus >= (1000 if steps > 1000 else steps // 2)


def test_unfiltered_ex_is_plain(ih):
    """Filters that keep the whole vocabulary (top_k >= V, top_p = 1,
    min_p = 0) take ihip_spec_accept's own bonus draw: the same tokens."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(5)
    Lt, Ld, draft = _batch(g, 64, 2.0, 0.8)
    ua = torch.zeros((64, K), device="cuda")
    ur = torch.rand(64, generator=g, device="cuda")
    ub = torch.rand(64, generator=g, device="cuda")
    for m in (0, 1):
        a = ih.spec_accept(Lt, Ld, draft, 0.8, ua, ur, ub, mode=m)
        b = ih.spec_accept(Lt, Ld, draft, 0.8, ua, ur, ub, mode=m, top_k=V, top_p=1.0, min_p=0.0)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
