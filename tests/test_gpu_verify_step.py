"""GPU: one verify step end to end at small dimensions, composed exactly as
the benchmark composes it - per layer the RMSNorm input stage of [q; k; v]
folding the previous layer's deferred `down` partials into the residual, `o`
deferred and folded into the [gate; up] RMSNorm input stage, SiLU gating in
`down`'s input stage, `down` deferred (two ragged K-slices here); then the
final fold + RMSNorm + Q6_K lm_head and a k = 4 accept - against the
oracle's chain of the same operations: fp64 products of the dequantized
weights (src/QuantizedKernels.jl:55-190 formats), RMSNorm as
src/ModelCPU.jl:110-122, SiLU gating and residual adds as
src/ModelCPU.jl:447-473 / :870-891, and the accept rule of
src/SpeculativeDecoding.jl:37-107 (standard mode). Logits within rel-L2
1e-5; the accepted drafts and the resampled / bonus token identical on every
step."""
import numpy as np
import pytest

from _util import rel_l2

import oracle as O
from inferno_hip import formats as F
from inferno_hip import synth

pytestmark = pytest.mark.gpu

H, NQ, NKV, FF, V, LAYERS = 256, 256, 64, 4608, 1000, 2
M, K_DRAFT, EPS = 5, 4, 1e-6
# the chained synthetic weights give logits of row std ~64: the accept runs at
# T = 40 with draft noise of std 60 so that the steps span every accepted
# length (at T = 0.8 both distributions are one-hot and every draft stands)
T, DRAFT_NOISE = 40.0, 60.0
STEPS = 32  # accept steps over the same logits, each with its own drafts and uniforms
TOL_HALF = 1e-2  # north-star bar per matmul output on the half-precision MFMA path
SANITY_HALF = 2e-3  # fp16 operands land near 2e-4 per operation


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


def _weights(m=M):
    rng = np.random.default_rng(2024)
    st = synth.stream_for
    layers = []
    for L in range(LAYERS):
        layers.append({
            "qkv": synth.matrix(F.Q4_K, NQ + 2 * NKV, H, st(L, "e2e_qkv")),
            "o": synth.matrix(F.Q4_K, H, NQ, st(L, "e2e_o")),
            "gu": synth.matrix(F.Q4_K, 2 * FF, H, st(L, "e2e_gu")),
            "down": synth.matrix(F.Q6_K, H, FF, st(L, "e2e_down")),
            "attn_norm": (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32),
            "ffn_norm": (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32),
        })
    lm = synth.matrix(F.Q6_K, V, H, st(9, "e2e_lm"))
    out_norm = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    x0 = rng.standard_normal((m, H)).astype(np.float32)
    return layers, lm, out_norm, x0


def _rms(x, w):
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).mean(axis=1, keepdims=True) + EPS) * w


def _oracle_logits(layers, lm, out_norm, x0):
    f32 = lambda a: np.asarray(a, np.float32)
    M = x0.shape[0]
    x = x0.astype(np.float64)
    for lw in layers:
        qkv = O.gemv_f64(F.Q4_K, lw["qkv"], f32(_rms(x, lw["attn_norm"])), M, NQ + 2 * NKV, H)
        x = x + O.gemv_f64(F.Q4_K, lw["o"], f32(qkv[:, :NQ]), M, H, NQ)
        gu = O.gemv_f64(F.Q4_K, lw["gu"], f32(_rms(x, lw["ffn_norm"])), M, 2 * FF, H)
        g, u = gu[:, :FF], gu[:, FF:]
        with np.errstate(over="ignore"):
            h = g / (1.0 + np.exp(-g)) * u
        x = x + O.gemv_f64(F.Q6_K, lw["down"], f32(h), M, H, FF)
    return O.gemv_f64(F.Q6_K, lm, f32(_rms(x, out_norm)), M, V, H)


def _gpu_logits(ih, layers, lm, out_norm, x0, prec=None):
    """prec: GEMM_F32 (default) or GEMM_HALF, with packed weights."""
    import torch
    ex = ih.gemm_q_ex
    M = x0.shape[0]
    f32 = (ih.GEMM_F32 if prec is None else prec) | ih.GEMM_PACKED
    dfr = f32 | ih.GEMM_DEFER
    dl = [{k: (ih.pack_weights(q, _dev(lw[k]), n, kk) if q is not None else _dev(lw[k]))
           for k, q, n, kk in (("qkv", F.Q4_K, NQ + 2 * NKV, H), ("o", F.Q4_K, H, NQ), ("gu", F.Q4_K, 2 * FF, H),
                               ("down", F.Q6_K, H, FF), ("attn_norm", None, 0, 0), ("ffn_norm", None, 0, 0))}
          for lw in layers]
    plm = ih.pack_weights(F.Q6_K, _dev(lm), V, H)
    gws = ih.quantized_kernels.gemm_ws_bytes
    wsb = max(gws(F.Q4_K, M, NQ + 2 * NKV, H, f32), gws(F.Q4_K, M, H, NQ, f32), gws(F.Q4_K, M, 2 * FF, H, f32),
              gws(F.Q6_K, M, H, FF, f32), gws(F.Q6_K, M, V, H, f32))
    ws, ws_o, ws_down = (torch.empty(wsb, dtype=torch.uint8, device="cuda") for _ in range(3))
    parts = ih.gemm_partials(F.Q6_K, M, H, FF, f32, ws_down)
    o_parts = ih.gemm_partials(F.Q4_K, M, H, NQ, f32, ws_o)
    gu_parts = ih.gemm_partials(F.Q4_K, M, 2 * FF, H, f32, ws)
    assert parts[1] >= 2, parts  # down runs K-sliced (fp32-accurate at M = 5: 16 + 2 units)
    fold_gu = gu_parts[1] > 1
    x = _dev(x0)
    qkv = torch.empty((M, NQ + 2 * NKV), device="cuda")
    gu = torch.empty((M, 2 * FF), device="cuda")
    logits = torch.empty((M, V), device="cuda")
    for i, lw in enumerate(dl):
        ex(F.Q4_K, lw["qkv"], x, NQ + 2 * NKV, H, act=ih.ACT_RMSNORM, norm_w=lw["attn_norm"], eps=EPS, flags=f32,
           out=qkv, ws=ws, add=parts if i > 0 else None)
        ex(F.Q4_K, lw["o"], qkv[:, :NQ], H, NQ, flags=dfr, ws=ws_o)
        ex(F.Q4_K, lw["gu"], x, 2 * FF, H, act=ih.ACT_RMSNORM, norm_w=lw["ffn_norm"], eps=EPS,
           flags=dfr if fold_gu else f32, out=None if fold_gu else gu, ws=ws, add=o_parts)
        if fold_gu:
            ex(F.Q6_K, lw["down"], None, H, FF, act=ih.ACT_SILU_MUL, flags=dfr, ws=ws_down, add=gu_parts, m=M,
               ldx=2 * FF)
        else:
            ex(F.Q6_K, lw["down"], gu, H, FF, act=ih.ACT_SILU_MUL, flags=dfr, ws=ws_down)
    ex(F.Q6_K, plm, x, V, H, act=ih.ACT_RMSNORM, norm_w=_dev(out_norm), eps=EPS, flags=f32, out=logits, ws=ws,
       add=parts)
    torch.cuda.synchronize()
    return logits


def test_verify_step_end_to_end(ih):
    import torch
    layers, lm, out_norm, x0 = _weights()
    ref = _oracle_logits(layers, lm, out_norm, x0)
    logits = _gpu_logits(ih, layers, lm, out_norm, x0)
    got = logits.cpu().numpy()
    err = rel_l2(got, ref)
    print(f"verify step logits rel-L2 {err:.3e}", flush=True)
    assert err <= 1e-5, err

    # draft side around the target rows; per step its own drafts and uniforms
    rng = np.random.default_rng(77)
    ref32 = ref.astype(np.float32)
    Ld = (ref32[:K_DRAFT] + DRAFT_NOISE * rng.standard_normal((K_DRAFT, V))).astype(np.float32)
    z = Ld.astype(np.float64) / T
    q = np.exp(z - z.max(axis=1, keepdims=True))
    q /= q.sum(axis=1, keepdims=True)
    draft = np.stack([[rng.choice(V, p=q[i]) for i in range(K_DRAFT)] for _ in range(STEPS)]).astype(np.int32)
    u_acc = rng.random((STEPS, K_DRAFT)).astype(np.float32)
    u_res = rng.random(STEPS).astype(np.float32)
    u_bonus = rng.random(STEPS).astype(np.float32)
    tgt = logits.unsqueeze(0).expand(STEPS, M, V).contiguous()
    drf = _dev(Ld).unsqueeze(0).expand(STEPS, K_DRAFT, V).contiguous()
    out_tok, out_n = ih.spec_accept(tgt, drf, _dev(draft), T, _dev(u_acc), _dev(u_res), _dev(u_bonus))
    out_tok, out_n = out_tok.cpu().numpy(), out_n.cpu().numpy()
    lengths = []
    for s in range(STEPS):
        toks, n = O.spec_accept(ref32, Ld, draft[s], T, u_acc[s], float(u_res[s]), float(u_bonus[s]))
        assert out_n[s] == n, (s, out_n[s], n)
        assert list(out_tok[s, :n + 1]) == list(toks), (s, out_tok[s], toks)
        lengths.append(n)
    print(f"accepted lengths over {STEPS} steps: {np.bincount(lengths, minlength=K_DRAFT + 1).tolist()}", flush=True)
    assert len(set(lengths)) > 1  # the steps exercise both acceptance and rejection


def test_tree_step_end_to_end(ih):
    """Config 5's composition at M = 64 (half-precision MFMA operands, the
    several-token-tile kernel, `o` and `down` deferred and folded as above),
    then the tree accept walk over a 64-node tree (branching 4, BFS order).
    The half-precision bar applies per matmul output, so every operation of
    the chain is checked against the oracle applied to the GPU's own inputs of
    that operation (each fold as the change it makes to the residual): this
    synthetic chain (o fed by [q; k; v] itself, no attention, residuals
    growing to ~1e6) amplifies fp16-sized rounding of its matmul inputs to
    ~1e-2 .. 4e-2 at the logits (the oracle chain alone, with random 2^-11
    relative perturbations, does so too) while every single operation stays
    near 2e-4. The walk over the GPU logits is identical to the oracle's
    walk over the same logits."""
    import torch
    n, ex = 64, ih.gemm_q_ex
    layers, lm, out_norm, x0 = _weights(n)
    f = ih.GEMM_HALF | ih.GEMM_PACKED
    dfr = f | ih.GEMM_DEFER
    gws = ih.quantized_kernels.gemm_ws_bytes
    wsb = max(gws(F.Q4_K, n, NQ + 2 * NKV, H, f), gws(F.Q4_K, n, H, NQ, f), gws(F.Q4_K, n, 2 * FF, H, f),
              gws(F.Q6_K, n, H, FF, f), gws(F.Q6_K, n, V, H, f))
    ws, ws_o, ws_down = (torch.empty(wsb, dtype=torch.uint8, device="cuda") for _ in range(3))
    parts = ih.gemm_partials(F.Q6_K, n, H, FF, f, ws_down)
    o_parts = ih.gemm_partials(F.Q4_K, n, H, NQ, f, ws_o)
    assert parts[1] >= 2, parts
    x = _dev(x0)
    qkv = torch.empty((n, NQ + 2 * NKV), device="cuda")
    gu = torch.empty((n, 2 * FF), device="cuda")
    logits = torch.empty((n, V), device="cuda")
    h32 = lambda a: a.cpu().numpy()
    errs = {}

    def check(name, got, ref):
        e = rel_l2(got, ref)
        errs[name] = max(errs.get(name, 0.0), e)
        assert e <= TOL_HALF and e <= SANITY_HALF, (name, e)

    d_ref = None
    for i, lw in enumerate(layers):
        pq = ih.pack_weights(F.Q4_K, _dev(lw["qkv"]), NQ + 2 * NKV, H)
        po = ih.pack_weights(F.Q4_K, _dev(lw["o"]), H, NQ)
        pg = ih.pack_weights(F.Q4_K, _dev(lw["gu"]), 2 * FF, H)
        pd = ih.pack_weights(F.Q6_K, _dev(lw["down"]), H, FF)
        xb = h32(x)
        ex(F.Q4_K, pq, x, NQ + 2 * NKV, H, act=ih.ACT_RMSNORM, norm_w=_dev(lw["attn_norm"]), eps=EPS, flags=f,
           out=qkv, ws=ws, add=parts if i > 0 else None)
        xa = h32(x)
        if i > 0:
            check("down (folded)", xa - xb, d_ref)
        q_in = h32(qkv)
        check("qkv", q_in, O.gemv_f64(F.Q4_K, lw["qkv"], _rms(xa, lw["attn_norm"]).astype(np.float32), n,
                                      NQ + 2 * NKV, H))
        ex(F.Q4_K, po, qkv[:, :NQ], H, NQ, flags=dfr, ws=ws_o)
        ex(F.Q4_K, pg, x, 2 * FF, H, act=ih.ACT_RMSNORM, norm_w=_dev(lw["ffn_norm"]), eps=EPS, flags=f, out=gu,
           ws=ws, add=o_parts)
        xo = h32(x)
        check("o (folded)", xo - xa, O.gemv_f64(F.Q4_K, lw["o"], q_in[:, :NQ], n, H, NQ))
        g_out = h32(gu)
        check("gate/up", g_out, O.gemv_f64(F.Q4_K, lw["gu"], _rms(xo, lw["ffn_norm"]).astype(np.float32), n,
                                           2 * FF, H))
        g, u = g_out[:, :FF].astype(np.float64), g_out[:, FF:].astype(np.float64)
        with np.errstate(over="ignore"):
            hh = (g / (1.0 + np.exp(-g)) * u).astype(np.float32)
        d_ref = O.gemv_f64(F.Q6_K, lw["down"], hh, n, H, FF)
        ex(F.Q6_K, pd, gu, H, FF, act=ih.ACT_SILU_MUL, flags=dfr, ws=ws_down)
    plm = ih.pack_weights(F.Q6_K, _dev(lm), V, H)
    xb = h32(x)
    ex(F.Q6_K, plm, x, V, H, act=ih.ACT_RMSNORM, norm_w=_dev(out_norm), eps=EPS, flags=f, out=logits, ws=ws,
       add=parts)
    xf = h32(x)
    check("down (folded)", xf - xb, d_ref)
    got = h32(logits)
    check("lm_head", got, O.gemv_f64(F.Q6_K, lm, _rms(xf, out_norm).astype(np.float32), n, V, H))
    print("tree step (M = 64, half) per-operation rel-L2: "
          + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)

    rng = np.random.default_rng(64)
    par = np.array([-1] + [(i - 1) // 4 for i in range(1, n)], dtype=np.int32)
    Ld = (got + 85.0 * rng.standard_normal((n, V))).astype(np.float32)  # (paths of every length 1..4)
    z = Ld.astype(np.float64) / T
    q = np.exp(z - z.max(axis=1, keepdims=True))
    q /= q.sum(axis=1, keepdims=True)
    tok = np.array([0] + [rng.choice(V, p=q[par[i]]) for i in range(1, n)], dtype=np.int32)
    lens = []
    for trial in range(8):
        u = rng.random(n).astype(np.float32)
        path = ih.tree_accept(logits, _dev(Ld), _dev(tok), _dev(par), T, _dev(u)).cpu().numpy()
        want = O.tree_accept(got, Ld, tok, par, T, u)
        assert list(path) == list(want), (trial, path, want)
        lens.append(len(want))
    print(f"tree accepted path lengths: {lens}", flush=True)
    assert len(set(lens)) > 1
