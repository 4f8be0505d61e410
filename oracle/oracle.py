"""ctypes bindings for the CPU oracle and the reference kernel built in _ref/.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py. The product path never imports this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("INFERNO_ORACLE_LIB", os.path.join(HERE, "liboracle.so"))
REF_PATH = os.path.join(HERE, "_ref", "libquant_kernels_ref.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


def build(ref: bool = False) -> None:
    targets = ["all"] + (["ref"] if ref else [])
    subprocess.run(["make", "-s", "-C", HERE] + targets, check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.orc_fp16_to_fp32.restype = C.c_float
        L.orc_fp16_to_fp32.argtypes = [C.c_uint16]
        L.orc_dequant.argtypes = [C.c_int, _u8p, C.c_int64, _f32p]
        L.orc_gemv_f64.argtypes = [C.c_int, _u8p, _f32p, _f64p, C.c_int, C.c_int, C.c_int]
        L.orc_gemv_seq_f32.argtypes = [C.c_int, _u8p, _f32p, _f32p, C.c_int, C.c_int, C.c_int]
        L.orc_quantize_q8_K.argtypes = [_f32p, _u8p, C.c_int64]
        for n in ("orc_vec_dot_q4_K_q8_K", "orc_vec_dot_q5_K_q8_K", "orc_vec_dot_q6_K_q8_K"):
            getattr(L, n).restype = C.c_float
            getattr(L, n).argtypes = [_u8p, _u8p, C.c_int]
        L.orc_gemv_q8k.argtypes = [C.c_int, _u8p, _f32p, _f32p, _u8p, C.c_int, C.c_int, C.c_int]
        L.orc_softmax_stats.argtypes = [_f32p, C.c_int, C.c_float,
                                        C.POINTER(C.c_double), C.POINTER(C.c_double)]
        L.orc_argmax_first.restype = C.c_int32
        L.orc_argmax_first.argtypes = [_f32p, C.c_int]
        L.orc_spec_accept.argtypes = [_f32p, _f32p, _i32p, C.c_int, C.c_int, C.c_float, _f32p,
                                      C.c_float, C.c_float, C.c_int, _i32p, C.POINTER(C.c_int32)]
        L.orc_spec_accept_batch.argtypes = [_f32p, _f32p, _i32p, C.c_int, C.c_int, C.c_int, C.c_float, _f32p,
                                            _f32p, _f32p, C.c_int, _i32p, _i32p]
        L.orc_greedy_verify.argtypes = [_f32p, _i32p, C.c_int, C.c_int,
                                        C.POINTER(C.c_int32), _i32p]
        L.orc_tree_accept.argtypes = [_f32p, _f32p, _i32p, _i32p, C.c_int, C.c_int, C.c_float,
                                      _f32p, _i32p, C.POINTER(C.c_int32)]
        L.orc_rmsnorm.argtypes = [_f32p, C.c_void_p, C.c_int, C.c_float, _f32p]
        L.orc_cpu_verify_step.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, _u8p, _f32p] + \
            [C.c_int] * 6 + [_f32p, C.c_void_p, C.c_void_p, C.c_float, C.c_void_p, C.c_float, C.c_float, _f32p,
                             _i32p, C.POINTER(C.c_int32)] + [C.POINTER(C.c_double)] * 2 + [_f64p]
        _lib = L
    return _lib


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def dequant(qtype: int, data: np.ndarray, n_blocks: int, block_elems: int) -> np.ndarray:
    out = np.empty(n_blocks * block_elems, dtype=np.float32)
    rc = lib().orc_dequant(qtype, _c(data, np.uint8), n_blocks, out)
    assert rc == 0, rc
    return out


def gemv_f64(qtype, w, x, M, N, K) -> np.ndarray:
    y = np.empty(M * N, dtype=np.float64)
    rc = lib().orc_gemv_f64(qtype, _c(w, np.uint8), _c(x, np.float32), y, M, N, K)
    assert rc == 0, rc
    return y.reshape(M, N)


def gemv_seq_f32(qtype, w, x, M, N, K) -> np.ndarray:
    y = np.empty(M * N, dtype=np.float32)
    rc = lib().orc_gemv_seq_f32(qtype, _c(w, np.uint8), _c(x, np.float32), y, M, N, K)
    assert rc == 0, rc
    return y.reshape(M, N)


def quantize_q8_K(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32)
    q8 = np.zeros((x.size // 256) * 292, dtype=np.uint8)
    lib().orc_quantize_q8_K(x, q8, x.size)
    return q8


def gemv_q8k(qtype, w, x, K, N, nthreads=1) -> np.ndarray:
    out = np.empty(N, dtype=np.float32)
    q8 = np.zeros(max(1, K // 256) * 292, dtype=np.uint8)
    rc = lib().orc_gemv_q8k(qtype, _c(w, np.uint8), _c(x, np.float32), out, q8, K, N, nthreads)
    assert rc == 0, rc
    return out


def softmax_stats(L: np.ndarray, T: float):
    m, s = C.c_double(), C.c_double()
    L = _c(L, np.float32)
    lib().orc_softmax_stats(L, L.size, T, C.byref(m), C.byref(s))
    return m.value, s.value


def argmax_first(L: np.ndarray) -> int:
    L = _c(L, np.float32)
    return int(lib().orc_argmax_first(L, L.size))


def _filtered(V: int, top_p: float, top_k: int, min_p: float) -> bool:
    return (0 < top_k < V) or top_p < 1.0 or min_p > 0.0


def _bonus_slot(n: int, k: int, mode: int) -> int:
    """Index of the bonus token in a step's tokens, or -1 when the step draws
    none: after an all-accept (n == k), and in mode 1 after a rejection of
    the last draft (n == k - 1, src/SpeculativeDecoding.jl:100)."""
    if n == k and n >= 0:
        return k
    if mode == 1 and k >= 1 and n == k - 1:
        return k
    return -1


def spec_accept(Lt, Ld, draft, T, u_acc, u_res, u_bonus, mode=0, top_p: float = 1.0, top_k: int = 0,
                min_p: float = 0.0):
    """speculate_and_verify's accept (src/SpeculativeDecoding.jl:75-104) with
    explicit uniforms: orc_spec_accept, then, when top_p / top_k / min_p
    filter, each bonus token redrawn by softmax_sample(Lt[k]; T, top_p,
    top_k, min_p) with u_bonus (:100-104: the reference's bonus is
    softmax_sample with the same keywords; the ratio tests and residuals do
    not see the filters)."""
    tok, n = _spec_accept_plain(Lt, Ld, draft, T, u_acc, u_res, u_bonus, mode)
    Lt = np.asarray(Lt, dtype=np.float32)
    k, V = Lt.shape[0] - 1, Lt.shape[1]
    b = _bonus_slot(n, k, mode)
    if b >= 0 and _filtered(V, top_p, top_k, min_p):
        tok[b] = softmax_sample(Lt[k], float(np.asarray(u_bonus).ravel()[0]), T, top_p, top_k, min_p)
    return tok, n


def _spec_accept_plain(Lt, Ld, draft, T, u_acc, u_res, u_bonus, mode=0):
    Lt = _c(Lt, np.float32)
    k, V = Lt.shape[0] - 1, Lt.shape[1]
    Ld = _c(Ld, np.float32).reshape(max(k, 1) if k else 1, -1) if k else np.zeros((1, V), np.float32)
    out = np.zeros(k + 1, dtype=np.int32)
    n = C.c_int32()
    ua = _c(u_acc if k else np.zeros(1), np.float32)
    dr = _c(draft if k else np.zeros(1), np.int32)
    rc = lib().orc_spec_accept(Lt, _c(Ld, np.float32), dr, k, V, T, ua, u_res, u_bonus, mode,
                               out, C.byref(n))
    assert rc == 0, rc
    return out[: n_tokens(n.value, k, mode)].copy(), n.value


def n_tokens(n: int, k: int, mode: int) -> int:
    """Tokens a step returns: the n accepted drafts and the resampled or
    bonus token, plus in mode 1 the bonus the reference appends after a
    rejection of the last draft (src/SpeculativeDecoding.jl:100)."""
    if n < 0:
        return 0
    return n + 1 + (1 if mode == 1 and k >= 1 and n == k - 1 else 0)


def spec_accept_batch(Lt, Ld, draft, T, u_acc, u_res, u_bonus, mode=0, top_p: float = 1.0, top_k: int = 0,
                      min_p: float = 0.0):
    """orc_spec_accept over steps (parallel on the host): Lt [S, k+1, V],
    Ld [S, k, V], draft / u_acc [S, k], u_res / u_bonus [S] ->
    (out_tok [S, k+1] padded with -1, out_n [S], -1 for an invalid draft);
    filtered bonus tokens as in spec_accept."""
    Lt = _c(Lt, np.float32)
    S, k1, V = Lt.shape
    k = k1 - 1
    out = np.full((S, k1), -1, dtype=np.int32)
    n = np.zeros(S, dtype=np.int32)
    rc = lib().orc_spec_accept_batch(Lt, _c(Ld, np.float32), _c(draft, np.int32), S, k, V, T, _c(u_acc, np.float32),
                                     _c(u_res, np.float32), _c(u_bonus, np.float32), mode, out, n)
    assert rc == 0, rc
    for s in range(S):  # entries past the step's tokens are left as -1
        out[s, n_tokens(int(n[s]), k, mode):] = -1
    if _filtered(V, top_p, top_k, min_p):
        ub = np.asarray(u_bonus, dtype=np.float32).ravel()
        todo = [(s, _bonus_slot(int(n[s]), k, mode)) for s in range(S)]
        todo = [(s, b) for s, b in todo if b >= 0]
        draw = lambda sb: softmax_sample(Lt[sb[0], k], float(ub[sb[0]]), T, top_p, top_k, min_p)  # noqa: E731
        from concurrent.futures import ThreadPoolExecutor
        with ThreadPoolExecutor(min(8, os.cpu_count() or 1)) as ex:  # numpy's sorts release the GIL
            for (s, b), t in zip(todo, ex.map(draw, todo)):
                out[s, b] = t
    return out, n


def greedy_verify(logits, draft):
    logits = _c(logits, np.float32)
    k, V = logits.shape[0] - 1, logits.shape[1]
    n = C.c_int32()
    am = np.zeros(k + 1, dtype=np.int32)
    dr = _c(draft if k else np.zeros(1), np.int32)
    rc = lib().orc_greedy_verify(logits, dr, k, V, C.byref(n), am)
    assert rc == 0, rc
    return n.value, am


def tree_accept(Lt, Ld, tok, parent, T, u):
    Lt = _c(Lt, np.float32)
    n, V = Lt.shape
    path = np.zeros(n, dtype=np.int32)
    ln = C.c_int32()
    rc = lib().orc_tree_accept(Lt, _c(Ld, np.float32), _c(tok, np.int32), _c(parent, np.int32),
                               n, V, T, _c(u, np.float32), path, C.byref(ln))
    assert rc == 0, rc
    return path[: ln.value].copy()


def rmsnorm(x, eps=1e-6, w=None):
    x = _c(x, np.float32)
    out = np.empty_like(x)
    wp = None if w is None else _c(w, np.float32)
    lib().orc_rmsnorm(x, None if wp is None else wp.ctypes.data, x.size, eps, out)
    return out


# ---- draft-side sampler: numpy restatement (float32 like the reference) ----

def julia_desc_order(L) -> np.ndarray:
    """sortperm(L, rev=true) (src/ModelCPU.jl:1136): Julia's isless
    reversed, stable: every NaN first (NaNs equal), then descending values
    with +0.0 before -0.0, equals in index order."""
    L = np.asarray(L, dtype=np.float32)
    nan = np.isnan(L)
    val = np.where(nan, np.float32(0), L).astype(np.float64)
    pos_zero_first = np.where(np.signbit(L), 0, 1)
    idx = np.arange(L.size)
    return np.lexsort((idx, -pos_zero_first, -val, -nan.astype(np.int8)))


def sample_dist(logits, temperature: float = 1.0, top_p: float = 1.0, top_k: int = 0,
                min_p: float = 0.0) -> np.ndarray:
    """The float32 distribution softmax_sample (src/ModelCPU.jl:1123-1200)
    draws from at temperature > 0: z = L / T (:1130-1132); top-k by the
    stable descending sortperm (:1135-1143); softmax with max subtraction
    (:1146-1148; a NaN kept by top-k makes the maximum and every
    probability NaN, as Julia's maximum propagates NaN); top-p: the shortest
    prefix of the stable descending sortperm of p whose cumulative sum is
    >= top_p, renormalized when the sum
    is > 0 (:1151-1173); min-p: drop p < max(p) * min_p, renormalize
    (:1176-1188). Probabilities are float32 element by element as in the
    reference; its cumulative sums are sequential float32 loops, which over
    ~10^5 terms drift from the exact prefix sum by up to ~1e-4, so the
    contract (as for the residual draw of the accept path) is the exact
    prefix sum, taken here in float64."""
    L = np.asarray(logits, dtype=np.float32).copy()
    V = L.size
    T = np.float32(temperature)
    if T != np.float32(1.0):
        L = L / T
    if top_k > 0:
        order = julia_desc_order(L)
        keep = np.zeros(V, dtype=bool)
        keep[order[:min(top_k, V)]] = True
        L[~keep] = -np.inf
    m = L.max()
    with np.errstate(invalid="ignore", over="ignore"):
        e = np.exp(L - m).astype(np.float32)
    p = (e / e.sum(dtype=np.float32)).astype(np.float32)
    if top_p < 1.0:
        order = np.argsort(-p, kind="stable")
        c = np.cumsum(p[order], dtype=np.float64)
        hit = np.nonzero(c >= float(np.float32(top_p)))[0]  # top_p::Float32 (src/ModelCPU.jl:1123)
        n_keep = int(hit[0]) + 1 if hit.size else V
        keep = np.zeros(V, dtype=bool)
        keep[order[:n_keep]] = True
        p[~keep] = 0.0
        total = p.sum(dtype=np.float32)
        if total > 0:
            p = (p / total).astype(np.float32)
    if min_p > 0.0:
        thr = np.float32(p.max() * np.float32(min_p))
        p[p < thr] = 0.0
        total = p.sum(dtype=np.float32)
        if total > 0:
            p = (p / total).astype(np.float32)
    return p


def softmax_sample(logits, r: float, temperature: float = 1.0, top_p: float = 1.0, top_k: int = 0,
                   min_p: float = 0.0) -> int:
    """softmax_sample (src/ModelCPU.jl:1123-1200), 0-based, with the uniform r
    that the reference draws by rand(Float32) at :1191 given explicitly:
    T = 0 -> Julia's argmax (:1125-1127: findmax order, the first NaN above
    every number, +0.0 above -0.0, the first of equals; argmax_first);
    otherwise the first i with r <= the (exact, float64) prefix sum of
    sample_dist, else the last index (:1191-1198); r <= 0 gives index 0 as
    the reference's loop does."""
    if temperature == 0.0:
        return argmax_first(np.asarray(logits, dtype=np.float32))
    p = sample_dist(logits, temperature, top_p, top_k, min_p)
    c = np.cumsum(p, dtype=np.float64)
    hit = np.nonzero(float(np.float32(r)) <= c)[0]
    return int(hit[0]) if hit.size else p.size - 1


def apply_penalties(logits, token_ids, presence: float = 0.0, repetition: float = 1.0) -> np.ndarray:
    """apply_presence_penalty! then apply_repetition_penalty!
    (src/ModelCPU.jl:1202-1225, in that order at :1247-1248) on a copy, over
    the distinct ids in [0, V) (the keys of the reference's token_counts)."""
    L = np.asarray(logits, dtype=np.float32).copy()
    ids = sorted(set(int(i) for i in np.asarray(token_ids).ravel() if 0 <= int(i) < L.size))
    pres, rep = np.float32(presence), np.float32(repetition)
    if presence != 0.0:
        for i in ids:
            L[i] = L[i] - pres
    if repetition != 1.0:
        for i in ids:
            L[i] = L[i] / rep if L[i] > 0 else L[i] * rep
    return L


# ---- the reference's own C kernel, built from its source into _ref/ ----

_ref = None


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref():
    """Reference src/kernels/quant_kernels.c (signatures at lines 166, 602-697)."""
    global _ref
    if _ref is None:
        R = C.CDLL(REF_PATH)
        for n in ("q4_k_gemv", "q5_k_gemv", "q6_k_gemv"):
            getattr(R, n).restype = None
            getattr(R, n).argtypes = [_u8p, _f32p, _f32p, _u8p, C.c_int, C.c_int]
        R.q8_0_gemv.restype = None
        R.q8_0_gemv.argtypes = [_u8p, _f32p, _f32p, C.c_int, C.c_int]
        R.quantize_row_q8_K.restype = None
        R.quantize_row_q8_K.argtypes = [_f32p, _u8p, C.c_int64]
        for n in ("vec_dot_q4_K_q8_K", "vec_dot_q5_K_q8_K", "vec_dot_q6_K_q8_K"):
            getattr(R, n).restype = C.c_float
            getattr(R, n).argtypes = [_u8p, _u8p, C.c_int]
        _ref = R
    return _ref


def ref_gemv(qtype: int, w: np.ndarray, x: np.ndarray, K: int, N: int) -> np.ndarray:
    R = ref()
    out = np.empty(N, dtype=np.float32)
    w = _c(w, np.uint8)
    x = _c(x, np.float32)
    if qtype == 8:
        R.q8_0_gemv(w, x, out, K, N)
    else:
        q8 = np.zeros((K // 256) * 292, dtype=np.uint8)
        fn = {12: R.q4_k_gemv, 13: R.q5_k_gemv, 14: R.q6_k_gemv}[qtype]
        fn(w, x, out, q8, K, N)
    return out


def ref_quantize_q8_K(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32)
    q8 = np.zeros((x.size // 256) * 292, dtype=np.uint8)
    ref().quantize_row_q8_K(x, q8, x.size)
    return q8


_DOT = {12: "vec_dot_q4_K_q8_K", 13: "vec_dot_q5_K_q8_K", 14: "vec_dot_q6_K_q8_K"}


def ref_vec_dot(qtype: int, w: np.ndarray, q8: np.ndarray, nb: int) -> float:
    """The reference's vec_dot_q*_K_q8_K (src/kernels/quant_kernels.c:204-521)."""
    return float(getattr(ref(), _DOT[qtype])(_c(w, np.uint8), _c(q8, np.uint8), nb))


def vec_dot(qtype: int, w: np.ndarray, q8: np.ndarray, nb: int) -> float:
    """The oracle's restatement of the same lane order (orc_vec_dot_*)."""
    return float(getattr(lib(), "orc_" + _DOT[qtype])(_c(w, np.uint8), _c(q8, np.uint8), nb))


# ---- CPU baseline step driver (bench.py's cpu_baseline leg) ----

class StepLayer(C.Structure):
    """struct orc_step_layer"""
    _fields_ = [(n, C.c_void_p) for n in ("q", "k", "v", "o", "gate", "up", "down", "attn_norm", "ffn_norm")]


def cpu_verify_step(layers, lm, out_norm, x0, H, NQ, NKV, FF, V, Ld=None, draft=None, T=0.8, u_acc=None,
                    u_res=0.5, u_bonus=0.5, kernels="reference"):
    """orc_cpu_verify_step: one verify step of M = x0.shape[0] tokens through
    `layers` (dicts of host GGUF bytes: q [NQ x H], kv [2 NKV x H] (k rows then
    v rows), o [H x NQ], gu [2 FF x H] (gate rows then up rows), down
    [H x FF] (Q6_K), attn_norm / ffn_norm [H]), the Q6_K LM head and, with
    Ld / draft / u_acc, the accept. kernels: "reference" (oracle/_ref, the
    reference's own C build) or "port" (orc_q*_gemv). Returns (logits
    [M x V], tokens, n, seconds in the layers, in head + accept, seconds
    [inside the layers' gemv calls, inside the head's, in the accept])."""
    L = lib()
    if kernels == "reference":
        R = ref()
        f4, f6 = C.cast(R.q4_k_gemv, C.c_void_p), C.cast(R.q6_k_gemv, C.c_void_p)
    else:
        f4, f6 = C.cast(L.orc_q4_k_gemv, C.c_void_p), C.cast(L.orc_q6_k_gemv, C.c_void_p)
    x0 = _c(x0, np.float32)
    M = x0.shape[0]
    keep = []

    def ptr(a, off=0):
        keep.append(a)
        return a.ctypes.data + off

    arr = (StepLayer * max(1, len(layers)))()
    kvb, gub = NKV * (H // 256) * 144, FF * (H // 256) * 144
    for i, lw in enumerate(layers):
        arr[i] = StepLayer(ptr(lw["q"]), ptr(lw["kv"]), ptr(lw["kv"], kvb), ptr(lw["o"]), ptr(lw["gu"]),
                           ptr(lw["gu"], gub), ptr(lw["down"]), ptr(_c(lw["attn_norm"], np.float32)),
                           ptr(_c(lw["ffn_norm"], np.float32)))
    logits = np.empty((M, V), np.float32)
    tok = np.full(M, -1, np.int32)
    n = C.c_int32(-1)
    sl, sh, sg = C.c_double(), C.c_double(), np.zeros(3, np.float64)
    acc = Ld is not None
    rc = L.orc_cpu_verify_step(f4, f6, C.cast(arr, C.c_void_p), len(layers), _c(lm, np.uint8),
                               _c(out_norm, np.float32), M, H, NQ, NKV, FF, V, x0,
                               ptr(_c(Ld, np.float32)) if acc else None, ptr(_c(draft, np.int32)) if acc else None,
                               T, ptr(_c(u_acc, np.float32)) if acc else None, u_res, u_bonus, logits, tok,
                               C.byref(n), C.byref(sl), C.byref(sh), sg)
    assert rc == 0, rc
    return logits, tok, n.value, sl.value, sh.value, sg
