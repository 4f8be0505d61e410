"""Pins of the CPU oracle's dequantization and GEMV (no GPU).

The oracle restates src/QuantsCPU.jl:491-658 and src/kernels/quant_kernels.c.
It is checked here against:
* golden vectors written by tests/golden/gen_golden.py from the reference's
  own C kernel (compiled from source into oracle/_ref), on activations whose
  Q8_K quantization is exact, so the reference's integer path computes the
  same product as the dequantize-then-dot formulas;
* the reference kernel live, when oracle/_ref is built;
* brute force over every 6-bit scale/min value and quant value, IEEE fp16
  conversion of all 65536 bit patterns, and closed-form special cases.
"""
import os

import numpy as np
import pytest

import oracle as O
from inferno_hip import formats as F, synth

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_v1.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


@pytest.mark.parametrize("qt", F.QTYPES)
def test_dequant_formulas_match_reference_kernel(gold, qt):
    """With Q8_K-exact activations the reference C kernel's integer dot equals
    sum(dequant(W) * x) up to its fp32 accumulation: pins the oracle's block
    layouts and scale/min unpacking against the reference's own code."""
    name = F.NAMES[qt]
    w, xi = gold[f"{name}_w"], gold[f"{name}_xi"]
    y = O.gemv_f64(qt, w, xi, 1, 8, 512)[0]
    assert rel(y, gold[f"{name}_ref_gemv_xi"]) < 1e-6


@pytest.mark.parametrize("qt", F.QTYPES)
def test_q8k_port_bit_exact_vs_reference(gold, qt):
    """The oracle's restatement of the reference fast path (Q8_K quantize,
    integer dot, 8-lane fp32 accumulation) reproduces the reference's
    outputs bit for bit on random activations."""
    name = F.NAMES[qt]
    out = O.gemv_q8k(qt, gold[f"{name}_w"], gold[f"{name}_xr"], 512, 8)
    assert np.array_equal(out.view(np.uint32), gold[f"{name}_ref_gemv_xr"].view(np.uint32))


def test_quantize_q8k_bit_exact(gold):
    assert np.array_equal(O.quantize_q8_K(gold["q8k_x"]), gold["q8k_ref"])


@pytest.mark.parametrize("qt", F.QTYPES)
def test_dequant_regression(gold, qt):
    name = F.NAMES[qt]
    nblk = 8 * 512 // F.BLOCK_ELEMS[qt]
    got = O.dequant(qt, gold[f"{name}_w"], nblk, F.BLOCK_ELEMS[qt])
    assert np.array_equal(got.view(np.uint32), gold[f"{name}_dequant"].view(np.uint32))


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("qt", F.QTYPES)
def test_live_reference_kernel(qt):
    rng = np.random.default_rng(qt)
    for N, K in ((5, 256), (33, 1024), (70, 2048)):
        w = synth.matrix(qt, N, K, synth.stream_for(K + N, "live"))
        xi = rng.integers(-127, 128, K).astype(np.float32)
        xi[::256] = -127.0
        assert rel(O.gemv_f64(qt, w, xi, 1, N, K)[0], O.ref_gemv(qt, w, xi, K, N)) < 1e-6
        xr = rng.standard_normal(K).astype(np.float32)
        a = O.gemv_q8k(qt, w, xr, K, N)
        b = O.ref_gemv(qt, w, xr, K, N)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        # the reference's Q8_K path is not fp32-accurate: its error against
        # the exact product is what the fp32-accurate GPU path removes
        assert rel(b, O.gemv_f64(qt, w, xr, 1, N, K)[0]) > 1e-5 or qt == F.Q8_0


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("qt", [F.Q4_K, F.Q5_K, F.Q6_K])
def test_live_reference_vec_dot(qt):
    """orc_vec_dot_* against the reference's exported vec_dot_q*_K_q8_K on
    single rows (the symbols QuantizedKernels binds at src/QuantizedKernels.jl
    :157-175), bit for bit."""
    rng = np.random.default_rng(100 + qt)
    for nb in (1, 3, 16):
        w = synth.blocks(qt, nb, synth.stream_for(qt, f"vdref{nb}"))
        for scale in (1.0, 1e-3, 50.0):
            q8 = O.ref_quantize_q8_K((rng.standard_normal(256 * nb) * scale).astype(np.float32))
            a = np.float32(O.vec_dot(qt, w, q8, nb))
            b = np.float32(O.ref_vec_dot(qt, w, q8, nb))
            assert a.view(np.uint32) == b.view(np.uint32), (nb, scale, a, b)


def test_fp16_conversion_all_patterns():
    bits = np.arange(65536, dtype=np.uint32)
    ref = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    lib = O.lib()
    got = np.array([lib.orc_fp16_to_fp32(int(b)) for b in range(0, 65536, 1)], dtype=np.float32)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


def test_scale_pack_unpack_brute_force():
    """Every 6-bit value in every scale/min slot round-trips through the
    pack (generator) and the unpack (src/QuantsCPU.jl:501-513)."""
    vals = np.arange(64, dtype=np.uint8)
    for slot in range(8):
        sc = np.zeros((64, 8), np.uint8)
        m = np.zeros((64, 8), np.uint8)
        sc[:, slot] = vals
        m[:, slot] = vals[::-1]
        s2, m2 = synth.unpack_scales_k4(synth.pack_scales_k4(sc, m))
        assert np.array_equal(s2, sc) and np.array_equal(m2, m)


def _block_k(qt, d, dmin, sc, m, q):
    """A Q4_K/Q5_K block with given fields; q: 256 ints in 0..15 (Q4_K) or 0..31."""
    bb = F.BLOCK_BYTES[qt]
    b = np.zeros(bb, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:4] = np.array([dmin], np.float16).view(np.uint8)
    b[4:16] = synth.pack_scales_k4(np.array([sc], np.uint8), np.array([m], np.uint8))[0]
    qs_off = 16 if qt == F.Q4_K else 48
    for j in range(4):
        for l in range(32):
            lo, hi = q[64 * j + l], q[64 * j + 32 + l]
            b[qs_off + 32 * j + l] = (lo & 15) | ((hi & 15) << 4)
            if qt == F.Q5_K:
                b[16 + l] |= ((lo >> 4) & 1) << (2 * j)
                b[16 + l] |= ((hi >> 4) & 1) << (2 * j + 1)
    return b


@pytest.mark.parametrize("qt", [F.Q4_K, F.Q5_K])
def test_k4_closed_forms(qt):
    rng = np.random.default_rng(0)
    qmax = 15 if qt == F.Q4_K else 31
    q = rng.integers(0, qmax + 1, 256)
    # d = 1, every sc = 1, m = 0: w = q exactly
    w = O.dequant(qt, _block_k(qt, 1.0, 0.0, [1] * 8, [0] * 8, q), 1, 256)
    assert np.array_equal(w, q.astype(np.float32))
    # d = 0, dmin = 1: w = -m of the element's sub-block, for every m value
    for trial in range(8):
        m = rng.integers(0, 64, 8)
        w = O.dequant(qt, _block_k(qt, 0.0, 1.0, [0] * 8, m, q), 1, 256)
        assert np.array_equal(w, -np.repeat(m, 32).astype(np.float32))
    # d = 1, dmin = 0, all q = 1: w = sc of the element's sub-block
    sc = np.arange(8) * 9 % 64
    w = O.dequant(qt, _block_k(qt, 1.0, 0.0, sc, [0] * 8, np.ones(256, int)), 1, 256)
    assert np.array_equal(w, np.repeat(sc, 32).astype(np.float32))
    # d = dmin = 0: +0.0 everywhere
    w = O.dequant(qt, _block_k(qt, 0.0, 0.0, sc, sc, q), 1, 256)
    assert np.array_equal(w.view(np.uint32), np.zeros(256, np.uint32))


def test_q6k_closed_forms():
    rng = np.random.default_rng(1)
    q = rng.integers(0, 64, 256)
    b = np.zeros(210, np.uint8)
    for n in range(2):
        for l in range(32):
            q1, q2, q3, q4 = (q[128 * n + l + 32 * i] for i in range(4))
            b[64 * n + l] = (q1 & 15) | ((q3 & 15) << 4)
            b[64 * n + l + 32] = (q2 & 15) | ((q4 & 15) << 4)
            b[128 + 32 * n + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    b[192:208] = np.ones(16, np.int8).view(np.uint8)
    b[208:210] = np.array([1.0], np.float16).view(np.uint8)
    assert np.array_equal(O.dequant(F.Q6_K, b, 1, 256), (q - 32).astype(np.float32))
    # scale of element i is sc[i // 16]
    sc = rng.integers(-128, 128, 16).astype(np.int8)
    b[192:208] = sc.view(np.uint8)
    assert np.array_equal(O.dequant(F.Q6_K, b, 1, 256), (q - 32) * np.repeat(sc.astype(np.float32), 16))


def test_q8_0_closed_form():
    q = np.arange(-127, 128, 8)[:32].astype(np.int8)
    b = np.zeros(34, np.uint8)
    b[0:2] = np.array([1.0], np.float16).view(np.uint8)
    b[2:] = q.view(np.uint8)
    assert np.array_equal(O.dequant(F.Q8_0, b, 1, 32), q.astype(np.float32))


@pytest.mark.parametrize("qt", F.QTYPES)
def test_gemv_invariants(qt):
    N, K = 24, 512
    w = synth.matrix(qt, N, K, synth.stream_for(3, "inv"))
    full = O.dequant(qt, w, N * K // F.BLOCK_ELEMS[qt], F.BLOCK_ELEMS[qt]).reshape(N, K)
    for k in (0, 1, 255, 256, 511):
        e = np.zeros(K, np.float32)
        e[k] = 1.0
        assert np.array_equal(O.gemv_f64(qt, w, e, 1, N, K)[0], full[:, k].astype(np.float64))
    rng = np.random.default_rng(qt)
    x = rng.standard_normal((3, K)).astype(np.float32)
    y = O.gemv_f64(qt, w, x, 3, N, K)
    assert rel(O.gemv_f64(qt, w, (x[0] + 2 * x[1]).astype(np.float32), 1, N, K)[0], y[0] + 2 * y[1]) < 1e-6
    assert rel(O.gemv_seq_f32(qt, w, x, 3, N, K), y) < 1e-6
    assert np.allclose(y, x.astype(np.float64) @ full.T.astype(np.float64), rtol=1e-12, atol=1e-9)


@pytest.mark.parametrize("kernels", ["port", "reference"])
def test_cpu_verify_step_driver(kernels):
    """The CPU baseline's C step driver (orc_cpu_verify_step) computes the
    step it times: its logits equal the same step composed in numpy from
    the pinned pieces (orc_gemv_q8k, bit-exact to the reference kernel;
    orc_rmsnorm; silu; token-major order of forward_cpu!), and its accept
    equals orc_spec_accept on those logits."""
    if kernels == "reference" and not O.ref_available():
        pytest.skip("oracle/_ref not built (no reference tree)")
    H, NQ, NKV, FF, V, M, nl = 512, 512, 256, 768, 1000, 3, 2
    st = lambda n: synth.stream_for(0x5EED, n)  # noqa: E731
    layers = []
    for i in range(nl):
        layers.append({"q": synth.matrix(F.Q4_K, NQ, H, st(f"q{i}")), "kv": synth.matrix(F.Q4_K, 2 * NKV, H, st(f"kv{i}")),
                       "o": synth.matrix(F.Q4_K, H, NQ, st(f"o{i}")), "gu": synth.matrix(F.Q4_K, 2 * FF, H, st(f"gu{i}")),
                       "down": synth.matrix(F.Q6_K, H, FF, st(f"d{i}")),
                       "attn_norm": 1 + 0.1 * synth.gaussian(st(f"an{i}"), H),
                       "ffn_norm": 1 + 0.1 * synth.gaussian(st(f"fn{i}"), H)})
    lm = synth.matrix(F.Q6_K, V, H, st("lm"))
    on = 1 + 0.1 * synth.gaussian(st("on"), H)
    x0 = synth.gaussian(st("x0"), M * H).reshape(M, H)
    rng = np.random.default_rng(3)
    Ld = rng.standard_normal((M - 1, V)).astype(np.float32)
    draft = np.array([5, 17], np.int32)
    ua = np.zeros(M - 1, np.float32)
    logits, tok, n, sl, sh, sg = O.cpu_verify_step(layers, lm, on, x0, H, NQ, NKV, FF, V, Ld, draft, 0.8, ua, 0.5,
                                                   0.25, kernels=kernels)
    assert sl > 0 and sh > 0 and 0 < sg[0] <= sl and 0 < sg[1] and sg[1] + sg[2] <= sh
    g = lambda qt, w, v, K, N: O.gemv_q8k(qt, w, v, K, N, 1)  # noqa: E731
    want = np.empty((M, V), np.float32)
    with np.errstate(over="ignore"):  # exp(-g) of very negative gates: silu -> -0, as in fp32 C
        for m in range(M):
            x = x0[m].copy()
            for lw in layers:
                h = O.rmsnorm(x, w=lw["attn_norm"])
                q = g(F.Q4_K, lw["q"], h, H, NQ)
                x = x + g(F.Q4_K, lw["o"], q, NQ, H)
                h = O.rmsnorm(x, w=lw["ffn_norm"])
                gu = g(F.Q4_K, lw["gu"], h, H, 2 * FF)
                a = (gu[:FF] / (np.float32(1) + np.exp(-gu[:FF])) * gu[FF:]).astype(np.float32)
                x = x + g(F.Q6_K, lw["down"], a, FF, H)
            want[m] = g(F.Q6_K, lm, O.rmsnorm(x, w=on), H, V)
    assert rel(logits, want) < 1e-5
    rt, rn = O.spec_accept(logits, Ld, draft, 0.8, ua, 0.5, 0.25, 0)
    assert n == rn and tok[: len(rt)].tolist() == rt.tolist()
