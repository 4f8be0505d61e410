"""Writes the committed golden fixtures of tests/golden/.

Inputs are seeded synthetic GGUF blocks and activations (inferno_hip.synth).
Expected outputs come from two sources:

* the reference's own C kernel, src/kernels/quant_kernels.c, compiled from
  source into oracle/_ref/ by `make -C oracle ref` (never copied): its
  q{4,5,6}_k_gemv / q8_0_gemv outputs on activations whose Q8_K quantization
  is exact (integers in [-127, 127] with 127 present in every 256-block), and
  its Q8_K quantization of a random row;
* the CPU oracle (oracle/liboracle.so): bit-exact dequantized blocks, the
  fp64 GEMV, and accept / greedy / tree decisions at small V.

Run from the repository root: python tests/golden/gen_golden.py
"""
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "inferno.jl_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import oracle as O  # noqa: E402
from inferno_hip import formats as F, synth  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def exact_q8k_x(rng, K):
    x = rng.integers(-127, 128, K).astype(np.float32)
    x[::256] = 127.0
    return x


def main():
    if not O.ref_available():
        sys.exit("oracle/_ref/libquant_kernels_ref.so missing: run make -C oracle ref")
    rng = np.random.default_rng(20261201)
    fx = {}
    for qt in F.QTYPES:
        name = F.NAMES[qt]
        N, K = 8, 512
        w = synth.matrix(qt, N, K, synth.stream_for(0x1F3E0000, f"golden.{name}"))
        xi = exact_q8k_x(rng, K)
        xr = rng.standard_normal(K).astype(np.float32)
        nblk = N * K // F.BLOCK_ELEMS[qt]
        fx[f"{name}_w"] = w
        fx[f"{name}_xi"] = xi
        fx[f"{name}_xr"] = xr
        fx[f"{name}_ref_gemv_xi"] = O.ref_gemv(qt, w, xi, K, N)
        fx[f"{name}_ref_gemv_xr"] = O.ref_gemv(qt, w, xr, K, N)
        fx[f"{name}_dequant"] = O.dequant(qt, w, nblk, F.BLOCK_ELEMS[qt])
        fx[f"{name}_f64_xr"] = O.gemv_f64(qt, w, xr, 1, N, K)[0]
    xq = rng.standard_normal(512).astype(np.float32)
    fx["q8k_x"] = xq
    fx["q8k_ref"] = O.ref_quantize_q8_K(xq)
    # accept cases at small V
    V, k, S = 16, 4, 64
    Lt = rng.standard_normal((S, k + 1, V)).astype(np.float32) * 2
    Ld = (Lt[:, :k] + rng.standard_normal((S, k, V)).astype(np.float32)).astype(np.float32)
    draft = rng.integers(0, V, (S, k)).astype(np.int32)
    ua = rng.random((S, k)).astype(np.float32)
    ur = rng.random(S).astype(np.float32)
    ub = rng.random(S).astype(np.float32)
    for mode in (0, 1):
        toks = np.full((S, k + 1), -1, dtype=np.int32)
        ns = np.zeros(S, dtype=np.int32)
        for s in range(S):
            t, n = O.spec_accept(Lt[s], Ld[s], draft[s], 0.8, ua[s], float(ur[s]), float(ub[s]), mode)
            toks[s, : len(t)] = t
            ns[s] = n
        fx[f"accept_mode{mode}_tok"] = toks
        fx[f"accept_mode{mode}_n"] = ns
    fx["accept_Lt"], fx["accept_Ld"], fx["accept_draft"] = Lt, Ld, draft
    fx["accept_ua"], fx["accept_ur"], fx["accept_ub"] = ua, ur, ub
    np.savez_compressed(os.path.join(OUT, "golden_v1.npz"), **fx)
    meta = {"generator": "tests/golden/gen_golden.py", "reference_kernel": "src/kernels/quant_kernels.c via oracle/_ref",
            "shapes": {"gemv": [8, 512], "accept": [S, k, V]}, "accept_temperature": 0.8}
    with open(os.path.join(OUT, "golden_v1.json"), "w") as f:
        json.dump(meta, f, indent=1)
    print("wrote", os.path.join(OUT, "golden_v1.npz"))


if __name__ == "__main__":
    main()
