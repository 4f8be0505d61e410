"""GPU: the LDS-staged matmul kernel, the one that takes packed weights of
2 GiB and more and outputs past 32-bit offsets (every smaller call takes the
streaming or several-tile kernels). The plan reads its kernel choice once per
process, so the checks run in one child process with IHIP_STREAM=0, which
sends every call to the LDS kernel. Same bars as the other matmul paths
against the oracle's fp64 product of the dequantized weights
(src/QuantizedKernels.jl:55-190): rel-L2 1e-5 fp32-accurate, 1e-2 half
(with the tighter sanity bound the fp16 operands reach); the deferred
partials folded into the next input stage equal accumulate-then-matmul bit
for bit."""
import os
import subprocess
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-5
TOL_HALF = 1e-2
SANITY_HALF = 2e-3


def test_lds_kernel_parity():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    env = dict(os.environ, IHIP_STREAM="0")
    r = subprocess.run([sys.executable, "-u", os.path.abspath(__file__)], capture_output=True, text=True, env=env,
                       timeout=110)
    print(r.stdout[-4000:], r.stderr[-4000:], flush=True)
    assert r.returncode == 0
    assert "lds kernel ok" in r.stdout


def _child():
    import torch
    from _util import rel_l2
    import oracle as O
    import inferno_hip as ih
    from inferno_hip import formats as F
    from inferno_hip import synth

    assert ih.quant_kernels_available(), ih._lib.last_error()

    def dev(a):
        return torch.from_numpy(np.ascontiguousarray(a)).cuda()

    N = 200  # the last 64-row group is partly past N
    for qt in F.QTYPES:
        for K in (768, 2560):
            rng = np.random.default_rng(5 * K + qt)
            w = synth.matrix(qt, N, K, synth.stream_for(N + K, f"lds{qt}"))
            wd = dev(w)
            wp = ih.pack_weights(qt, wd, N, K)
            for M in (1, 5, 16, 37, 64):
                x = rng.standard_normal((M, K)).astype(np.float32)
                ref = O.gemv_f64(qt, w, x, M, N, K)
                for name, wt, lay in (("gguf", wd, 0), ("packed", wp, ih.GEMM_PACKED)):
                    for mode, fl, bar in (("f32", ih.GEMM_F32, TOL_F32), ("half", ih.GEMM_HALF, SANITY_HALF)):
                        got = ih.gemm_q(qt, wt, dev(x), N, K, flags=fl | lay).cpu().numpy()
                        err = rel_l2(got, ref)
                        print(f"{F.NAMES[qt]} K={K} M={M} {name} {mode} rel-L2={err:.3e}", flush=True)
                        assert err <= bar, (qt, K, M, name, mode, err)
                y0 = torch.randn(M, N, device="cuda")
                y = y0.clone()
                ih.gemm_q(qt, wp, dev(x), N, K, flags=ih.GEMM_HALF | ih.GEMM_PACKED | ih.GEMM_ACCUM, out=y)
                assert rel_l2((y - y0).cpu().numpy(), ref) <= SANITY_HALF, (qt, K, M)

    # RMSNorm input stage and a deferred Q6_K down projection (K-sliced)
    # folded into the next matmul's residual add
    H, FF, N2 = 512, 2048, 96
    rng = np.random.default_rng(9)
    wdn = synth.matrix(F.Q6_K, H, FF, synth.stream_for(3, "lds_down"))
    w2 = synth.matrix(F.Q4_K, N2, H, synth.stream_for(4, "lds_next"))
    pd, p2 = ih.pack_weights(F.Q6_K, dev(wdn), H, FF), ih.pack_weights(F.Q4_K, dev(w2), N2, H)
    nw = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    for M, fl in ((5, ih.GEMM_F32 | ih.GEMM_PACKED), (64, ih.GEMM_HALF | ih.GEMM_PACKED)):
        bar = TOL_F32 if fl & ih.GEMM_F32 else SANITY_HALF
        h = dev(rng.standard_normal((M, FF)).astype(np.float32))
        x0 = dev((2.0 * rng.standard_normal((M, H))).astype(np.float32))
        xr = x0.clone()
        ih.gemm_q(F.Q6_K, pd, h, H, FF, flags=fl | ih.GEMM_ACCUM, out=xr)
        yr = ih.gemm_q_ex(F.Q4_K, p2, xr, N2, H, act=ih.ACT_RMSNORM, norm_w=dev(nw), flags=fl)
        ws = torch.empty(ih.quantized_kernels.gemm_ws_bytes(F.Q6_K, M, H, FF, fl), dtype=torch.uint8,
                         device="cuda")
        ih.gemm_q_ex(F.Q6_K, pd, h, H, FF, flags=fl | ih.GEMM_DEFER, ws=ws)
        parts = ih.gemm_partials(F.Q6_K, M, H, FF, fl, ws)
        assert parts[1] >= 2, parts
        xf = x0.clone()
        yf = ih.gemm_q_ex(F.Q4_K, p2, xf, N2, H, act=ih.ACT_RMSNORM, norm_w=dev(nw), flags=fl, add=parts)
        assert torch.equal(xf, xr), M
        assert torch.equal(yf, yr), M
        xref = O.gemv_f64(F.Q6_K, wdn, h.cpu().numpy(), M, H, FF) + x0.cpu().numpy()
        assert rel_l2(xf.cpu().numpy(), xref) <= bar, M
        n = np.stack([O.rmsnorm(r, 1e-6, nw) for r in xf.cpu().numpy()]).astype(np.float32)
        err = rel_l2(yf.cpu().numpy(), O.gemv_f64(F.Q4_K, w2, n, M, N2, H))
        print(f"rmsnorm + fold M={M} rel-L2={err:.3e}", flush=True)
        assert err <= bar, M
    torch.cuda.synchronize()
    print("lds kernel ok", flush=True)


if __name__ == "__main__":
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    for p in (os.path.join(root, "inferno.jl_amd"), os.path.join(root, "oracle"), root,
              os.path.dirname(os.path.abspath(__file__))):
        sys.path.insert(0, p)
    _child()
