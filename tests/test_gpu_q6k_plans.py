"""GPU parity of the one-token-tile Q6_K plan for long K (K a multiple of
3072, at least 6144: 4 waves of 3 units, one wave per SIMD, K-slices of 12
units): plain calls (slices reduced), deferred calls (the partials summed
here), accumulation and the GGUF layout, against the CPU oracle, with rows
that end inside a tile. K = 12288 (down) runs in the full-shape tests."""
import numpy as np
import pytest

from _util import rel_l2

import oracle as O
from inferno_hip import formats as F
from inferno_hip import synth

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-5


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


@pytest.mark.parametrize("K", [9216, 24576])
def test_q6k_long_k_plan(ih, K):
    import torch
    N = 400  # 25 tiles: not a multiple of the 4 tiles a workgroup takes
    q = ih.quantized_kernels
    w = synth.matrix(F.Q6_K, N, K, synth.stream_for(K, "q6plan"))
    wg = _dev(w)
    wp = ih.pack_weights(F.Q6_K, wg, N, K)
    rng = np.random.default_rng(K)
    f32p = ih.GEMM_F32 | ih.GEMM_PACKED
    for M in (1, 3, 8):
        x = rng.standard_normal((M, K)).astype(np.float32)
        xd = _dev(x)
        ref = O.gemv_f64(F.Q6_K, w, x, M, N, K)
        y = ih.gemm_q_ex(F.Q6_K, wp, xd, N, K, flags=f32p)
        err = rel_l2(y.cpu().numpy(), ref)
        print(f"Q6_K N={N} K={K} M={M} packed rel-L2={err:.3e}", flush=True)
        assert err <= TOL_F32, (M, err)
        # GGUF layout: the same plan and summation order, the same bits
        y2 = ih.gemm_q_ex(F.Q6_K, wg, xd, N, K, flags=ih.GEMM_F32)
        assert torch.equal(y, y2), M
        # deferred: K / 3072 slices of partials
        ws = torch.empty(q.gemm_ws_bytes(F.Q6_K, M, N, K, f32p), dtype=torch.uint8, device="cuda")
        ih.gemm_q_ex(F.Q6_K, wp, xd, N, K, flags=f32p | ih.GEMM_DEFER, ws=ws)
        torch.cuda.synchronize()
        ptr, ns, stride = ih.gemm_partials(F.Q6_K, M, N, K, f32p, ws)
        assert ns == K // 3072, ns
        off = (ptr - ws.data_ptr()) // 4
        sl = ws.view(torch.float32)[off: off + ns * stride].view(ns, stride)[:, : M * N].reshape(ns, M, N)
        part = sl.cpu().numpy().astype(np.float64).sum(axis=0)
        assert rel_l2(part, ref) <= TOL_F32
        # accumulate into an existing output
        y0 = rng.standard_normal((M, N)).astype(np.float32)
        ya = _dev(y0)
        ih.gemm_q_ex(F.Q6_K, wp, xd, N, K, flags=f32p | ih.GEMM_ACCUM, out=ya)
        assert rel_l2(ya.cpu().numpy(), y0.astype(np.float64) + ref) <= TOL_F32
