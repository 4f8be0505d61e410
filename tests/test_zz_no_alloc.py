"""The allocation-free matmul entry point (ihip_gemm_q_noalloc, through the C
ABI) against ihip_gemm_q with a caller workspace: identical bits, on two
calls in a row whose second is smaller (the shared device scratch keeps the
first call's contents), in both precisions and with the accumulate flag;
shapes past the fixed scratch are rejected before any launch."""
import ctypes as C

import numpy as np
import pytest

from inferno_hip import formats as F

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ih():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import inferno_hip
    assert inferno_hip.quant_kernels_available(), inferno_hip._lib.last_error()
    return inferno_hip


def _noalloc(ih, qt, w, x, y, n, k, flags):
    import torch
    L = ih.load()
    rc = L.ihip_gemm_q_noalloc(qt, w.data_ptr(), x.data_ptr(), y.data_ptr(), x.shape[0], n, k, flags,
                               torch.cuda.current_stream().cuda_stream)
    ih._lib.check(rc)
    return y


def _with_ws(ih, qt, w, x, y, n, k, flags):
    import torch
    L = ih.load()
    nb = C.c_size_t()
    ih._lib.check(L.ihip_gemm_q_ws_bytes(qt, x.shape[0], n, k, flags, C.byref(nb)))
    ws = torch.empty(max(nb.value, 16), dtype=torch.uint8, device="cuda")
    ih._lib.check(L.ihip_gemm_q(qt, w.data_ptr(), x.data_ptr(), y.data_ptr(), x.shape[0], n, k, flags,
                                ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream))
    return y


@pytest.mark.parametrize("qt", [F.Q4_K, F.Q6_K, F.Q8_0])
def test_noalloc_matches_workspace_entry_point(ih, qt):
    import torch
    q = ih.quantized_kernels
    st = ih.synth.stream_for
    cases = [(64, 12288, 4096, ih.GEMM_HALF), (5, 4096, 2048, ih.GEMM_F32),       # large, then smaller
             (8, 151936, 2048, ih.GEMM_F32), (3, 1000, 1024, ih.GEMM_F32 | ih.GEMM_ACCUM)]
    for i, (M, N, K, fl) in enumerate(cases):
        print(f"noalloc qt={qt} case {i}: M={M} N={N} K={K} flags={fl}", flush=True)
        g = q.synth_blocks(qt, st(77, f"na.{qt}.{i}"), N * K // F.BLOCK_ELEMS[qt])
        for packed in (False, True):
            w = ih.pack_weights(qt, g, N, K) if packed else g
            f = fl | (ih.GEMM_PACKED if packed else 0)
            x = q.synth_gaussian(st(78, f"na.x.{i}"), M * K).view(M, K)
            base = q.synth_gaussian(st(79, f"na.y.{i}"), M * N).view(M, N)
            y_ref = _with_ws(ih, qt, w, x, base.clone(), N, K, f)
            y_na = _noalloc(ih, qt, w, x, base.clone(), N, K, f)
            torch.cuda.synchronize()
            assert torch.equal(y_ref, y_na), (i, packed)


def test_noalloc_rejects_oversized_shape(ih):
    """The 151936-row LM head at M = 64 needs more than the fixed scratch."""
    import torch
    L = ih.load()
    nb = C.c_size_t()
    ih._lib.check(L.ihip_gemm_q_ws_bytes(F.Q6_K, 64, 151936, 4096, ih.GEMM_HALF, C.byref(nb)))
    assert nb.value > 64 << 20
    w = torch.zeros(16, dtype=torch.uint8, device="cuda")
    x = torch.zeros(16, dtype=torch.float32, device="cuda")
    rc = L.ihip_gemm_q_noalloc(F.Q6_K, w.data_ptr(), x.data_ptr(), x.data_ptr(), 64, 151936, 4096, ih.GEMM_HALF,
                               None)
    assert rc == -12 and b"scratch" in L.ihip_last_error()
    # a valid call right after still works
    q = ih.quantized_kernels
    g = q.synth_blocks(F.Q4_K, 5, 64 * 4)
    xx = q.synth_gaussian(6, 2 * 1024).view(2, 1024)
    y1 = _with_ws(ih, F.Q4_K, g, xx, torch.empty(2, 64, device="cuda"), 64, 1024, ih.GEMM_F32)
    y2 = _noalloc(ih, F.Q4_K, g, xx, torch.empty(2, 64, device="cuda"), 64, 1024, ih.GEMM_F32)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)


def test_noalloc_under_graph_capture(ih):
    """ihip_gemm_q_noalloc captured into a HIP graph (its scratch address
    looked up by ihip_init beforehand, so the capture makes no lookup) and
    replayed: every replay, with eager work and synchronisations between,
    gives ihip_gemm_q's bits; then a smaller eager call after the replays."""
    import torch
    L = ih.load()
    ih._lib.check(L.ihip_init(torch.cuda.current_device()))
    q = ih.quantized_kernels
    st = ih.synth.stream_for
    N, K, M = 4096, 4096, 5
    w = ih.pack_weights(F.Q4_K, q.synth_blocks(F.Q4_K, st(81, "na.g.w"), N * K // 256), N, K)
    x = q.synth_gaussian(st(81, "na.g.x"), M * K).view(M, K)
    fl = ih.GEMM_F32 | ih.GEMM_PACKED
    y_ref = _with_ws(ih, F.Q4_K, w, x, torch.empty(M, N, device="cuda"), N, K, fl)
    y = torch.empty(M, N, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _noalloc(ih, F.Q4_K, w, x, y, N, K, fl)  # warm-up outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        ih._lib.check(L.ihip_gemm_q_noalloc(F.Q4_K, w.data_ptr(), x.data_ptr(), y.data_ptr(), M, N, K, fl,
                                            s.cuda_stream))
    for r in range(4):
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref), r
        _with_ws(ih, F.Q4_K, w, x, torch.empty(M, N, device="cuda"), N, K, fl)  # eager work between replays
    x2 = x[:2].contiguous()
    y2 = _noalloc(ih, F.Q4_K, w, x2, torch.empty(2, N, device="cuda"), N, K, fl)
    y2_ref = _with_ws(ih, F.Q4_K, w, x2, torch.empty(2, N, device="cuda"), N, K, fl)
    torch.cuda.synchronize()
    assert torch.equal(y2, y2_ref)
