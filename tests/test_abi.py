"""The C-ABI library: it loads, exports every symbol include/inferno_hip.h
declares, and its host-side argument checks and failure reporting work
without a GPU (no compute calls)."""
import ctypes as C
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "inferno_hip.h")
LIB = os.path.join(ROOT, "inferno.jl_amd", "lib", "libinferno_hip.so")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        subprocess.run(["make", "-s", "-j8", "-C", os.path.join(ROOT, "inferno.jl_amd")], check=True)
    from inferno_hip import _lib
    return _lib.load()


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_ ]*[ *]+([A-Za-z_][A-Za-z0-9_]*)\s*\(", text, re.M)
    return sorted(set(n for n in names if n not in ("if", "while")))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for n in ("q4_k_gemv", "q5_k_gemv", "q6_k_gemv", "q8_0_gemv", "ihip_gemm_q", "ihip_dequant",
              "ihip_spec_accept", "ihip_greedy_verify", "ihip_tree_accept", "ihip_softmax_stats"):
        assert n in names


def test_every_declared_symbol_is_exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    exported = set(l.split()[-1] for l in out.splitlines() if " T " in l)
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, missing
    from inferno_hip._lib import SIGNATURES
    assert set(SIGNATURES) == set(declared_functions())


def test_argument_checks_without_gpu(lib):
    nb = C.c_size_t()
    assert lib.ihip_gemm_q(12, None, None, None, 1, 1, 256, 0, None, 0, None) == -14
    buf = (C.c_uint8 * 64)()
    p = C.addressof(buf)
    p16 = (p + 15) & ~15
    assert lib.ihip_gemm_q(99, p16, p16, p16, 1, 1, 256, 0, p16, 16, None) == -22
    assert lib.ihip_gemm_q(12, p16, p16, p16, 0, 1, 256, 0, p16, 16, None) == -22
    assert lib.ihip_gemm_q(12, p16, p16, p16, 65, 1, 256, 0, p16, 16, None) == -22
    assert lib.ihip_gemm_q(12, p16, p16, p16, 1, 1, 300, 0, p16, 16, None) == -22
    assert lib.ihip_gemm_q(12, p16, p16, p16, 1, 1, 256, 3, p16, 16, None) == -22
    assert lib.ihip_gemm_q(12, p16 + 4, p16, p16, 1, 1, 256, 0, p16, 16, None) == -22
    assert b"16-byte aligned" in lib.ihip_last_error()
    assert lib.ihip_gemm_q(12, p16, p16, p16, 1, 1, 256, 0, None, 0, None) == -14
    assert lib.ihip_gemm_q(12, p16, p16, p16, 1, 1, 256, 0, p16, 1, None) == -12
    assert lib.ihip_gemm_q_ws_bytes(8, 1, 10, 96, 0, C.byref(nb)) == 0 and nb.value > 0
    assert lib.ihip_gemm_q_ws_bytes(12, 1, 10, 96, 0, C.byref(nb)) == -22
    assert lib.ihip_dequant(14, p16, p16, 100, None) == -22
    assert lib.ihip_spec_accept(None, None, None, 1, 4, 10, 1.0, None, None, None, 0, None, None, None, 0, None) == -14
    assert lib.ihip_tree_accept(p16, p16, p16, p16, 4, 10, 0.0, p16, p16, p16, p16, 1 << 20, None) == -22


def test_spec_accept_ex_checks_without_gpu(lib):
    """ihip_spec_accept_ex: filters that keep every token need no more
    workspace than ihip_spec_accept; a filtered bonus adds the sampler's;
    bad filters, workspaces and vocabularies are refused before any launch."""
    nb, nf = C.c_size_t(), C.c_size_t()
    S, k, V = 3, 4, 151936
    assert lib.ihip_spec_accept_ws_bytes(S, k, V, C.byref(nb)) == 0
    assert lib.ihip_spec_accept_ex_ws_bytes(S, k, V, 0, 1.0, 0.0, C.byref(nf)) == 0
    assert nb.value <= nf.value < nb.value + 256
    assert lib.ihip_spec_accept_ex_ws_bytes(S, k, V, V, 1.0, 0.0, C.byref(nf)) == 0 and nf.value < nb.value + 256
    sws = C.c_size_t()
    assert lib.ihip_sample_ws_bytes(S, V, C.byref(sws)) == 0
    for kw in ((40, 1.0, 0.0), (0, 0.9, 0.0), (0, 1.0, 0.1)):
        assert lib.ihip_spec_accept_ex_ws_bytes(S, k, V, *kw, C.byref(nf)) == 0
        assert nf.value >= nb.value + S * V * 4 + sws.value + S * 4
    assert lib.ihip_spec_accept_ex_ws_bytes(S, k, V, -1, 1.0, 0.0, C.byref(nf)) == -22
    buf = (C.c_uint8 * 4096)()
    p16 = (C.addressof(buf) + 15) & ~15
    args = lambda top_k, top_p, min_p, ws_bytes, V=V: (p16, p16, p16, S, k, V, 0.8, top_k, top_p, min_p, p16, p16,  # noqa: E731
                                                        p16, 1, p16, p16, p16, ws_bytes, None)
    assert lib.ihip_spec_accept_ex(*args(40, 1.0, 0.0, 1024)) == -12  # workspace short of the filtered need
    assert lib.ihip_spec_accept_ex(*args(-2, 1.0, 0.0, 1 << 40)) == -22
    assert lib.ihip_spec_accept_ex(*args(0, float("nan"), 0.0, 1 << 40)) == -22
    assert lib.ihip_spec_accept_ex(*args(40, 1.0, 0.0, 1 << 40, V=5000000)) == -22
    assert b"above 4194304" in lib.ihip_last_error()


def _dropin_child(env_extra, inner_dim, outer_dim=3):
    code = (
        "import ctypes as C, numpy as np, sys; sys.path.insert(0, %r);"
        "from inferno_hip import _lib; L = _lib.load();"
        "w = np.zeros(144 * 4 * %d, np.uint8); x = np.zeros(1024, np.float32); o = np.full(%d, 7.0, np.float32);"
        "L.q4_k_gemv(w.ctypes.data, x.ctypes.data, o.ctypes.data, None, %d, %d);"
        "print(L.ihip_last_status(), ' '.join(repr(float(v)) for v in o), L.ihip_available())"
    ) % (os.path.join(ROOT, "inferno.jl_amd"), outer_dim, outer_dim + 1, inner_dim, outer_dim)
    env = dict(os.environ, **env_extra)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=120)
    f = r.stdout.split()
    return int(f[0]), [float(v) for v in f[1:-1]], int(f[-1]), r.stderr


def test_dropin_reports_failure_without_gpu():
    """With no usable device the drop-in sets ENODEV and prints a message
    (the reference's library-missing error path), and fills out[0..N) with
    NaN so an unmodified caller, which never reads the status, sees it;
    nothing past N is touched."""
    vis = os.environ.get("HIP_VISIBLE_DEVICES")
    status, out, avail, err = _dropin_child({"HIP_VISIBLE_DEVICES": "-1" if vis is None else vis}, 256)
    if avail == 1:
        pytest.skip("a GPU is visible")
    assert status == -19
    assert all(v != v for v in out[:3]) and out[3] == 7.0
    assert "inferno_hip:" in err


def test_dropin_nan_on_bad_shape_and_kill_switch():
    """A bad inner_dim (not a multiple of 256) and the INFERNO_NO_QUANT_KERNELS
    switch also leave NaN in out[0..N), GPU or not."""
    status, out, _, err = _dropin_child({"INFERNO_NO_QUANT_KERNELS": "1"}, 256)
    assert status == -19 and all(v != v for v in out[:3]) and out[3] == 7.0
    assert "INFERNO_NO_QUANT_KERNELS" in err
    status, out, _, err = _dropin_child({}, 300)
    assert status in (-19, -22) and all(v != v for v in out[:3]) and out[3] == 7.0


def test_env_kill_switch():
    code = ("import sys; sys.path.insert(0, %r); from inferno_hip import _lib; L = _lib.load();"
            "print(L.ihip_available())") % os.path.join(ROOT, "inferno.jl_amd")
    env = dict(os.environ, INFERNO_NO_QUANT_KERNELS="1")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=120)
    assert r.stdout.strip() == "0"


def test_mlp_forward_argument_checks(lib):
    """ihip_mlp_forward validates before touching the GPU."""
    nb = C.c_size_t()
    assert lib.ihip_mlp_ws_bytes(12, 14, 5, 512, 1024, 1, None) == -14
    assert lib.ihip_mlp_ws_bytes(12, 14, 5, 512, 1024, 4, C.byref(nb)) == -22  # ACCUM is implied, not a flag
    assert lib.ihip_mlp_ws_bytes(12, 14, 5, 500, 1024, 1, C.byref(nb)) == -22  # H not a multiple of 256
    assert lib.ihip_mlp_ws_bytes(12, 14, 5, 512, 1024, 9, C.byref(nb)) == 0 and nb.value >= 5 * 2048 * 4
    buf = (C.c_uint8 * 64)()
    p16 = (C.addressof(buf) + 15) & ~15
    assert lib.ihip_mlp_forward(12, None, 14, p16, p16, None, 1e-6, 5, 512, 1024, 1, p16, 64, None) == -14
    assert lib.ihip_mlp_forward(12, p16, 14, p16, p16, None, -1.0, 5, 512, 1024, 1, p16, 64, None) == -22
    assert lib.ihip_mlp_forward(12, p16, 14, p16, p16, None, 1e-6, 5, 512, 1024, 1, p16, 64, None) == -12
    assert b"workspace" in lib.ihip_last_error()


def test_sampler_argument_checks(lib):
    """ihip_sample / ihip_sample_ex / ihip_apply_penalties validate before
    touching the GPU (any V >= 1, any logits alignment and any top_k pass
    these checks: only calls that fail here are made without a GPU)."""
    buf = (C.c_uint8 * 64)()
    p16 = (C.addressof(buf) + 15) & ~15
    assert lib.ihip_sample(None, 1, 8, 1.0, 0, 1.0, 0.0, p16, p16, None) == -14
    assert lib.ihip_sample(p16, 1, 0, 1.0, 0, 1.0, 0.0, p16, p16, None) == -22      # V
    assert lib.ihip_sample(p16, 1, 5000000, 1.0, 0, 1.0, 0.0, p16, p16, None) == -22  # V above 4194304
    assert lib.ihip_sample(p16, 0, 8, 1.0, 0, 1.0, 0.0, p16, p16, None) == -22      # rows
    assert lib.ihip_sample(p16, 1, 8, -1.0, 0, 1.0, 0.0, p16, p16, None) == -22     # temperature
    assert lib.ihip_sample(p16, 1, 8, 1.0, -1, 1.0, 0.0, p16, p16, None) == -22
    assert b"top_k" in lib.ihip_last_error()
    assert lib.ihip_sample(p16, 1, 8, 1.0, 0, float("nan"), 0.0, p16, p16, None) == -22
    # ihip_sample_ex: the same checks, plus its workspace (4104 bytes per 4096 logits of each row, and
    # 49408 bytes per row)
    nb = C.c_size_t()
    assert lib.ihip_sample_ws_bytes(2, 151936, C.byref(nb)) == 0 and nb.value == 2 * 38 * 4104 + 2 * 49408
    assert lib.ihip_sample_ws_bytes(1, 6, C.byref(nb)) == 0 and nb.value == 4104 + 49408  # any V
    assert lib.ihip_sample_ws_bytes(1, 0, C.byref(nb)) == -22
    assert lib.ihip_sample_ws_bytes(1, 8, None) == -14
    assert lib.ihip_sample_ex(p16, 1, 8, 1.0, 0, 1.0, 0.0, p16, p16, None, 1 << 20, None) == -14  # no workspace
    assert lib.ihip_sample_ex(p16, 2, 151936, 1.0, 0, 1.0, 0.0, p16, p16, p16, 8, None) == -12  # too small
    assert lib.ihip_sample_ex(p16, 1, 8, 1.0, 0, 1.0, 0.0, p16, p16, p16 + 4, 1 << 20, None) == -22  # alignment
    assert lib.ihip_sample_ex(p16, 1, 8, -1.0, 0, 1.0, 0.0, p16, p16, p16, 1 << 20, None) == -22
    assert lib.ihip_apply_penalties(None, 1, 8, p16, 1, 0, 0.5, 1.0, None) == -14
    assert lib.ihip_apply_penalties(p16, 1, 0, p16, 1, 0, 0.5, 1.0, None) == -22
    assert lib.ihip_apply_penalties(p16, 2, 8, p16, 4, 2, 0.5, 1.0, None) == -22  # stride < n_tok


def test_commit_state_argument_checks(lib):
    buf = (C.c_uint8 * 64)()
    p16 = (C.addressof(buf) + 15) & ~15
    assert lib.ihip_spec_commit_state(None, p16, 16, 16, 4, p16, 1, 0, 0, None) == -14
    assert lib.ihip_spec_commit_state(p16, p16, 6, 8, 4, p16, 1, 0, 0, None) == -22   # not whole words
    assert lib.ihip_spec_commit_state(p16, p16, 16, 8, 4, p16, 1, 0, 0, None) == -22  # snapshot stride < bytes
    assert lib.ihip_spec_advance_len(None, p16, 1, None) == -14
    assert lib.ihip_spec_advance_len(p16, p16, 0, None) == -22


def test_gemm_ex_input_checks(lib):
    """ihip_gemm_q_ex: x may be absent only when the add slices are the input
    (then [M x ldx] slices); SILU_MUL folds only in that form."""
    from inferno_hip import _lib as L
    buf = (C.c_uint8 * 64)()
    p16 = (C.addressof(buf) + 15) & ~15
    gi = L.GemmInput(None, 512, 2, None, 1e-6, None, 0, 0)
    assert lib.ihip_gemm_q_ex(12, p16, C.byref(gi), p16, 5, 256, 256, 9, p16, 64, None) == -14
    gi = L.GemmInput(p16, 512, 2, None, 1e-6, p16, 2, 5 * 512)
    assert lib.ihip_gemm_q_ex(12, p16, C.byref(gi), p16, 5, 256, 256, 9, p16, 64, None) == -22
    assert b"SILU_MUL" in lib.ihip_last_error()
    gi = L.GemmInput(None, 512, 2, None, 1e-6, p16, 2, 5 * 256)  # slice stride below M x ldx
    assert lib.ihip_gemm_q_ex(12, p16, C.byref(gi), p16, 5, 256, 256, 9, p16, 64, None) == -22
    assert b"add slices" in lib.ihip_last_error()
    gi = L.GemmInput(None, 512, 2, None, 1e-6, p16, 2, 5 * 512)  # well-formed: fails only on the workspace size
    assert lib.ihip_gemm_q_ex(12, p16, C.byref(gi), p16, 5, 256, 256, 9, p16, 64, None) == -12


def test_q8k_exports_report_failure():
    """The Q8_K exports have no status return (void / float, as the
    reference's): with the kill switch set, quantize_row_q8_K leaves d = NaN
    in every block and vec_dot_q*_K_q8_K return NaN."""
    code = (
        "import numpy as np, sys; sys.path.insert(0, %r);"
        "from inferno_hip import _lib; L = _lib.load();"
        "x = np.ones(512, np.float32); y = np.zeros(584, np.uint8);"
        "L.quantize_row_q8_K(x.ctypes.data, y.ctypes.data, 512);"
        "d = np.frombuffer(y.tobytes(), np.uint8).reshape(2, 292)[:, :4].copy().view(np.float32).ravel();"
        "w = np.zeros(210, np.uint8);"
        "r = [L.vec_dot_q4_K_q8_K(w.ctypes.data, y.ctypes.data, 1), L.vec_dot_q5_K_q8_K(w.ctypes.data, y.ctypes.data, 1),"
        "     L.vec_dot_q6_K_q8_K(w.ctypes.data, y.ctypes.data, 1)];"
        "print(' '.join(repr(float(v)) for v in list(d) + r), L.ihip_last_status())"
    ) % os.path.join(ROOT, "inferno.jl_amd")
    env = dict(os.environ, INFERNO_NO_QUANT_KERNELS="1")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=120)
    f = r.stdout.split()
    vals = [float(v) for v in f[:-1]]
    assert len(vals) == 5 and all(v != v for v in vals), r.stdout + r.stderr
    assert int(f[-1]) == -19
