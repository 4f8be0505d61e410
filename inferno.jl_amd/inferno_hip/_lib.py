"""Loader for lib/libinferno_hip.so (the C ABI of include/inferno_hip.h).

There is no CPU fallback: if the library is missing or cannot start on a
gfx950 device, calls raise.
"""
from __future__ import annotations

import ctypes as C
import os

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("INFERNO_HIP_LIB", os.path.join(PKG_ROOT, "lib", "libinferno_hip.so"))
HEADER_PATH = os.path.join(os.path.dirname(PKG_ROOT), "include", "inferno_hip.h")

IHIP_OK = 0
STATUS_NAMES = {0: "OK", -14: "EFAULT", -22: "EINVAL", -12: "ENOMEM", -19: "ENODEV", -1000: "EHIP"}

_vp, _i, _i64, _u64, _f, _sz = C.c_void_p, C.c_int, C.c_int64, C.c_uint64, C.c_float, C.c_size_t

# name -> (restype, argtypes)
SIGNATURES = {
    "ihip_last_error": (C.c_char_p, []),
    "ihip_last_status": (_i, []),
    "ihip_init": (_i, [_i]),
    "ihip_available": (_i, []),
    "ihip_weight_cache_clear": (None, []),
    "q4_k_gemv": (None, [_vp, _vp, _vp, _vp, _i, _i]),
    "q5_k_gemv": (None, [_vp, _vp, _vp, _vp, _i, _i]),
    "q6_k_gemv": (None, [_vp, _vp, _vp, _vp, _i, _i]),
    "q8_0_gemv": (None, [_vp, _vp, _vp, _i, _i]),
    "quantize_row_q8_K": (None, [_vp, _vp, _i64]),
    "vec_dot_q4_K_q8_K": (C.c_float, [_vp, _vp, _i]),
    "vec_dot_q5_K_q8_K": (C.c_float, [_vp, _vp, _i]),
    "vec_dot_q6_K_q8_K": (C.c_float, [_vp, _vp, _i]),
    "ihip_gemm_q_ws_bytes": (_i, [_i, _i, _i, _i, _i, C.POINTER(_sz)]),
    "ihip_gemm_q": (_i, [_i, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "ihip_gemm_q_ex": (_i, [_i, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "ihip_gemm_q_noalloc": (_i, [_i, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "ihip_gemm_q_chain": (_i, [_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "ihip_chain_operand_bytes": (_sz, [_i]),
    "ihip_pack_weights_gated": (_i, [_i, _vp, _vp, _i, _i, _vp]),
    "ihip_gemm_q_partials": (_i, [_i, _i, _i, _i, _i, _vp, C.POINTER(_vp), C.POINTER(_i), C.POINTER(_i64)]),
    "ihip_mlp_ws_bytes": (_i, [_i, _i, _i, _i, _i, _i, C.POINTER(_sz)]),
    "ihip_mlp_forward": (_i, [_i, _vp, _i, _vp, _vp, _vp, _f, _i, _i, _i, _i, _vp, _sz, _vp]),
    "ihip_packed_bytes": (_i, [_i, _i, _i, C.POINTER(_sz)]),
    "ihip_pack_weights": (_i, [_i, _vp, _vp, _i, _i, _vp]),
    "ihip_dequant": (_i, [_i, _vp, _vp, _i64, _vp]),
    "ihip_rmsnorm": (_i, [_vp, _vp, _vp, _i, _i, _f, _vp]),
    "ihip_silu_mul": (_i, [_vp, _i, _i, _vp, _vp]),
    "ihip_add": (_i, [_vp, _vp, _i64, _vp]),
    "ihip_accept_ws_bytes": (_i, [_i, _i, C.POINTER(_sz)]),
    "ihip_softmax_stats": (_i, [_vp, _i, _i, _f, _vp, _vp, _vp, _sz, _vp]),
    "ihip_spec_accept_ws_bytes": (_i, [_i, _i, _i, C.POINTER(_sz)]),
    "ihip_spec_accept": (_i, [_vp, _vp, _vp, _i, _i, _i, _f, _vp, _vp, _vp, _i, _vp, _vp, _vp, _sz, _vp]),
    "ihip_spec_accept_ex_ws_bytes": (_i, [_i, _i, _i, _i, _f, _f, C.POINTER(_sz)]),
    "ihip_spec_accept_ex": (_i, [_vp, _vp, _vp, _i, _i, _i, _f, _i, _f, _f, _vp, _vp, _vp, _i, _vp, _vp, _vp, _sz,
                                 _vp]),
    "ihip_greedy_verify": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp, _sz, _vp]),
    "ihip_tree_accept": (_i, [_vp, _vp, _vp, _vp, _i, _i, _f, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ihip_spec_commit_state": (_i, [_vp, _vp, _sz, _i64, _i, _vp, _i, _i64, _i64, _vp]),
    "ihip_spec_advance_len": (_i, [_vp, _vp, _i, _vp]),
    "ihip_sample": (_i, [_vp, _i, _i, _f, _i, _f, _f, _vp, _vp, _vp]),
    "ihip_sample_ws_bytes": (_i, [_i, _i, C.POINTER(_sz)]),
    "ihip_sample_ex": (_i, [_vp, _i, _i, _f, _i, _f, _f, _vp, _vp, _vp, _sz, _vp]),
    "ihip_apply_penalties": (_i, [_vp, _i, _i, _vp, _i, _i64, _f, _f, _vp]),
    "ihip_gguf_open": (_i, [C.c_char_p, C.POINTER(_vp)]),
    "ihip_gguf_close": (_i, [_vp]),
    "ihip_gguf_info": (_i, [_vp, C.POINTER(C.c_uint32), C.POINTER(_i64), C.POINTER(_i64), C.POINTER(_u64),
                            C.POINTER(_u64)]),
    "ihip_gguf_tensor": (_i, [_vp, _i64, C.POINTER(C.c_char_p), C.POINTER(_i), C.POINTER(_i), C.POINTER(_i64),
                              C.POINTER(_u64), C.POINTER(_u64)]),
    "ihip_gguf_find_tensor": (_i64, [_vp, C.c_char_p]),
    "ihip_gguf_find_key": (_i64, [_vp, C.c_char_p]),
    "ihip_gguf_kv": (_i, [_vp, _i64, C.POINTER(C.c_char_p), C.POINTER(_i), C.POINTER(_i), C.POINTER(_u64)]),
    "ihip_gguf_kv_number": (_i, [_vp, _i64, _u64, C.POINTER(_i64), C.POINTER(C.c_double)]),
    "ihip_gguf_kv_string": (_i, [_vp, _i64, _u64, C.POINTER(_vp), C.POINTER(_u64)]),
    "ihip_gguf_tensor_data": (_vp, [_vp, _i64]),
    "ihip_gguf_upload": (_i, [_vp, _i64, _vp, _sz, _i, _vp]),
    "ihip_synth_blocks": (_i, [_i, _u64, _i64, _i64, _vp, _vp]),
    "ihip_synth_gaussian": (_i, [_u64, _i64, _f, _vp, _vp, _vp]),
    "ihip_stream_read": (_i, [_vp, _sz, _vp, _vp]),
}


class GemmInput(C.Structure):
    """struct ihip_gemm_input"""
    _fields_ = [("x", _vp), ("ldx", _i), ("act", _i), ("norm_w", _vp), ("eps", _f), ("add", _vp),
                ("n_add", _i), ("add_stride", _i64)]


class ChainIn(C.Structure):
    """struct ihip_chain_in"""
    _fields_ = [("operand", _vp), ("tile_sum", _vp), ("sum_stride", _i), ("tiles_per_unit", _i),
                ("tile_ssq", _vp), ("ssq_tiles", _i), ("eps", _f)]


class ChainOut(C.Structure):
    """struct ihip_chain_out"""
    _fields_ = [("epi", _i), ("y", _vp), ("ldy", _i), ("norm_w", _vp), ("consumer_qtype", _i), ("operand", _vp),
                ("tile_sum", _vp), ("sum_stride", _i), ("tile_ssq", _vp), ("stat_rows", _i)]


class HipError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"inferno_hip {STATUS_NAMES.get(status, status)}: {msg}")
        self.status = status


_lib = None


def load(path: str | None = None):
    """Load the shared library and bind every declared symbol (raises if absent)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise OSError(f"libinferno_hip.so not built at {p}: run __graft_entry__.build() or make -C inferno.jl_amd")
    L = C.CDLL(p)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = L
    return L


def check(rc: int) -> None:
    if rc != IHIP_OK:
        raise HipError(rc, load().ihip_last_error().decode(errors="replace"))


def last_status() -> int:
    return load().ihip_last_status()


def last_error() -> str:
    return load().ihip_last_error().decode(errors="replace")
