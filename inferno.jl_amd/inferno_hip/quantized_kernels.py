"""Host mirror of the reference's QuantizedKernels module
(src/QuantizedKernels.jl:12-177) over the gfx950 library.

Same names (Julia's `q4_k_gemv!` is `q4_k_gemv_` here), argument order and
meaning: `out`, `weight_data` (GGUF row-major block bytes), `x`, `inner_dim`
(K) and `outer_dim` (N); `out[r] = sum_k W[r,k] x[k]`. The reference raises
`error("Quantized C kernel not available")` when its library is missing
(src/QuantizedKernels.jl:84); these raise HipError or OSError the same way,
and there is no CPU fallback. INFERNO_NO_QUANT_KERNELS disables the kernels
as in the reference (src/QuantizedKernels.jl:26-32).

The device-resident form (`gemm_q`) is the batched path the verify step uses:
all M verify tokens against one pass over the weights.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from .formats import BLOCK_BYTES, BLOCK_ELEMS, Q4_K, Q5_K, Q6_K, Q8_0, NAMES

GEMM_AUTO, GEMM_F32, GEMM_HALF, GEMM_ACCUM, GEMM_PACKED, GEMM_REUSE, GEMM_DEFER = 0, 1, 2, 4, 8, 16, 32
GEMM_SUM_OUT = 64
ACT_PLAIN, ACT_RMSNORM, ACT_SILU_MUL = 0, 1, 2


def quant_kernels_available() -> bool:
    """src/QuantizedKernels.jl:49-50: library present, gfx950 found, not disabled."""
    try:
        return bool(_lib.load().ihip_available())
    except OSError:
        return False


def _host_gemv(sym: str, qtype: int, out, weight_data, x, inner_dim: int, outer_dim: int, with_q8: bool):
    L = _lib.load()
    out = np.asarray(out)
    if out.dtype != np.float32 or not out.flags.c_contiguous or out.size < outer_dim:
        raise ValueError("out must be a contiguous float32 array of length >= outer_dim")
    w = np.ascontiguousarray(weight_data, dtype=np.uint8)
    xv = np.ascontiguousarray(x, dtype=np.float32)
    if xv.size < inner_dim:
        raise ValueError("x shorter than inner_dim")
    need = outer_dim * (inner_dim // BLOCK_ELEMS[qtype]) * BLOCK_BYTES[qtype]
    if inner_dim % BLOCK_ELEMS[qtype] or w.size < need:
        raise ValueError(f"{NAMES[qtype]} weight: inner_dim={inner_dim} outer_dim={outer_dim} needs {need} bytes")
    fn = getattr(L, sym)
    if with_q8:
        fn(w.ctypes.data, xv.ctypes.data, out.ctypes.data, None, inner_dim, outer_dim)
    else:
        fn(w.ctypes.data, xv.ctypes.data, out.ctypes.data, inner_dim, outer_dim)
    _lib.check(L.ihip_last_status())
    return out


def q4_k_gemv_(out, weight_data, x, inner_dim: int, outer_dim: int):
    """q4_k_gemv! (src/QuantizedKernels.jl:82-93)."""
    return _host_gemv("q4_k_gemv", Q4_K, out, weight_data, x, inner_dim, outer_dim, True)


def q5_k_gemv_(out, weight_data, x, inner_dim: int, outer_dim: int):
    """q5_k_gemv! (src/QuantizedKernels.jl:100-111)."""
    return _host_gemv("q5_k_gemv", Q5_K, out, weight_data, x, inner_dim, outer_dim, True)


def q6_k_gemv_(out, weight_data, x, inner_dim: int, outer_dim: int):
    """q6_k_gemv! (src/QuantizedKernels.jl:119-130)."""
    return _host_gemv("q6_k_gemv", Q6_K, out, weight_data, x, inner_dim, outer_dim, True)


def q8_0_gemv_(out, weight_data, x, inner_dim: int, outer_dim: int):
    """q8_0_gemv! (src/QuantizedKernels.jl:137-146)."""
    return _host_gemv("q8_0_gemv", Q8_0, out, weight_data, x, inner_dim, outer_dim, False)


GEMV_BY_QTYPE = {Q4_K: q4_k_gemv_, Q5_K: q5_k_gemv_, Q6_K: q6_k_gemv_, Q8_0: q8_0_gemv_}


# ---------------------------------------------------------------- device path

def _stream(stream=None) -> int:
    import torch
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    return getattr(stream, "cuda_stream", stream)


def _ptr(t) -> int:
    return t.data_ptr()


def check_tensor(t, name: str, dtype=None, shape=None, contiguous: bool = True, min_numel: int | None = None):
    """Raise ValueError unless t is a GPU tensor of the given dtype, shape
    (None entries match any size) and layout: the C ABI sees only raw
    pointers, so a mis-shaped or host tensor would become out-of-bounds
    device accesses."""
    import torch
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if contiguous and not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if shape is not None:
        if t.dim() != len(shape) or any(w is not None and int(g) != int(w) for g, w in zip(t.shape, shape)):
            raise ValueError(f"{name} must have shape {tuple('*' if w is None else w for w in shape)}, "
                             f"got {tuple(t.shape)}")
    if min_numel is not None and t.numel() < min_numel:
        raise ValueError(f"{name} needs at least {min_numel} elements, has {t.numel()}")
    return t


def _check_weights(qtype: int, w_dev, n: int, k: int, flags: int):
    import torch
    if qtype not in BLOCK_BYTES:
        raise ValueError(f"unsupported qtype {qtype}")
    need = packed_bytes(qtype, n, k) if flags & GEMM_PACKED else n * (k // BLOCK_ELEMS[qtype]) * BLOCK_BYTES[qtype]
    check_tensor(w_dev, "w_dev", torch.uint8, min_numel=need)


def gemm_q(qtype: int, w_dev, x, n: int, k: int, flags: int = GEMM_AUTO, out=None, stream=None, ws=None):
    """Y[M x N] = X[M x K] W^T for a device-resident GGUF weight (torch
    uint8 CUDA tensor). x: float32 CUDA tensor [M, K] (M = 1..64). ws: optional
    caller-owned uint8 CUDA workspace of gemm_ws_bytes() bytes."""
    import torch
    if x.dim() == 1:
        x = x.view(1, -1)
    check_tensor(x, "x", torch.float32, (None, k))
    m = x.shape[0]
    _check_weights(qtype, w_dev, n, k, flags)
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=x.device)
    check_tensor(out, "out", torch.float32, (m, n))
    L = _lib.load()
    if ws is None:
        ws = torch.empty(gemm_ws_bytes(qtype, m, n, k, flags), dtype=torch.uint8, device=x.device)
    check_tensor(ws, "ws", torch.uint8, min_numel=gemm_ws_bytes(qtype, m, n, k, flags))
    _lib.check(L.ihip_gemm_q(qtype, _ptr(w_dev), _ptr(x), _ptr(out), m, n, k, flags, _ptr(ws), ws.numel(),
                             _stream(stream)))
    return out


def gemm_q_ex(qtype: int, w_dev, x, n: int, k: int, act: int = ACT_PLAIN, norm_w=None, eps: float = 1e-6,
              flags: int = GEMM_AUTO, out=None, stream=None, ws=None, m: int | None = None, add=None,
              ldx: int | None = None):
    """gemm_q with its input stage fused: act = ACT_PLAIN / ACT_RMSNORM
    (RMSNorm(x) * norm_w per row) / ACT_SILU_MUL (x rows [gate | up]). x may
    be a row-strided view (x.stride(1) == 1); m defaults to x.shape[0].
    add: (pointer, n_slices, slice_stride) of K-slice partials (from
    gemm_partials) folded into x first and stored back; with x None the
    slices' sum is the input itself ([m, ldx] slices, m and ldx given); with
    GEMM_SUM_OUT and x given, likewise, and x[:m, :ldx] (ldx = x's row
    stride) is written with that sum (not read). With GEMM_DEFER the product
    stays in ws as partials and `out` is not written."""
    import torch
    width = 2 * k if act == ACT_SILU_MUL else k
    if (flags & GEMM_SUM_OUT) and (x is None or add is None):
        raise ValueError("GEMM_SUM_OUT needs x (where the slices' sum goes) and add")
    if x is None:
        if add is None or m is None or ldx is None:
            raise ValueError("x=None needs add, m and ldx")
        dev, xp = torch.device("cuda"), None
    else:
        if x.dim() == 1:
            x = x.view(1, -1)
        check_tensor(x, "x", torch.float32, contiguous=False)
        if x.dim() != 2 or x.stride(1) != 1 or x.shape[1] < width or (m is not None and m > x.shape[0]):
            raise ValueError(f"x must be [M, >= {width}] float32 with unit column stride")
        m = x.shape[0] if m is None else m
        dev, xp, ldx = x.device, _ptr(x), x.stride(0)
    _check_weights(qtype, w_dev, n, k, flags)
    if norm_w is not None:
        check_tensor(norm_w, "norm_w", torch.float32, min_numel=k)
    if out is None and not (flags & GEMM_DEFER):
        out = torch.empty((m, n), dtype=torch.float32, device=dev)
    if out is not None:
        check_tensor(out, "out", torch.float32, (m, n))
    L = _lib.load()
    if ws is None:
        ws = torch.empty(gemm_ws_bytes(qtype, m, n, k, flags), dtype=torch.uint8, device=dev)
    check_tensor(ws, "ws", torch.uint8, min_numel=gemm_ws_bytes(qtype, m, n, k, flags))
    gi = _lib.GemmInput(xp, ldx, act, None if norm_w is None else _ptr(norm_w), eps,
                        None if add is None else add[0], 0 if add is None else add[1],
                        0 if add is None else add[2])
    _lib.check(L.ihip_gemm_q_ex(qtype, _ptr(w_dev), C.byref(gi), None if out is None else _ptr(out), m, n, k, flags,
                                _ptr(ws), ws.numel(), _stream(stream)))
    return out


EPI_STORE, EPI_STATS, EPI_RESID, EPI_GATE = 0, 1, 2, 3


def chain_operand_bytes(k: int) -> int:
    """ihip_chain_operand_bytes: bytes of a chained operand for k inputs."""
    return int(_lib.load().ihip_chain_operand_bytes(k))


def chain_buffers(k: int, tiles_per_unit: int = 16, ssq: bool = False, device="cuda"):
    """Buffers a chained producer fills for a consumer with k inputs: the
    operand (uint8), tile sums [8, stride] (stride = k / 256 * tiles_per_unit)
    and, with ssq, tile sums of squares [tiles, 8]."""
    import torch
    tiles = k // 256 * tiles_per_unit
    op = torch.zeros(chain_operand_bytes(k), dtype=torch.uint8, device=device)
    tsum = torch.zeros((8, (tiles + 3) // 4 * 4), dtype=torch.float32, device=device)
    tssq = torch.zeros((tiles, 8), dtype=torch.float32, device=device) if ssq else None
    return op, tsum, tssq


def chain_in(operand, tile_sum, tiles_per_unit: int = 16, tile_ssq=None, eps: float = 1e-6):
    """ihip_chain_in: the consumer's operand as a chained producer wrote it
    (operand, tile_sum from chain_buffers); tile_ssq applies the RMSNorm row
    scale from the producer's sums of squares."""
    import torch
    check_tensor(operand, "operand", torch.uint8)
    if tile_sum is not None:
        check_tensor(tile_sum, "tile_sum", torch.float32, (8, None))
    ci = _lib.ChainIn(_ptr(operand), None if tile_sum is None else _ptr(tile_sum),
                      0 if tile_sum is None else tile_sum.stride(0), tiles_per_unit,
                      None if tile_ssq is None else _ptr(tile_ssq), 0 if tile_ssq is None else tile_ssq.shape[0], eps)
    ci._refs = (operand, tile_sum, tile_ssq)
    return ci


def chain_out(epi: int, y, consumer_qtype: int = Q4_K, operand=None, tile_sum=None, norm_w=None, tile_ssq=None,
              stat_rows: int = 0):
    """ihip_chain_out: where a chained producer leaves its output (y, unit
    column stride; EPI_RESID adds into it), the consumer's operand of y *
    norm_w in consumer_qtype's layout, its tile sums and sums of squares."""
    import torch
    check_tensor(y, "y", torch.float32, contiguous=False)
    if y.dim() != 2 or y.stride(1) != 1:
        raise ValueError("y must be [M, N] float32 with unit column stride")
    if operand is not None:
        check_tensor(operand, "operand", torch.uint8)
    if tile_sum is not None:
        check_tensor(tile_sum, "tile_sum", torch.float32, (8, None))
    co = _lib.ChainOut(epi, _ptr(y), y.stride(0), None if norm_w is None else _ptr(norm_w), consumer_qtype,
                       None if operand is None else _ptr(operand), None if tile_sum is None else _ptr(tile_sum),
                       0 if tile_sum is None else tile_sum.stride(0), None if tile_ssq is None else _ptr(tile_ssq),
                       stat_rows)
    co._refs = (y, operand, tile_sum, norm_w, tile_ssq)
    return co


def _check_chain_buffers(m: int, n: int, k: int, cin, cout):
    """Sizes of the chain descriptors' buffers against the call shape (the
    descriptors carry raw pointers; chain_in / chain_out keep the tensors):
    the consumer reads chain_operand_bytes(k) operand bytes and k / 256 *
    tiles_per_unit tile sums; the producer writes y [m, width] (width = n, or
    n / 2 for EPI_GATE), and for the width its operand covers (stat_rows for
    EPI_STATS) the operand, its tile sums and sums of squares [tiles, 8] and
    reads norm_w."""
    import torch
    if cin is not None:
        operand, tile_sum, tile_ssq = cin._refs
        tiles = k // 256 * cin.tiles_per_unit
        check_tensor(operand, "cin operand", torch.uint8, min_numel=chain_operand_bytes(k))
        if tile_sum is not None and tile_sum.shape[1] < tiles:
            raise ValueError(f"cin tile_sum must be [8, >= {tiles}]")
        if tile_ssq is not None:
            check_tensor(tile_ssq, "cin tile_ssq", torch.float32, (None, 8))
    if cout is not None:
        y, operand, tile_sum, norm_w, tile_ssq = cout._refs
        width = n // 2 if cout.epi == EPI_GATE else n
        if y.shape[0] < m or y.shape[1] < width:
            raise ValueError(f"cout y must be [>= {m}, >= {width}]")
        kn = cout.stat_rows if cout.epi == EPI_STATS else width
        tiles = kn // 8 if cout.epi == EPI_GATE else kn // 16
        if operand is not None:
            check_tensor(operand, "cout operand", torch.uint8, min_numel=chain_operand_bytes(kn))
        if tile_sum is not None and tile_sum.shape[1] < tiles:
            raise ValueError(f"cout tile_sum must be [8, >= {tiles}]")
        if tile_ssq is not None:
            check_tensor(tile_ssq, "cout tile_ssq", torch.float32, min_numel=tiles * 8)
        if norm_w is not None:
            check_tensor(norm_w, "cout norm_w", torch.float32, min_numel=kn)


def gemm_q_chain(qtype: int, w_packed, n: int, k: int, m: int, x=None, act: int = ACT_PLAIN, norm_w=None,
                 eps: float = 1e-6, add=None, cin=None, cout=None, flags: int = GEMM_F32 | GEMM_PACKED, ws=None,
                 stream=None):
    """ihip_gemm_q_chain: a fp32-accurate one-tile matmul (m <= 8) on packed
    weights whose input is either x through the usual input stage (act,
    norm_w, add as gemm_q_ex) or a chained producer's rows (cin, from
    chain_in), and whose output goes through cout (chain_out), or stays as
    K-slice partials in ws with GEMM_DEFER. A K-split matmul with an output
    descriptor keeps per-tile counts in ws, which must start zeroed (a
    workspace allocated here is)."""
    import torch
    if (x is None) == (cin is None):
        raise ValueError("pass exactly one of x / cin")
    _check_weights(qtype, w_packed, n, k, GEMM_PACKED)
    _check_chain_buffers(m, n, k, cin, cout)
    gi = None
    if x is not None:
        check_tensor(x, "x", torch.float32, contiguous=False)
        width = 2 * k if act == ACT_SILU_MUL else k
        if x.dim() != 2 or x.stride(1) != 1 or x.shape[0] < m or x.shape[1] < width:
            raise ValueError(f"x must be [M, >= {width}] float32 with unit column stride")
        if act == ACT_RMSNORM and norm_w is not None:
            check_tensor(norm_w, "norm_w", torch.float32, min_numel=k)
        gi = _lib.GemmInput(_ptr(x), x.stride(0), act, None if norm_w is None else _ptr(norm_w), eps,
                            None if add is None else add[0], 0 if add is None else add[1],
                            0 if add is None else add[2])
    need = gemm_ws_bytes(qtype, m, n, k, GEMM_F32 | GEMM_PACKED)
    if ws is None:  # (zeroed: a K-split chained epilogue's per-tile counts start at zero)
        ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    check_tensor(ws, "ws", torch.uint8, min_numel=need)
    _lib.check(_lib.load().ihip_gemm_q_chain(qtype, _ptr(w_packed), None if gi is None else C.byref(gi),
                                             None if cin is None else C.byref(cin),
                                             None if cout is None else C.byref(cout), m, n, k, flags, _ptr(ws),
                                             ws.numel(), _stream(stream)))
    return ws


def pack_weights_gated(qtype: int, w_gate_up_dev, f: int, k: int, out=None, stream=None):
    """Pack a device [gate; up] GGUF matrix [2f x k] into tiles of 8 gate rows
    and their 8 up rows (the layout of an EPI_GATE chained producer)."""
    import torch
    check_tensor(w_gate_up_dev, "w_gate_up_dev", torch.uint8,
                 min_numel=2 * f * (k // BLOCK_ELEMS[qtype]) * BLOCK_BYTES[qtype])
    if out is None:
        out = torch.empty(packed_bytes(qtype, 2 * f, k), dtype=torch.uint8, device=w_gate_up_dev.device)
    _lib.check(_lib.load().ihip_pack_weights_gated(qtype, _ptr(w_gate_up_dev), _ptr(out), f, k, _stream(stream)))
    return out


def mlp_ws_bytes(qt_gate_up: int, qt_down: int, m: int, h: int, f: int, flags: int = GEMM_AUTO) -> int:
    """Workspace bytes of mlp_forward_."""
    nb = C.c_size_t()
    _lib.check(_lib.load().ihip_mlp_ws_bytes(qt_gate_up, qt_down, m, h, f, flags, C.byref(nb)))
    return int(nb.value)


def mlp_forward_(qt_gate_up: int, w_gate_up, qt_down: int, w_down, x, h: int, f: int, norm_w=None,
                 eps: float = 1e-6, flags: int = GEMM_AUTO, ws=None, stream=None):
    """The MLP half of a decoder layer in place on the residual x [M, H]
    (src/ModelCPU.jl:884-889 with mlp_forward, :447-473): x += W_down
    (silu(W_gate n) * (W_up n)), n = rmsnorm(x, norm_w, eps). w_gate_up is
    the [gate; up] matrix (2f rows x h). Returns x."""
    import torch
    if x.dim() != 2 or x.dtype != torch.float32 or not x.is_contiguous() or x.shape[1] != h:
        raise ValueError("x must be a contiguous float32 [M, h] tensor")
    m = x.shape[0]
    if ws is None:
        ws = torch.empty(mlp_ws_bytes(qt_gate_up, qt_down, m, h, f, flags), dtype=torch.uint8, device=x.device)
    _lib.check(_lib.load().ihip_mlp_forward(qt_gate_up, _ptr(w_gate_up), qt_down, _ptr(w_down), _ptr(x),
                                            None if norm_w is None else _ptr(norm_w), eps, m, h, f, flags,
                                            _ptr(ws), ws.numel(), _stream(stream)))
    return x


def gemm_partials(qtype: int, m: int, n: int, k: int, flags: int, ws):
    """(pointer, n_slices, slice_stride) of the partials a GEMM_DEFER call
    left in ws."""
    p, ns, st = C.c_void_p(), C.c_int(), C.c_int64()
    _lib.check(_lib.load().ihip_gemm_q_partials(qtype, m, n, k, flags, _ptr(ws), C.byref(p), C.byref(ns),
                                                C.byref(st)))
    return p.value, ns.value, st.value


def gemm_ws_bytes(qtype: int, m: int, n: int, k: int, flags: int = GEMM_AUTO) -> int:
    """Workspace bytes ihip_gemm_q needs for this call shape."""
    nb = C.c_size_t()
    _lib.check(_lib.load().ihip_gemm_q_ws_bytes(qtype, m, n, k, flags & ~(GEMM_REUSE | GEMM_DEFER | GEMM_SUM_OUT),
                                                    C.byref(nb)))
    return max(int(nb.value), 16)


def packed_bytes(qtype: int, n: int, k: int) -> int:
    """Size of the packed layout of an [n x k] matrix."""
    nb = C.c_size_t()
    _lib.check(_lib.load().ihip_packed_bytes(qtype, n, k, C.byref(nb)))
    return int(nb.value)


def pack_weights(qtype: int, w_dev, n: int, k: int, out=None, stream=None):
    """Repack a device GGUF matrix [n x k] into the tile-contiguous layout
    that gemm_q reads with GEMM_PACKED (done once, at model load)."""
    import torch
    if out is None:
        out = torch.empty(packed_bytes(qtype, n, k), dtype=torch.uint8, device=w_dev.device)
    _lib.check(_lib.load().ihip_pack_weights(qtype, _ptr(w_dev), _ptr(out), n, k, _stream(stream)))
    return out


def dequant(qtype: int, w_dev, n_elems: int, stream=None):
    """Bit-exact fp32 dequantization of the first n_elems weights."""
    import torch
    out = torch.empty(n_elems, dtype=torch.float32, device=w_dev.device)
    _lib.check(_lib.load().ihip_dequant(qtype, _ptr(w_dev), _ptr(out), n_elems, _stream(stream)))
    return out


def rmsnorm(x, eps: float = 1e-6, weight=None, out=None, stream=None):
    """src/ModelCPU.jl:110-122 per row of x [rows, n]."""
    import torch
    if x.dim() == 1:
        x = x.view(1, -1)
    out = torch.empty_like(x) if out is None else out
    wp = None if weight is None else _ptr(weight)
    _lib.check(_lib.load().ihip_rmsnorm(_ptr(x), wp, _ptr(out), x.shape[0], x.shape[1], eps, _stream(stream)))
    return out


def synth_blocks(qtype: int, stream_id: int, n_blocks: int, first_block: int = 0, out=None, stream=None):
    """Seeded GGUF blocks generated on the device (same bytes as synth.blocks)."""
    import torch
    if out is None:
        out = torch.empty(n_blocks * BLOCK_BYTES[qtype], dtype=torch.uint8, device="cuda")
    _lib.check(_lib.load().ihip_synth_blocks(qtype, C.c_uint64(stream_id), first_block, n_blocks, _ptr(out),
                                             _stream(stream)))
    return out


def synth_gaussian(stream_id: int, n: int, scale: float = 1.0, add=None, out=None, stream=None):
    import torch
    if out is None:
        out = torch.empty(n, dtype=torch.float32, device="cuda")
    ap = None if add is None else _ptr(add)
    _lib.check(_lib.load().ihip_synth_gaussian(C.c_uint64(stream_id), n, scale, ap, _ptr(out), _stream(stream)))
    return out


def stream_read(buf, out=None, stream=None):
    """Read every byte of the uint8 CUDA tensor buf once (the HBM
    read-bandwidth probe); returns the XOR sink (one word per workgroup)."""
    import torch
    if out is None:
        out = torch.zeros(2048, dtype=torch.int32, device=buf.device)
    if out.numel() < 2048:
        raise ValueError("stream_read: out needs 2048 words")
    _lib.check(_lib.load().ihip_stream_read(_ptr(buf), buf.numel() // 16 * 16, _ptr(out), _stream(stream)))
    return out


def silu_mul(gu, f: int, out=None, stream=None):
    """silu(gate) * up for rows of gu = [gate | up] (src/ModelCPU.jl:447-473)."""
    import torch
    m = gu.shape[0]
    out = torch.empty((m, f), dtype=torch.float32, device=gu.device) if out is None else out
    _lib.check(_lib.load().ihip_silu_mul(_ptr(gu), m, f, _ptr(out), _stream(stream)))
    return out


def add_(y, x, stream=None):
    """y += x in place (residual add)."""
    _lib.check(_lib.load().ihip_add(_ptr(y), _ptr(x), y.numel(), _stream(stream)))
    return y
