"""Host mirror of the reference's draft-side sampler over the gfx950
library: softmax_sample (temperature, top-k, top-p, min-p;
src/ModelCPU.jl:1123-1200) and the presence / repetition penalties the
generation loop applies to the logits first (src/ModelCPU.jl:1202-1225,
called at :1247-1248).

The reference draws r = rand(Float32) inside softmax_sample; here the
uniforms are explicit inputs, one per row. Token ids are 0-based (the Julia
shim adds 1). There is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C

from . import _lib
from .quantized_kernels import _ptr, _stream


def sample_ws_bytes(rows: int, V: int) -> int:
    """Workspace bytes of ihip_sample_ex for rows x V."""
    nb = C.c_size_t()
    _lib.check(_lib.load().ihip_sample_ws_bytes(rows, V, C.byref(nb)))
    return max(int(nb.value), 16)


def softmax_sample(logits, u, temperature: float = 1.0, top_p: float = 1.0, top_k: int = 0, min_p: float = 0.0,
                   out=None, stream=None, spread: bool = True, ws=None):
    """One token per row of logits [rows, V] (float32, contiguous) with the
    uniforms u [rows]; returns int32 [rows]. spread: ihip_sample_ex, whose
    every setting spreads each row over workgroups of 4096 logits, with ws
    (uint8, sample_ws_bytes; allocated here when None); else ihip_sample
    (one workgroup per row)."""
    import torch
    if logits.dim() == 1:
        logits = logits.view(1, -1)
    if logits.dtype != torch.float32 or not logits.is_contiguous() or not logits.is_cuda:
        raise ValueError("logits must be a contiguous float32 GPU tensor")
    rows, V = logits.shape
    if not u.is_cuda or u.dtype != torch.float32 or u.numel() < rows:
        raise ValueError("u must be a float32 GPU tensor with one uniform per row")
    if out is None:
        out = torch.empty(rows, dtype=torch.int32, device=logits.device)
    elif not out.is_cuda or out.dtype != torch.int32 or out.numel() < rows:
        raise ValueError("out must be an int32 GPU tensor with one entry per row")
    if not spread:
        _lib.check(_lib.load().ihip_sample(_ptr(logits), rows, V, float(temperature), int(top_k), float(top_p),
                                           float(min_p), _ptr(u), _ptr(out), _stream(stream)))
        return out
    need = sample_ws_bytes(rows, V)
    if ws is None:
        ws = torch.empty(need, dtype=torch.uint8, device=logits.device)
    elif not ws.is_cuda or ws.dtype != torch.uint8 or ws.numel() < need:
        raise ValueError(f"ws must be a uint8 GPU tensor of at least {need} bytes")
    _lib.check(_lib.load().ihip_sample_ex(_ptr(logits), rows, V, float(temperature), int(top_k), float(top_p),
                                          float(min_p), _ptr(u), _ptr(out), _ptr(ws), ws.numel(), _stream(stream)))
    return out


def apply_penalties_(logits, token_ids, presence: float = 0.0, repetition: float = 1.0, stream=None):
    """apply_presence_penalty! then apply_repetition_penalty! in place.
    token_ids: int32 [n] (one list for every row) or [rows, n] (per row);
    repeated ids count once (the reference iterates a Dict's keys)."""
    import torch
    if logits.dim() == 1:
        logits = logits.view(1, -1)
    if logits.dtype != torch.float32 or not logits.is_contiguous() or not logits.is_cuda:
        raise ValueError("logits must be a contiguous float32 GPU tensor")
    rows, V = logits.shape
    ids = torch.as_tensor(token_ids).to(device=logits.device, dtype=torch.int32).contiguous()
    n = ids.shape[-1] if ids.numel() else 0
    stride = 0 if ids.dim() == 1 else ids.stride(0)
    if ids.dim() == 2 and ids.shape[0] != rows:
        raise ValueError("token_ids [rows, n] must have one row per logits row")
    _lib.check(_lib.load().ihip_apply_penalties(_ptr(logits), rows, V, _ptr(ids) if n else None, n, stride,
                                                float(presence), float(repetition), _stream(stream)))
    return logits
