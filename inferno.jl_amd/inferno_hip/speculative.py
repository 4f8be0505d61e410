"""Host mirror of the reference's verify/accept interface over the gfx950
library: speculate_and_verify's accept loop (src/SpeculativeDecoding.jl:
37-107), mtp_verify_step!'s greedy verify (src/ModelCPU.jl:1914-1930), the
speculative statistics of generate_speculative_cpu
(src/SpeculativeDecoding.jl:163-171), and a tree-accept walk (no reference
counterpart).

The reference draws its uniforms from Julia's global RNG inside the loop;
here they are explicit inputs so that CPU and GPU decide on the same draws.
Token ids are 0-based (the Julia shim adds 1).
"""
from __future__ import annotations

from dataclasses import dataclass

from . import _lib
from .quantized_kernels import _ptr, _stream, check_tensor

MODE_STANDARD = 0   # p, q at temperature T; residual max(0, p - q)
MODE_REFERENCE = 1  # src/SpeculativeDecoding.jl:61-63,79-93 as written


def _ws(nbytes: int, device):
    import torch
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)


def softmax_stats(logits, temperature: float, stream=None):
    """(zmax, zsum) per row of logits [rows, V] for z = logits / T."""
    import torch
    import ctypes as C
    rows, V = logits.shape
    L = _lib.load()
    nb = C.c_size_t()
    _lib.check(L.ihip_accept_ws_bytes(rows, V, C.byref(nb)))
    ws = _ws(nb.value, logits.device)
    zmax = torch.empty(rows, dtype=torch.float32, device=logits.device)
    zsum = torch.empty_like(zmax)
    _lib.check(L.ihip_softmax_stats(_ptr(logits), rows, V, temperature, _ptr(zmax), _ptr(zsum), _ptr(ws),
                                    ws.numel(), _stream(stream)))
    return zmax, zsum


def spec_accept(target_logits, draft_logits, draft_tokens, temperature: float, u_acc, u_res, u_bonus,
                mode: int = MODE_STANDARD, stream=None, out_tok=None, out_n=None, ws=None, top_p: float = 1.0,
                top_k: int = 0, min_p: float = 0.0):
    """Batched accept step.

    target_logits [S, k+1, V], draft_logits [S, k, V], draft_tokens [S, k]
    int32, u_acc [S, k], u_res [S], u_bonus [S] (float32, CUDA).
    Returns (out_tok [S, k+1] int32, out_n [S] int32): the accepted drafts
    followed by the resampled or bonus token at index out_n; in
    MODE_REFERENCE a step whose last draft is rejected (out_n == k - 1) also
    carries the reference's bonus token at index k
    (src/SpeculativeDecoding.jl:100). n_tokens() gives the count.
    top_p / top_k (speculate_and_verify's keywords, src/SpeculativeDecoding.jl
    :44-45) and min_p filter every bonus draw as softmax_sample does
    (:100-104); the ratio tests and residuals stay unfiltered.
    """
    import torch
    import ctypes as C
    check_tensor(target_logits, "target_logits", torch.float32)
    if target_logits.dim() == 2:
        target_logits = target_logits.unsqueeze(0)
        draft_logits = draft_logits.unsqueeze(0)
        draft_tokens = draft_tokens.view(1, -1)
        u_acc = u_acc.view(1, -1)
        u_res = u_res.view(1)
        u_bonus = u_bonus.view(1)
    if target_logits.dim() != 3:
        raise ValueError("target_logits must be [S, k+1, V] (or [k+1, V])")
    S, k1, V = target_logits.shape
    k = k1 - 1
    check_tensor(draft_logits, "draft_logits", torch.float32, (S, k, V))
    check_tensor(draft_tokens, "draft_tokens", torch.int32, (S, k))
    check_tensor(u_acc, "u_acc", torch.float32, (S, k))
    check_tensor(u_res, "u_res", torch.float32, (S,))
    check_tensor(u_bonus, "u_bonus", torch.float32, (S,))
    L = _lib.load()
    nb = C.c_size_t()
    _lib.check(L.ihip_spec_accept_ex_ws_bytes(S, k, V, top_k, top_p, min_p, C.byref(nb)))
    dev = target_logits.device
    if ws is None:
        ws = _ws(nb.value, dev)
    check_tensor(ws, "ws", torch.uint8, min_numel=nb.value)
    if out_tok is None:
        out_tok = torch.zeros((S, k + 1), dtype=torch.int32, device=dev)
    if out_n is None:
        out_n = torch.zeros(S, dtype=torch.int32, device=dev)
    check_tensor(out_tok, "out_tok", torch.int32, (S, k + 1))
    check_tensor(out_n, "out_n", torch.int32, (S,))
    _lib.check(L.ihip_spec_accept_ex(_ptr(target_logits), _ptr(draft_logits), _ptr(draft_tokens), S, k, V,
                                     temperature, top_k, top_p, min_p, _ptr(u_acc), _ptr(u_res), _ptr(u_bonus),
                                     mode, _ptr(out_tok), _ptr(out_n), _ptr(ws), ws.numel(), _stream(stream)))
    return out_tok, out_n


def n_tokens(n: int, k: int, mode: int = MODE_STANDARD) -> int:
    """Number of tokens a step of spec_accept returns for out_n = n: the
    accepted drafts and the resampled or bonus token, plus the reference
    mode's bonus after a rejection of the last draft (0 for an invalid
    step)."""
    if n < 0:
        return 0
    return n + 1 + (1 if mode == MODE_REFERENCE and k >= 1 and n == k - 1 else 0)


def greedy_verify(logits, draft_tokens, stream=None):
    """logits [S, k+1, V], draft_tokens [S, k] -> (out_n [S], argmax [S, k+1])."""
    import torch
    import ctypes as C
    check_tensor(logits, "logits", torch.float32)
    if logits.dim() == 2:
        logits = logits.unsqueeze(0)
        draft_tokens = draft_tokens.view(1, -1)
    if logits.dim() != 3:
        raise ValueError("logits must be [S, k+1, V] (or [k+1, V])")
    S, k1, V = logits.shape
    k = k1 - 1
    check_tensor(draft_tokens, "draft_tokens", torch.int32, (S, k))
    L = _lib.load()
    nb = C.c_size_t()
    _lib.check(L.ihip_accept_ws_bytes(S * k1, V, C.byref(nb)))
    ws = _ws(nb.value, logits.device)
    out_n = torch.zeros(S, dtype=torch.int32, device=logits.device)
    am = torch.zeros((S, k1), dtype=torch.int32, device=logits.device)
    _lib.check(L.ihip_greedy_verify(_ptr(logits), _ptr(draft_tokens) if k else None, S, k, V, _ptr(out_n),
                                    _ptr(am), _ptr(ws), ws.numel(), _stream(stream)))
    return out_n, am


def mtp_verify_step(logits, draft_tokens, stream=None):
    """mtp_verify_step! (src/ModelCPU.jl:1914-1930) given the full logits of
    the verify forward: rows 0..k for tokens [last, d_1..d_k]; draft_tokens
    are d_1..d_k. Returns (accepted_count, logits)."""
    n, _ = greedy_verify(logits, draft_tokens, stream)
    return int(n[0].item()), logits


def tree_accept(target_logits, draft_logits, node_tokens, parent, temperature: float, u, stream=None):
    """Longest accepted root-to-leaf path of a draft tree (node 0 = root).
    Raises ValueError for a malformed tree (a parent not earlier than its
    node, or a token outside the vocabulary), which the device reports as
    out_len = -1."""
    import torch
    import ctypes as C
    check_tensor(target_logits, "target_logits", torch.float32, (None, None))
    n, V = target_logits.shape
    check_tensor(draft_logits, "draft_logits", torch.float32, (n, V))
    check_tensor(node_tokens, "node_tokens", torch.int32, (n,))
    check_tensor(parent, "parent", torch.int32, (n,))
    check_tensor(u, "u", torch.float32, (n,))
    L = _lib.load()
    nb = C.c_size_t()
    _lib.check(L.ihip_accept_ws_bytes(3 * n, V, C.byref(nb)))
    ws = _ws(nb.value, target_logits.device)
    path = torch.zeros(n, dtype=torch.int32, device=target_logits.device)
    ln = torch.zeros(1, dtype=torch.int32, device=target_logits.device)
    _lib.check(L.ihip_tree_accept(_ptr(target_logits), _ptr(draft_logits), _ptr(node_tokens), _ptr(parent), n, V,
                                  temperature, _ptr(u), _ptr(path), _ptr(ln), _ptr(ws), ws.numel(),
                                  _stream(stream)))
    n_path = int(ln.item())
    if n_path < 0:
        raise ValueError("tree_accept: malformed tree (parent[i] must lie in [0, i), tokens in [0, V))")
    return path[:n_path]


@dataclass
class SpeculativeStats:
    """The statistics dict of generate_speculative_cpu
    (src/SpeculativeDecoding.jl:163-171)."""
    gamma: int
    draft_tokens_generated: int = 0
    tokens_accepted: int = 0
    tokens_generated: int = 0
    prompt_len: int = 0

    def record(self, n_out_tokens: int) -> None:
        # the reference counts every returned token (accepted drafts plus the
        # resampled or bonus token) as "accepted" (:156)
        self.draft_tokens_generated += self.gamma
        self.tokens_accepted += n_out_tokens
        self.tokens_generated += n_out_tokens

    def as_dict(self) -> dict:
        rate = self.tokens_accepted / self.draft_tokens_generated if self.draft_tokens_generated else 0.0
        speedup = ((self.tokens_generated - self.prompt_len) /
                   (self.draft_tokens_generated + self.tokens_generated) * (1 + self.gamma)
                   if (self.draft_tokens_generated + self.tokens_generated) else 0.0)
        return {"acceptance_rate": rate, "draft_tokens_generated": self.draft_tokens_generated,
                "tokens_accepted": self.tokens_accepted, "speedup_estimate": speedup}


def commit_state_(state, snapshots, n_accepted, stream=None):
    """After a verify step (no reference counterpart: src/SpeculativeDecoding.jl
    :69-70 keeps none): state[s] = snapshots[s, n] for n = n_accepted[s] >= 0,
    read on the device. state [steps, ...], snapshots [steps, k + 1, ...] of the
    same dtype, contiguous; n_accepted int32 [steps] (out_n of spec_accept)."""
    steps = state.shape[0]
    k = snapshots.shape[1] - 1
    per = state[0].numel() * state.element_size()
    if snapshots.shape[0] != steps or snapshots[0, 0].numel() != state[0].numel() or not state.is_contiguous() \
            or not snapshots.is_contiguous() or snapshots.dtype != state.dtype:
        raise ValueError("snapshots must be [steps, k + 1, *state.shape[1:]] of the state's dtype")
    _lib.check(_lib.load().ihip_spec_commit_state(_ptr(state), _ptr(snapshots), per, per, k, _ptr(n_accepted), steps,
                                                  per, (k + 1) * per, _stream(stream)))
    return state


def advance_len_(lengths, n_accepted, stream=None):
    """lengths[s] += n_accepted[s] + 1 where n_accepted[s] >= 0 (int32, on the device)."""
    _lib.check(_lib.load().ihip_spec_advance_len(_ptr(lengths), _ptr(n_accepted), lengths.numel(),
                                                 _stream(stream)))
    return lengths
