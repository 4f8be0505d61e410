#!/usr/bin/env python3
"""Benchmark of the speculative-verify hot path on one MI355X.

Workload (the metric's verify step): a full
9B-class verify step at M = 5 (1 accepted + k = 4 draft tokens):
32 decoder layers of projections, hidden 4096 - Q4_K q (4096x4096),
k/v (2 x 1024x4096), o (4096x4096), gate/up (2 x 12288x4096) and Q6_K down
(4096x12288) - chained in fp32 with RMSNorm before q/k/v and gate/up, SiLU
gating and residual adds, then RMSNorm, the Q6_K lm_head (151936x4096) and
the k = 4 rejection-sampling accept at T = 0.8. Weights are seeded synthetic
GGUF blocks (no checkpoint is available offline), resident in HBM; a step is
replayed from a captured HIP graph. `value` is verify steps per second.

Also reported: `roofline` for the dominant dequant-matmul (the Q4_K
gate/up projection, 24576x4096 at M = 5, timed live with HIP events over
cold weights), a dequant-matmul GB/s sweep at M = 1..8, and `cpu_baseline`:
the reference's own CPU kernels (src/kernels/quant_kernels.c built from
source into oracle/_ref) called once per token per matrix as forward_cpu!
does, on a bounded sample of the same step, timed on this host.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "inferno.jl_amd"))

METRIC = "dequant-matmul GB/s & % HBM peak at M=1..8; verify steps/sec (k=4, 1 GPU)"
HBM_PEAK_GBPS = 8000.0
SEED = 0x1F3E0003  # configs[3]

H, NQ, NKV, FF, VOCAB = 4096, 4096, 1024, 12288, 151936


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Model:
    """Device-resident synthetic weights of the config-4 shape, generated as
    GGUF blocks and repacked once into the matmul's tile-contiguous layout
    (as a model loader would at load time). The GGUF bytes of the first
    `keep_gguf` layers and of the lm_head are kept on the host for the CPU
    baseline."""

    SHAPES = {"q": ("Q4_K", NQ, H, "attn_q"), "kv": ("Q4_K", 2 * NKV, H, "attn_kv"),  # k rows then v rows
              "o": ("Q4_K", H, NQ, "attn_output"), "gu": ("Q4_K", 2 * FF, H, "ffn_gate_up"),  # gate then up
              "down": ("Q6_K", H, FF, "ffn_down")}

    def __init__(self, ih, n_layers: int, keep_gguf: int = 4, proj: str = "Q4_K", gated: bool = False):
        import torch
        F = ih.formats
        st = ih.synth.stream_for
        self.proj = getattr(F, proj)  # format of the q/k/v/o/gate/up projections (config 5: Q4_K or Q5_K)
        # gated: [gate; up] packed in tiles of 8 gate rows and their 8 up rows (the chained step's layout)
        self.gated = gated
        self.layers, self.host_gguf, self.gguf_bytes = [], [], 0
        for L in range(n_layers):
            lw, hw = {}, {}
            for key, (qn, rows, k, name) in self.SHAPES.items():
                qt = self.proj if qn == "Q4_K" else getattr(F, qn)
                g = ih.quantized_kernels.synth_blocks(qt, st(SEED, f"blk{L}.{name}"), rows * k // F.BLOCK_ELEMS[qt])
                if key == "gu" and gated:
                    lw[key] = ih.pack_weights_gated(qt, g, rows // 2, k)
                else:
                    lw[key] = ih.pack_weights(qt, g, rows, k)
                self.gguf_bytes += g.numel()
                if L < keep_gguf:
                    hw[key] = g.cpu().numpy()
                del g
            # q and k/v rows share the input: one matrix [q; k; v] (the packed
            # layout concatenates along tiles)
            lw["qkv"] = torch.cat([lw.pop("q"), lw.pop("kv")])
            for name in ("attn_norm", "ffn_norm"):  # RMSNorm weights around 1
                lw[name] = 1.0 + ih.quantized_kernels.synth_gaussian(st(SEED, f"blk{L}.{name}"), H, 0.1)
                if L < keep_gguf:
                    hw[name] = lw[name].cpu().numpy()
            self.layers.append(lw)
            if L < keep_gguf:
                self.host_gguf.append(hw)
        g = ih.quantized_kernels.synth_blocks(F.Q6_K, st(SEED, "output"), VOCAB * H // 256)
        self.lm = ih.pack_weights(F.Q6_K, g, VOCAB, H)
        self.out_norm = 1.0 + ih.quantized_kernels.synth_gaussian(st(SEED, "output_norm"), H, 0.1)
        self.gguf_bytes += g.numel()
        self.host_lm = g.cpu().numpy()
        self.host_out_norm = self.out_norm.cpu().numpy()
        del g
        torch.cuda.synchronize()

    def weight_bytes(self, n_layers: int) -> int:
        """GGUF bytes of the weights one step streams."""
        return self.gguf_bytes


class VerifyStep:
    """One verify step: layers, final norm, lm_head, accept."""

    def __init__(self, ih, model: Model, M: int, k: int, T: float, prec: int = 1, draft_from_target: bool = True):
        import torch
        dev = "cuda"
        F = ih.formats
        self.ih, self.model, self.M, self.k, self.T, self.prec = ih, model, M, k, T, prec
        st = ih.synth.stream_for
        self.x0 = ih.quantized_kernels.synth_gaussian(st(SEED, "x0"), M * H).view(M, H)
        self.x = torch.empty_like(self.x0)
        self.qkv = torch.empty((M, NQ + 2 * NKV), device=dev)
        self.gu = torch.empty((M, 2 * FF), device=dev)
        self.logits = torch.empty((M, VOCAB), device=dev)
        gws = ih.quantized_kernels.gemm_ws_bytes
        fl = prec | ih.GEMM_PACKED | ih.GEMM_ACCUM
        P = model.proj
        wsb = max(gws(P, M, NQ + 2 * NKV, H, fl), gws(P, M, H, NQ, fl),
                  gws(P, M, 2 * FF, H, fl), gws(F.Q6_K, M, H, FF, fl), gws(F.Q6_K, M, VOCAB, H, fl))
        # (zeroed: a K-split chained epilogue keeps per-tile slice counts there, zero between calls)
        self.ws = torch.zeros(wsb, dtype=torch.uint8, device=dev)
        self.ws_down = torch.zeros(wsb, dtype=torch.uint8, device=dev)  # holds the deferred down partials
        self.ws_o = torch.zeros(wsb, dtype=torch.uint8, device=dev)  # the deferred o partials (when K-sliced)
        # draft side (inputs of the verify step): draft logits around the
        # target rows (target + N(0, 1.5^2), as configs[2] draws them), draft
        # tokens drawn from the draft softmax at T, uniforms
        if draft_from_target and k <= M:
            self.forward()  # the step's target logits (every timed step recomputes the same)
            self.drf = ih.quantized_kernels.synth_gaussian(st(SEED, "draft_logits"), k * VOCAB, 1.5,
                                                           add=self.logits[:k].contiguous()).view(k, VOCAB)
        else:
            self.drf = ih.quantized_kernels.synth_gaussian(st(SEED, "draft_logits"), k * VOCAB, 3.0).view(k, VOCAB)
        g = torch.Generator(device="cpu").manual_seed(SEED)
        p = torch.softmax(self.drf.cpu().double() / T, -1)
        self.draft = torch.multinomial(p, 1, generator=g).view(1, k).to(torch.int32).to(dev)
        self.u_acc = torch.rand((1, k), generator=g).to(dev)
        self.u_res = torch.rand(1, generator=g).to(dev)
        self.u_bonus = torch.rand(1, generator=g).to(dev)
        nb = C.c_size_t()
        ih._lib.check(ih.load().ihip_spec_accept_ws_bytes(1, k, VOCAB, C.byref(nb)))
        self.acc_ws = torch.empty(nb.value, dtype=torch.uint8, device=dev)
        self.out_tok = torch.zeros((1, k + 1), dtype=torch.int32, device=dev)
        self.out_n = torch.zeros(1, dtype=torch.int32, device=dev)

    def run(self):
        self.forward()
        self.accept()

    def forward(self, probe=None):
        """The target forward of one verify step: per layer [residual += previous down] + RMSNorm
        -> [q; k; v] -> o -> [residual += o] + RMSNorm -> [gate; up] -> SiLU
        gating -> down (left as K-slice partials); final residual add +
        RMSNorm -> lm_head -> accept. RMSNorm, SiLU gating and the residual
        adds of o and down run inside the input stage of the matmul that
        consumes them, as does the sum of a K-sliced [q; k; v], which o's
        input stage also stores into qkv. probe(tag, layer), when given, is called (outside any
        graph capture) before each layer's [q; k; v] ("pre"), after it
        ("qkv"), after o ("o"), after [gate; up] ("gu") and after the
        lm_head ("head"), so a test can read x, qkv, gu, logits and the
        deferred partials in the workspaces at each point."""
        ih, F, M = self.ih, self.ih.formats, self.M
        P = self.model.proj
        ex = ih.gemm_q_ex
        f32 = self.prec | ih.GEMM_PACKED  # (GEMM_F32, or 0: fp32-accurate below 16 tokens, half above)
        acc = f32 | ih.GEMM_ACCUM
        dfr = f32 | ih.GEMM_DEFER
        parts = ih.gemm_partials(F.Q6_K, M, H, FF, f32, self.ws_down)
        # o leaves its partials to the next input stage, which adds them into
        # the residual while it reads it (no read-modify-write at the end of
        # o, no reduce launch when K-sliced); K-sliced [gate; up] (several
        # token tiles) likewise, summed by the SiLU-gating stage
        o_parts = ih.gemm_partials(P, M, H, NQ, f32, self.ws_o)
        gu_parts = ih.gemm_partials(P, M, 2 * FF, H, f32, self.ws)
        fold_o, fold_gu = True, gu_parts[1] > 1
        # a K-sliced [q; k; v] (several token tiles) is summed by o's input
        # stage, which also stores it (GEMM_SUM_OUT): no reduce launch
        qkv_parts = ih.gemm_partials(P, M, NQ + 2 * NKV, H, f32, self.ws)
        fold_qkv = qkv_parts[1] > 1
        self.x.copy_(self.x0)
        for i, lw in enumerate(self.model.layers):
            if probe:
                probe("pre", i)
            ex(P, lw["qkv"], self.x, NQ + 2 * NKV, H, act=ih.ACT_RMSNORM, norm_w=lw["attn_norm"],
               flags=dfr if fold_qkv else f32, out=None if fold_qkv else self.qkv, ws=self.ws,
               add=parts if i > 0 else None)
            if probe:
                probe("qkv", i)
            if fold_qkv:
                ex(P, lw["o"], self.qkv, H, NQ, flags=dfr | ih.GEMM_SUM_OUT, ws=self.ws_o, add=qkv_parts)
            elif fold_o:
                ex(P, lw["o"], self.qkv[:, :NQ], H, NQ, flags=dfr, ws=self.ws_o)
            else:
                ex(P, lw["o"], self.qkv[:, :NQ], H, NQ, flags=acc, out=self.x, ws=self.ws)
            if probe:
                probe("o", i)
            ex(P, lw["gu"], self.x, 2 * FF, H, act=ih.ACT_RMSNORM, norm_w=lw["ffn_norm"],
               flags=dfr if fold_gu else f32, out=None if fold_gu else self.gu, ws=self.ws,
               add=o_parts if fold_o else None)
            if probe:
                probe("gu", i)
            if fold_gu:
                ex(F.Q6_K, lw["down"], None, H, FF, act=ih.ACT_SILU_MUL, flags=dfr, ws=self.ws_down, add=gu_parts,
                   m=M, ldx=2 * FF)
            else:
                ex(F.Q6_K, lw["down"], self.gu, H, FF, act=ih.ACT_SILU_MUL, flags=dfr, ws=self.ws_down)
        ex(F.Q6_K, self.model.lm, self.x, VOCAB, H, act=ih.ACT_RMSNORM, norm_w=self.model.out_norm, flags=f32,
           out=self.logits, ws=self.ws, add=parts)
        if probe:
            probe("head", len(self.model.layers))

    def accept_histogram(self, n_steps: int = 256):
        """Accepted lengths of n_steps verify steps over this step's logits,
        each with its own draft tokens (drawn from the draft softmax at T) and
        uniforms: counts of out_n = 0..k (one batched accept call, untimed)."""
        import torch
        k, dev = self.k, self.logits.device
        g = torch.Generator(device="cpu").manual_seed(SEED + 11)
        p = torch.softmax(self.drf.cpu().double() / self.T, -1)
        draft = torch.multinomial(p, n_steps, replacement=True, generator=g).t().contiguous().to(torch.int32).to(dev)
        tgt = self.logits[:k + 1].unsqueeze(0).expand(n_steps, k + 1, VOCAB).contiguous()
        drf = self.drf.unsqueeze(0).expand(n_steps, k, VOCAB).contiguous()
        ua = torch.rand((n_steps, k), generator=g).to(dev)
        ur, ub = torch.rand(n_steps, generator=g).to(dev), torch.rand(n_steps, generator=g).to(dev)
        _, n = self.ih.spec_accept(tgt, drf, draft, self.T, ua, ur, ub)
        return torch.bincount(n.cpu().long(), minlength=k + 1).tolist()

    def accept(self):
        self.ih.spec_accept(self.logits.view(1, self.M, VOCAB), self.drf.view(1, self.k, VOCAB), self.draft,
                            self.T, self.u_acc, self.u_res, self.u_bonus, out_tok=self.out_tok, out_n=self.out_n,
                            ws=self.acc_ws)


class ChainStep(VerifyStep):
    """The verify step with chained matmuls (ihip_gemm_q_chain, gated model
    weights): per layer one input stage, that of [q; k; v] (the previous
    layer's down partials folded into the residual, RMSNorm). [q; k; v]
    writes o's operand (its q rows, split fp16 at per-tile scales); o adds
    its product into the residual and writes [gate; up]'s operand (the
    residual times the FFN norm weight) with the tile sums of squares of the
    RMSNorm; [gate; up] writes h = silu(gate) up and down's operand; down
    leaves K-slice partials. Same arithmetic as VerifyStep.forward
    (fp32-accurate, M <= 8), three input-stage launches fewer per layer."""

    def __init__(self, ih, model: Model, M: int, k: int, T: float):
        import torch
        assert model.gated and M <= 8, "the chained step needs gated weights and one token tile"
        F = ih.formats
        self.h = torch.empty((M, FF), device="cuda")
        self.op_q, self.ts_q, _ = ih.chain_buffers(NQ)
        self.op_x, self.ts_x, self.ssq_x = ih.chain_buffers(H, ssq=True)
        self.op_h, _, _ = ih.chain_buffers(FF, tiles_per_unit=32)
        super().__init__(ih, model, M, k, T, prec=1)

    def _descriptors(self):
        # (built at the first forward: VerifyStep's constructor runs one, after making x and qkv)
        ih, F = self.ih, self.ih.formats
        cin, cout = ih.chain_in, ih.chain_out
        self.o_in = cin(self.op_q, self.ts_q, 16)
        self.gu_in = cin(self.op_x, self.ts_x, 16, tile_ssq=self.ssq_x, eps=1e-6)
        self.down_in = cin(self.op_h, None, 32)
        self.qkv_out = cout(ih.EPI_STATS, self.qkv, F.Q4_K, self.op_q, self.ts_q, stat_rows=NQ)
        self.o_out = [cout(ih.EPI_RESID, self.x, F.Q4_K, self.op_x, self.ts_x, norm_w=lw["ffn_norm"],
                           tile_ssq=self.ssq_x) for lw in self.model.layers]
        self.gu_out = cout(ih.EPI_GATE, self.h, F.Q6_K, self.op_h)

    def forward(self, probe=None):
        ih, F, M = self.ih, self.ih.formats, self.M
        if not hasattr(self, "qkv_out"):
            self._descriptors()
        P = self.model.proj
        chain = ih.gemm_q_chain
        fl = ih.GEMM_F32 | ih.GEMM_PACKED
        parts = ih.gemm_partials(F.Q6_K, M, H, FF, fl, self.ws_down)
        self.x.copy_(self.x0)
        for i, lw in enumerate(self.model.layers):
            if probe:
                probe("pre", i)
            chain(P, lw["qkv"], NQ + 2 * NKV, H, M, x=self.x, act=ih.ACT_RMSNORM, norm_w=lw["attn_norm"],
                  add=parts if i > 0 else None, ws=self.ws, cout=self.qkv_out)
            if probe:
                probe("qkv", i)
            chain(P, lw["o"], H, NQ, M, cin=self.o_in, ws=self.ws_o, cout=self.o_out[i])
            if probe:
                probe("o", i)
            chain(P, lw["gu"], 2 * FF, H, M, ws=self.ws, cin=self.gu_in, cout=self.gu_out)
            if probe:
                probe("gu", i)
            chain(F.Q6_K, lw["down"], H, FF, M, cin=self.down_in, flags=fl | ih.GEMM_DEFER, ws=self.ws_down)
        ih.gemm_q_ex(F.Q6_K, self.model.lm, self.x, VOCAB, H, act=ih.ACT_RMSNORM, norm_w=self.model.out_norm,
                     flags=fl, out=self.logits, ws=self.ws, add=parts)
        if probe:
            probe("head", len(self.model.layers))


class TreeStep(VerifyStep):
    """Config 5: a 64-node draft tree (branching 4, 4, 4 in BFS order,
    truncated to 64 nodes) verified in one forward at M = 64 (half-precision
    MFMA operands, the default at M >= 16), then the tree accept walk at
    T = 1.0 with one uniform per node."""

    def __init__(self, ih, model: Model, n: int = 64, T: float = 1.0):
        import torch
        super().__init__(ih, model, n, 1, T, prec=0, draft_from_target=False)
        st = ih.synth.stream_for
        par = [-1]
        for i in range(1, n):  # node i's parent: BFS over branching 4
            par.append((i - 1) // 4)
        self.parent = torch.tensor(par, dtype=torch.int32, device="cuda")
        self.forward()  # target logits of the tree's rows (the timed steps recompute them)
        torch.cuda.synchronize()
        # draft rows around the target rows; each node's token drawn from its parent's draft row
        self.drf_t = ih.quantized_kernels.synth_gaussian(st(SEED, "tree_draft"), n * VOCAB, 1.5,
                                                         add=self.logits).view(n, VOCAB)
        g = torch.Generator(device="cpu").manual_seed(SEED + 5)
        tok = [0]
        for i in range(1, n):
            p = torch.softmax(self.drf_t[par[i]].cpu().double() / T, -1)
            tok.append(int(torch.multinomial(p, 1, generator=g)))
        self.tok = torch.tensor(tok, dtype=torch.int32, device="cuda")
        self.u = torch.rand(n, generator=g).to("cuda")
        nb = C.c_size_t()
        ih._lib.check(ih.load().ihip_accept_ws_bytes(3 * n, VOCAB, C.byref(nb)))
        self.tree_ws = torch.empty(nb.value, dtype=torch.uint8, device="cuda")
        self.path = torch.zeros(n, dtype=torch.int32, device="cuda")
        self.plen = torch.zeros(1, dtype=torch.int32, device="cuda")

    def accept(self):
        q = self.ih.quantized_kernels
        self.ih._lib.check(self.ih.load().ihip_tree_accept(
            q._ptr(self.logits), q._ptr(self.drf_t), q._ptr(self.tok), q._ptr(self.parent), self.M, VOCAB, self.T,
            q._ptr(self.u), q._ptr(self.path), q._ptr(self.plen), q._ptr(self.tree_ws), self.tree_ws.numel(),
            q._stream(None)))


def accept_cost(ih, step, replays: int = 10):
    """The accept launch of the timed step (ihip_spec_accept, M = 5 target
    rows, k = 4 draft rows, V = 151936) timed alone, microseconds per call
    (8 calls per replayed graph), on the step's own logits -- those of the
    configured synthetic blocks, whose sd of ~260 makes every softmax
    near one-hot, so nearly every draft is accepted -- and on spread rows of
    the same shape (target ~ N(0, 4^2), draft = target + N(0, 1.5^2), drafts
    drawn from the draft softmax), where most steps end in a residual draw
    over the whole vocabulary; with the accepted-length histogram of 256
    draws on the spread rows."""
    import torch
    st = ih.synth.stream_for
    M, k, T = step.M, step.k, step.T
    t_step = graph_launch_time(lambda i: step.accept(), 8, replays, 2)
    tgt = ih.quantized_kernels.synth_gaussian(st(SEED, "spread_target"), M * VOCAB, 4.0).view(1, M, VOCAB)
    drf = ih.quantized_kernels.synth_gaussian(st(SEED, "spread_draft"), k * VOCAB, 1.5,
                                              add=tgt[0, :k].contiguous()).view(1, k, VOCAB)
    g = torch.Generator(device="cpu").manual_seed(SEED + 21)
    p = torch.softmax(drf[0].cpu().double() / T, -1)
    draft = torch.multinomial(p, 1, generator=g).view(1, k).to(torch.int32).cuda()
    out_tok, out_n = torch.zeros_like(step.out_tok), torch.zeros_like(step.out_n)
    t_spread = graph_launch_time(lambda i: ih.spec_accept(tgt, drf, draft, T, step.u_acc, step.u_res, step.u_bonus,
                                                          out_tok=out_tok, out_n=out_n, ws=step.acc_ws),
                                 8, replays, 2)
    n_draws = 256
    drafts = torch.multinomial(p, n_draws, replacement=True, generator=g).t().contiguous().to(torch.int32).cuda()
    ua = torch.rand((n_draws, k), generator=g).cuda()
    ur, ub = torch.rand(n_draws, generator=g).cuda(), torch.rand(n_draws, generator=g).cuda()
    _, n = ih.spec_accept(tgt.expand(n_draws, M, VOCAB).contiguous(), drf.expand(n_draws, k, VOCAB).contiguous(),
                          drafts, T, ua, ur, ub)
    hist = torch.bincount(n.cpu().long(), minlength=k + 1).tolist()
    return round(t_step * 1e6, 2), round(t_spread * 1e6, 2), hist


def graph_launch_time(launch, iters: int, replays: int, warm: int) -> float:
    """`iters` calls of launch(i) captured in one HIP graph on a side stream,
    replayed `warm` times untimed, then `replays` times with an event pair
    around each replay on that stream: the median replay over `iters`, in
    seconds per launch."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        for i in range(iters):
            launch(i)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(replays + 1)]
    with torch.cuda.stream(s):  # replay() launches on the current stream
        for _ in range(warm):
            graph.replay()
        torch.cuda.synchronize()
        ev[0].record(s)
        for r in range(replays):
            graph.replay()
            ev[r + 1].record(s)
    ev[-1].synchronize()
    per = sorted(ev[r].elapsed_time(ev[r + 1]) for r in range(replays))
    del graph
    return per[len(per) // 2] * 1e-3 / iters


def gemm_roofline(ih, model: Model, n_layers: int, M: int, iters: int = 64, replays: int = 15, warm: int = 4):
    """Dominant kernel: the Q4_K gate/up dequant-matmul (24576x4096, M=5)
    over the layers' weights in turn (1.8 GB, far beyond the 256 MB cache),
    as the timed step runs it: with gated weights (the chained step) the
    chained call that loads the operand its producer wrote (rescaled per unit
    in registers) and writes h = silu(gate) up and down's operand
    (algorithmic bytes: weights + operand + h and its operand); otherwise the
    classic call with its activations
    prepared once and reused (weights + x + y). `iters` launches are timed as
    one replayed graph (graph_launch_time): the kernel plus its dispatch gap,
    which is what a kernel trace reports as its duration (its launches run
    back to back). Returns (seconds per launch, algorithmic bytes per
    launch)."""
    import torch
    F, q = ih.formats, ih.quantized_kernels
    N, K = 2 * FF, H
    x = q.synth_gaussian(123, M * K).view(M, K)
    fl = ih.GEMM_F32 | ih.GEMM_PACKED
    ws = torch.empty(q.gemm_ws_bytes(F.Q4_K, M, N, K, fl), dtype=torch.uint8, device="cuda")
    if model.gated:
        # gate/up's operand as the chained o leaves it: here from a producer call on the same
        # residual rows (the first layer's o as the matrix, an input stage), with the RMSNorm sums
        op, ts, ssq = ih.chain_buffers(K, ssq=True)
        y0 = torch.empty((M, K), device="cuda")
        ih.gemm_q_chain(F.Q4_K, model.layers[0]["o"], K, NQ, M, x=x[:, :NQ].contiguous(), ws=ws,
                        cout=ih.chain_out(ih.EPI_STATS, y0, F.Q4_K, op, ts, tile_ssq=ssq, stat_rows=K))
        h = torch.empty((M, FF), device="cuda")
        op_h, _, _ = ih.chain_buffers(FF, tiles_per_unit=32)
        cin = ih.chain_in(op, ts, 16, tile_ssq=ssq, eps=1e-6)
        cout = ih.chain_out(ih.EPI_GATE, h, F.Q6_K, op_h)

        def mat(i):
            ih.gemm_q_chain(F.Q4_K, model.layers[i % n_layers]["gu"], N, K, M, cin=cin, cout=cout, ws=ws)
        # algorithmic bytes: weights, the operand in (split fp16: 4 bytes a value) and h out with its operand
        alg = F.matrix_bytes(F.Q4_K, N, K) + M * K * 4 + M * FF * 8
    else:
        y = torch.empty((M, N), device="cuda")
        ih.gemm_q_ex(F.Q4_K, model.layers[0]["gu"], x, N, K, flags=fl, out=y, ws=ws)  # prepares x

        def mat(i):
            ih.gemm_q_ex(F.Q4_K, model.layers[i % n_layers]["gu"], x, N, K, flags=fl | ih.GEMM_REUSE, out=y, ws=ws)
        alg = F.matrix_bytes(F.Q4_K, N, K) + M * K * 4 + M * N * 4
    t = graph_launch_time(mat, iters, replays, warm)
    return t, alg


def profile_kernels(ih, model: Model, n_layers: int, M: int):
    """For rocprofv3 --pmc: the roofline kernel's graph, then a calibration
    kernel of known traffic (ihip_add over 64 Mi floats: y += x reads 512 MiB,
    writes 256 MiB)."""
    import torch
    gemm_roofline(ih, model, n_layers, M, replays=1, warm=1)
    n = 64 << 20
    a = torch.ones(n, device="cuda")
    b = torch.ones(n, device="cuda")
    for _ in range(3):
        ih.quantized_kernels.add_(a, b)
    torch.cuda.synchronize()
    log(f"profile_kernels: roofline graph + ihip_add over {n} floats")


def profile_m5(ih, reps: int = 5):
    """For rocprofv3 --pmc / --kernel-trace: one config-4 layer's four M = 5
    matmuls as the verify step runs them (input stage + matmul, packed
    weights, fp32-accurate), each launched `reps` times in a row, in the order
    [q; k; v], o (deferred), [gate; up], down (deferred); then the plain-read
    probe over 57,196,544 B (the [gate; up] weights) and 510,504,960 B (the
    lm_head's), `reps` times each, and the calibration kernel (ihip_add over 64
    Mi floats: reads 512 MiB, writes 256 MiB) three times."""
    import torch
    F, q = ih.formats, ih.quantized_kernels
    model = Model(ih, 1, keep_gguf=0)
    step = VerifyStep(ih, model, 5, 4, 0.8)
    lw = model.layers[0]
    ex = ih.gemm_q_ex
    f32 = ih.GEMM_F32 | ih.GEMM_PACKED
    dfr = f32 | ih.GEMM_DEFER
    o_parts = ih.gemm_partials(F.Q4_K, 5, H, NQ, f32, step.ws_o)
    torch.cuda.synchronize()
    for _ in range(reps):
        ex(F.Q4_K, lw["qkv"], step.x, NQ + 2 * NKV, H, act=ih.ACT_RMSNORM, norm_w=lw["attn_norm"], flags=f32,
           out=step.qkv, ws=step.ws)
    for _ in range(reps):
        ex(F.Q4_K, lw["o"], step.qkv[:, :NQ], H, NQ, flags=dfr, ws=step.ws_o)
    for _ in range(reps):
        ex(F.Q4_K, lw["gu"], step.x, 2 * FF, H, act=ih.ACT_RMSNORM, norm_w=lw["ffn_norm"], flags=f32, out=step.gu,
           ws=step.ws, add=o_parts)
    for _ in range(reps):
        ex(F.Q6_K, lw["down"], step.gu, H, FF, act=ih.ACT_SILU_MUL, flags=dfr, ws=step.ws_down)
    torch.cuda.synchronize()
    sink = torch.zeros(2048, dtype=torch.int32, device="cuda")
    for nb in (57_196_544, 510_504_960):
        buf = torch.ones(nb // 4, dtype=torch.float32, device="cuda").view(torch.uint8)
        for _ in range(reps):
            q.stream_read(buf, out=sink)
        torch.cuda.synchronize()
        del buf
    n = 64 << 20
    a = torch.ones(n, device="cuda")
    b = torch.ones(n, device="cuda")
    for _ in range(3):
        q.add_(a, b)
    torch.cuda.synchronize()
    log(f"profile_m5: {reps} x (qkv, o, gate/up, down) at M = 5, stream_read 57 MB and 510 MB, 3 x ihip_add")


def profile_chain(ih, reps: int = 5):
    """For rocprofv3 --pmc / --kernel-trace: one config-4 layer of the chained
    step (M = 5), each call launched `reps` times in a row with the buffers
    the step uses: [q; k; v] with its input stage (RMSNorm) and STATS
    epilogue, o (chained input, RESID epilogue), [gate; up] (chained input,
    GATE epilogue), down (chained input, deferred partials); then the
    plain-read probe over 57,196,544 B and 510,504,960 B and the calibration
    kernel (ihip_add over 64 Mi floats), as profile_m5."""
    import torch
    F, q = ih.formats, ih.quantized_kernels
    model = Model(ih, 1, keep_gguf=0, gated=True)
    step = ChainStep(ih, model, 5, 4, 0.8)
    step.forward()
    torch.cuda.synchronize()
    lw = model.layers[0]
    chain = ih.gemm_q_chain
    fl = ih.GEMM_F32 | ih.GEMM_PACKED
    for _ in range(reps):
        chain(F.Q4_K, lw["qkv"], NQ + 2 * NKV, H, 5, x=step.x, act=ih.ACT_RMSNORM, norm_w=lw["attn_norm"],
              ws=step.ws, cout=step.qkv_out)
    for _ in range(reps):
        chain(F.Q4_K, lw["o"], H, NQ, 5, cin=step.o_in, ws=step.ws_o, cout=step.o_out[0])
    for _ in range(reps):
        chain(F.Q4_K, lw["gu"], 2 * FF, H, 5, ws=step.ws, cin=step.gu_in, cout=step.gu_out)
    for _ in range(reps):
        chain(F.Q6_K, lw["down"], H, FF, 5, cin=step.down_in, flags=fl | ih.GEMM_DEFER, ws=step.ws_down)
    torch.cuda.synchronize()
    sink = torch.zeros(2048, dtype=torch.int32, device="cuda")
    for nb in (57_196_544, 510_504_960):
        buf = torch.ones(nb // 4, dtype=torch.float32, device="cuda").view(torch.uint8)
        for _ in range(reps):
            q.stream_read(buf, out=sink)
        torch.cuda.synchronize()
        del buf
    n = 64 << 20
    a = torch.ones(n, device="cuda")
    b = torch.ones(n, device="cuda")
    for _ in range(3):
        q.add_(a, b)
    torch.cuda.synchronize()
    log(f"profile_chain: {reps} x (qkv, o, gate/up, down) chained at M = 5, stream_read 57 MB and 510 MB, "
        "3 x ihip_add")


def profile_tall(ih, reps: int = 5):
    """For rocprofv3 --pmc: the M = 64 (config 5) half-precision matmuls of
    one layer, each launched `reps` times: Q4_K [gate; up] 24576x4096 with
    the RMSNorm input stage, Q6_K down 4096x12288 with the SiLU-gating
    stage (packed weights, seeded blocks)."""
    import torch
    F, q = ih.formats, ih.quantized_kernels
    st = ih.synth.stream_for
    M = 64
    gu = ih.pack_weights(F.Q4_K, q.synth_blocks(F.Q4_K, st(SEED, "pt.gu"), 2 * FF * H // 256), 2 * FF, H)
    dn = ih.pack_weights(F.Q6_K, q.synth_blocks(F.Q6_K, st(SEED, "pt.down"), H * FF // 256), H, FF)
    x = q.synth_gaussian(st(SEED, "pt.x"), M * H).view(M, H)
    g = q.synth_gaussian(st(SEED, "pt.g"), M * 2 * FF).view(M, 2 * FF)
    for _ in range(reps):
        ih.gemm_q_ex(F.Q4_K, gu, x, 2 * FF, H, act=ih.ACT_RMSNORM, flags=ih.GEMM_PACKED)
        ih.gemm_q_ex(F.Q6_K, dn, g, H, FF, act=ih.ACT_SILU_MUL, flags=ih.GEMM_PACKED)
    torch.cuda.synchronize()
    log(f"profile_tall: {reps} x (gate/up Q4_K 24576x4096, down Q6_K 4096x12288) at M = {M}")


def read_peak(ih, sizes=(57_196_544, 510_504_960, 4_398_624_768), replays: int = 10):
    """The plain-read ceiling beside the vendor peak: GB/s of ihip_stream_read
    (16-byte loads, XOR sink) over buffers of the dominant matmul's weight
    size, the lm_head's and one whole verify step's weights, each timed as the
    median per replay of a graph of 8 launches over rotating copies (cold:
    the copies of the small sizes together exceed the 256 MB cache)."""
    import torch
    out = {}
    for nb in sizes:
        copies = max(1, min(8, int(600e6 // nb) + 1))
        bufs = [torch.empty(nb, dtype=torch.uint8, device="cuda") for _ in range(copies)]
        for b in bufs:
            b.fill_(1)
        sink = torch.zeros(2048, dtype=torch.int32, device="cuda")
        t = graph_launch_time(lambda i: ih.quantized_kernels.stream_read(bufs[i % copies], out=sink), 8, replays, 2)
        out[str(nb)] = round(nb / t / 1e9, 1)
        del bufs
        torch.cuda.empty_cache()
    return out


def read_traffic(chained: bool):
    """HBM bytes per launch of the roofline kernel, from the committed
    rocprofv3 FETCH_SIZE/WRITE_SIZE summary of the kernel this composition
    times (None when absent)."""
    name = "q4k_gemm_24576x4096_m5_traffic.md" if chained else "q4k_gemm_classic_24576x4096_m5_traffic.md"
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def gemm_sweep(ih, model: Model, n_layers: int, launches: int = 32, replays: int = 5, warm: int = 2):
    """GB/s of the Q4_K gate/up and Q6_K down projections at M = 1..8: per M,
    `launches` matmuls over the layers' weights in turn (cold: 1.8 GB and
    1.3 GB, far beyond the caches) timed as one replayed graph
    (graph_launch_time; per launch, dispatch gap included); and the same at
    the lm_head's shape in both formats (8 launches of one 350 / 510 MB
    matrix), where the per-launch fixed cost is amortized."""
    import torch
    F = ih.formats
    out = {}
    # the lm_head shape (151936 x 4096: 510 MB in Q6_K, 350 MB in Q4_K, each
    # beyond the 256 MB cache, so repeated launches stream it from HBM): the
    # model's own lm_head, and a Q4_K matrix of that shape made for the sweep
    big_q4k = ih.pack_weights(F.Q4_K, ih.quantized_kernels.synth_blocks(
        F.Q4_K, ih.synth.stream_for(SEED, "sweep_q4k_big"), VOCAB * H // 256), VOCAB, H)
    mats = {"gu": [lw["gu"] for lw in model.layers[:n_layers]], "down": [lw["down"] for lw in model.layers[:n_layers]],
            "lm": [model.lm], "big_q4k": [big_q4k]}
    for name, key, qt, N, K, n_launch in (("q4k_24576x4096", "gu", F.Q4_K, 2 * FF, H, launches),
                                          ("q6k_4096x12288", "down", F.Q6_K, H, FF, launches),
                                          ("q4k_151936x4096", "big_q4k", F.Q4_K, VOCAB, H, 8),
                                          ("q6k_151936x4096", "lm", F.Q6_K, VOCAB, H, 8)):
        row = {}
        ws_list = mats[key]
        for M in (1, 2, 4, 5, 8):
            x = ih.quantized_kernels.synth_gaussian(7 + M, M * K).view(M, K)
            y = torch.empty((M, N), device="cuda")
            fl = ih.GEMM_F32 | ih.GEMM_PACKED
            ws = torch.empty(ih.quantized_kernels.gemm_ws_bytes(qt, M, N, K, fl), dtype=torch.uint8, device="cuda")
            ih.gemm_q_ex(qt, ws_list[0], x, N, K, flags=fl, out=y, ws=ws)  # prepares x

            def mat(i):
                ih.gemm_q_ex(qt, ws_list[i % len(ws_list)], x, N, K, flags=fl | ih.GEMM_REUSE, out=y, ws=ws)

            t = graph_launch_time(mat, n_launch, replays, warm)
            gbs = (F.matrix_bytes(qt, N, K) + M * K * 4 + M * N * 4) / t / 1e9
            row[str(M)] = round(gbs, 1)
        out[name] = row
    del big_q4k
    torch.cuda.empty_cache()
    return out


def graph_time(fn, replays: int = 5):
    """Seconds per replay of a HIP graph of fn()'s launches (captured once on a
    side stream after one eager run), timed with events on that stream."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        fn()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(s):
        graph.replay()
        torch.cuda.synchronize()
        e0.record(s)
        for _ in range(replays):
            graph.replay()
        e1.record(s)
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / replays


def config1(ih):
    """Config 1: one Q4_K GEMV, W[3072 x 1024], M = 1; cold (a graph over
    >= 300 MB of weight copies, beyond the 256 MB infinity cache) and warm
    (one copy). 'call' is the whole ihip_gemm_q call (input stage + matmul),
    'matmul' the matmul kernel with the input prepared once."""
    import torch
    F = ih.formats
    N, K = 3072, 1024
    wb = F.matrix_bytes(F.Q4_K, N, K)
    copies = int(300e6 // wb) + 1
    ws_ = [ih.pack_weights(F.Q4_K, ih.quantized_kernels.synth_blocks(F.Q4_K, ih.synth.stream_for(SEED - 2, f"c1.{c}"),
                                                                     N * K // 256), N, K) for c in range(copies)]
    x = ih.quantized_kernels.synth_gaussian(ih.synth.stream_for(SEED - 2, "x"), K).view(1, K)
    y = torch.empty((1, N), device="cuda")
    fl = ih.GEMM_F32 | ih.GEMM_PACKED
    wsp = torch.empty(ih.quantized_kernels.gemm_ws_bytes(F.Q4_K, 1, N, K, fl), dtype=torch.uint8, device="cuda")
    alg = wb + K * 4 + N * 4
    out = {"weight_bytes": wb, "algorithmic_bytes": alg}
    for mode, pick in (("cold", lambda i: ws_[i % copies]), ("warm", lambda i: ws_[0])):
        for kind, extra in (("call", 0), ("matmul", ih.GEMM_REUSE)):
            ih.gemm_q_ex(F.Q4_K, ws_[0], x, N, K, flags=fl, out=y, ws=wsp)
            t = graph_time(lambda: [ih.gemm_q_ex(F.Q4_K, pick(i), x, N, K, flags=fl | extra, out=y, ws=wsp)
                                    for i in range(copies)]) / copies
            out[f"{mode}_{kind}_us"] = round(t * 1e6, 2)
            out[f"{mode}_{kind}_GBps"] = round(alg / t / 1e9, 1)
    del ws_
    return out


def config2(ih):
    """Config 2: one verify batch at M = 5, hidden 2048: Q4_K q 2048x2048,
    k/v 512x2048, o 2048x2048, gate/up 6144x2048, Q6_K down 2048x6144, Q8_0
    2048x2048, cold over >= 300 MB of weight sets. Matrices that read the
    same input in a layer are one packed matrix, as in the verify step
    ([q; k; v], [gate; up]): five matmuls, each with its own input stage."""
    import torch
    F = ih.formats
    M, Hd, Fd = 5, 2048, 6144
    mats = [("q", F.Q4_K, Hd, Hd), ("k", F.Q4_K, 512, Hd), ("v", F.Q4_K, 512, Hd), ("o", F.Q4_K, Hd, Hd),
            ("gate", F.Q4_K, Fd, Hd), ("up", F.Q4_K, Fd, Hd), ("down", F.Q6_K, Hd, Fd), ("q8", F.Q8_0, Hd, Hd)]
    set_bytes = sum(F.matrix_bytes(qt, n, k) for _, qt, n, k in mats)
    sets = int(300e6 // set_bytes) + 1
    st = ih.synth.stream_for
    W = []
    for c in range(sets):
        w = {name: ih.pack_weights(qt, ih.quantized_kernels.synth_blocks(qt, st(SEED - 1, f"c2.{c}.{name}"),
                                                                        n * k // F.BLOCK_ELEMS[qt]), n, k)
             for name, qt, n, k in mats}
        # (the packed layout concatenates along 16-row tiles)
        W.append({"qkv": torch.cat([w["q"], w["k"], w["v"]]), "o": w["o"], "gu": torch.cat([w["gate"], w["up"]]),
                  "down": w["down"], "q8": w["q8"]})
        del w
    calls = [("qkv", F.Q4_K, Hd + 1024, Hd), ("o", F.Q4_K, Hd, Hd), ("gu", F.Q4_K, 2 * Fd, Hd),
             ("down", F.Q6_K, Hd, Fd), ("q8", F.Q8_0, Hd, Hd)]
    x = ih.quantized_kernels.synth_gaussian(st(SEED - 1, "x"), M * Hd).view(M, Hd)
    xf = ih.quantized_kernels.synth_gaussian(st(SEED - 1, "xf"), M * Fd).view(M, Fd)
    fl = ih.GEMM_F32 | ih.GEMM_PACKED
    ys = {name: torch.empty((M, n), device="cuda") for name, _, n, _ in calls}
    wsb = max(ih.quantized_kernels.gemm_ws_bytes(qt, M, n, k, fl) for _, qt, n, k in calls)
    wsp = torch.empty(wsb, dtype=torch.uint8, device="cuda")

    def batch():
        for c in range(sets):
            for name, qt, n, k in calls:
                ih.gemm_q_ex(qt, W[c][name], xf if name == "down" else x, n, k, flags=fl, out=ys[name], ws=wsp)
    t = graph_time(batch) / sets
    alg = set_bytes + sum(M * k * 4 + M * n * 4 for _, _, n, k in mats)
    del W
    return {"us_per_batch": round(t * 1e6, 2), "weight_bytes": set_bytes, "algorithmic_bytes": alg,
            "GBps": round(alg / t / 1e9, 1), "frac": round(alg / t / 1e9 / HBM_PEAK_GBPS, 4)}


def config3(ih, n_steps: int = 4096, per_call: int = 6):
    """Config 3: Q6_K lm_head 151936x2048 + rejection-sampling accept over
    n_steps independent verify steps (k = 4, T = 0.8, fresh hidden states per
    step). The target rows of `per_call` steps share one fp32-accurate matmul
    (5 per_call <= 32 rows) and one accept call covers all steps; inputs are
    resident in HBM (draft logits = target + N(0, 1.5^2), draft tokens drawn
    from them beforehand)."""
    import torch
    F = ih.formats
    Hd, k, T = 2048, 4, 0.8
    st = ih.synth.stream_for
    lm = ih.pack_weights(F.Q6_K, ih.quantized_kernels.synth_blocks(F.Q6_K, st(SEED - 3, "output"),
                                                                   VOCAB * Hd // 256), VOCAB, Hd)
    rows = n_steps * (k + 1)
    Hs = ih.quantized_kernels.synth_gaussian(st(SEED - 3, "h"), rows * Hd).view(rows, Hd)
    Lt = torch.empty((rows, VOCAB), device="cuda")
    fl = ih.GEMM_F32 | ih.GEMM_PACKED
    m = per_call * (k + 1)
    wsp = torch.empty(ih.quantized_kernels.gemm_ws_bytes(F.Q6_K, m, VOCAB, Hd, fl), dtype=torch.uint8, device="cuda")
    calls = [(r0, min(m, rows - r0)) for r0 in range(0, rows, m)]

    def gemms():
        for r0, mm in calls:
            ih.gemm_q_ex(F.Q6_K, lm, Hs[r0:r0 + mm], VOCAB, Hd, flags=fl, out=Lt[r0:r0 + mm], ws=wsp)
    gemms()
    torch.cuda.synchronize()
    L3 = Lt.view(n_steps, k + 1, VOCAB)
    Ld = torch.empty((n_steps, k, VOCAB), device="cuda")
    g = torch.Generator(device="cuda").manual_seed(SEED + 3)
    draft = torch.empty((n_steps, k), dtype=torch.int32, device="cuda")
    for s0 in range(0, n_steps, 256):
        blk = L3[s0:s0 + 256, :k].contiguous()
        ih.quantized_kernels.synth_gaussian(st(SEED - 3, f"d{s0}"), blk.numel(), 1.5, add=blk,
                                            out=Ld[s0:s0 + 256].view(-1))
        p = torch.softmax(Ld[s0:s0 + 256].view(-1, VOCAB) / T, -1)
        draft[s0:s0 + 256] = torch.multinomial(p, 1, generator=g).view(-1, k).to(torch.int32)
        del p
    u_acc = torch.rand((n_steps, k), generator=g, device="cuda")
    u_res = torch.rand(n_steps, generator=g, device="cuda")
    u_bon = torch.rand(n_steps, generator=g, device="cuda")
    nb = C.c_size_t()
    ih._lib.check(ih.load().ihip_spec_accept_ws_bytes(n_steps, k, VOCAB, C.byref(nb)))
    aws = torch.empty(nb.value, dtype=torch.uint8, device="cuda")
    out_tok = torch.zeros((n_steps, k + 1), dtype=torch.int32, device="cuda")
    out_n = torch.zeros(n_steps, dtype=torch.int32, device="cuda")

    def accept():
        ih.spec_accept(L3, Ld, draft, T, u_acc, u_res, u_bon, out_tok=out_tok, out_n=out_n, ws=aws)

    t_gemm = graph_time(gemms, replays=2)
    t_acc = graph_time(accept, replays=2)
    acc_rate = float(out_n.double().mean()) / k
    alg = len(calls) * F.matrix_bytes(F.Q6_K, VOCAB, Hd) + rows * Hd * 4 + rows * VOCAB * 4
    del Lt, Ld, Hs
    return {"steps": n_steps, "steps_per_matmul": per_call, "ms_matmuls": round(t_gemm * 1e3, 3),
            "ms_accept": round(t_acc * 1e3, 3), "steps_per_s": round(n_steps / (t_gemm + t_acc), 1),
            "matmul_GBps": round(alg / t_gemm / 1e9, 1), "mean_accepted_fraction": round(acc_rate, 4)}


def config4(ih, model: Model, replays: int = 20):
    """Config 4 across its token counts: the full verify step (32 layers,
    lm_head, accept at T = 0.8) at M = 1, 2, 4, 5, 8 with k = M - 1 drafts;
    M = 1 has no draft, so it is the forward alone (a plain decode step).
    fp32-accurate at every M (one token tile)."""
    import torch
    out = {}
    for M in (1, 2, 4, 5, 8):
        k = M - 1
        make = ChainStep if model.gated else VerifyStep
        step = make(ih, model, M, max(k, 1), 0.8)  # (M = 1: the draft side is set up, not used)
        t = graph_time(step.forward if k == 0 else step.run, replays=replays)
        w = model.weight_bytes(len(model.layers))
        out[str(M)] = {"k": k, "ms_per_step": round(t * 1e3, 4), "steps_per_s": round(1 / t, 1),
                       "weight_GBps": round(w / t / 1e9, 1)}
        del step
        torch.cuda.empty_cache()
    return out


def config5(ih, model: Model):
    """Config 5: 64-node tree verify (32 layers and the lm_head at M = 64 on
    the half-precision MFMA path, then the tree accept walk), with the
    projections in Q4_K (the config-4 model) and again in Q5_K."""
    import torch
    F = ih.formats

    def measure(m: Model):
        step = TreeStep(ih, m)
        t = graph_time(step.run, replays=5)
        t_fwd = graph_time(step.forward, replays=5)
        P = m.proj
        weights = sum(F.matrix_bytes(qt, n, k) // F.BLOCK_BYTES[qt] * F.BLOCK_ELEMS[qt]
                      for qt, n, k in [(P, NQ + 2 * NKV, H), (P, H, NQ), (P, 2 * FF, H),
                                       (F.Q6_K, H, FF)]) * len(m.layers) + VOCAB * H
        flops = 2 * 64 * weights
        return {"ms_per_tree": round(t * 1e3, 3), "trees_per_s": round(1 / t, 2),
                "ms_forward": round(t_fwd * 1e3, 3), "forward_TFLOPs": round(flops / t_fwd / 1e12, 1),
                "mfma_frac_fp16_dense": round(flops / t_fwd / 2.5e15, 4),
                "forward_GBps": round(m.weight_bytes(len(m.layers)) / t_fwd / 1e9, 1),
                "accepted_path_len": int(step.plen[0])}

    out = measure(model)
    m5 = Model(ih, len(model.layers), keep_gguf=0, proj="Q5_K")
    out["q5k_projections"] = measure(m5)
    del m5
    torch.cuda.empty_cache()
    return out


def cpu_topology() -> dict:
    """The host CPU as lscpu reports it (model, sockets, cores per socket,
    threads per core, NUMA nodes), the logical CPUs of the machine and of
    this process's affinity mask, and the physical cores behind the latter
    (distinct (package, core id) pairs in /sys)."""
    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            info[key.strip()] = val.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    aff = sorted(os.sched_getaffinity(0))
    cores = set()
    for c in aff:
        base = f"/sys/devices/system/cpu/cpu{c}/topology/"
        try:
            with open(base + "physical_package_id") as f1, open(base + "core_id") as f2:
                cores.add((f1.read().strip(), f2.read().strip()))
        except OSError:
            cores.add(("?", str(c)))
    num = lambda k: int(info[k]) if info.get(k, "").isdigit() else None  # noqa: E731
    return {"model": info.get("Model name"), "sockets": num("Socket(s)"),
            "cores_per_socket": num("Core(s) per socket"), "threads_per_core": num("Thread(s) per core"),
            "numa_nodes": num("NUMA node(s)"), "logical_cpus": os.cpu_count(), "affinity_cpus": len(aff),
            "physical_cores_in_affinity": len(cores)}


def cpu_baseline(ih, model: Model, n_layers: int, M: int, k: int, budget_s: float):
    """The reference CPU path on a bounded sample: S_L layers + lm_head + accept,
    scaled to the full step. The reference's own C kernels (oracle/_ref, kind
    "reference"; the oracle's port if that build is absent) driven by a C
    loop in forward_cpu!'s order with preallocated buffers and C RMSNorm /
    SiLU (orc_cpu_verify_step), as cheap as the Julia host's ccall glue.
    Timed at all physical cores of this process's CPUs (the figure the
    ratio is quoted against) and at the reference's default thread count
    clamp(Sys.CPU_THREADS / 2, 2, 8) (src/QuantizedKernels.jl:40-41); the
    kernel-only time (inside the gemv calls) beside each, and once the
    previous Python-glue driver for comparison."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    F = ih.formats
    kind = "reference" if O.ref_available() else "port"
    sample_layers = min(len(model.host_gguf), n_layers)
    hostw = model.host_gguf[:sample_layers]
    lm = model.host_lm
    rng = np.random.default_rng(0)
    x0 = rng.standard_normal((M, H)).astype(np.float32)
    Ld = rng.standard_normal((k, VOCAB)).astype(np.float32) * 3
    draft = Ld.argmax(-1).astype(np.int32)
    u_acc = np.zeros(k, np.float32)  # every draft accepted, then the bonus: the GPU's timed step (n = 4)
    topo = cpu_topology()

    gomp = None
    for name in ("libgomp.so.1", "libgomp.so"):
        try:
            gomp = C.CDLL(name)
            break
        except OSError:
            pass
    phys = topo["physical_cores_in_affinity"]
    ref_default = max(2, min(8, (os.cpu_count() or 2) // 2))  # src/QuantizedKernels.jl:40
    scale = n_layers / sample_layers

    def run_c():
        _, _, n, sl, sh, sg = O.cpu_verify_step(hostw, lm, model.host_out_norm, x0, H, NQ, NKV, FF, VOCAB, Ld,
                                                draft, 0.8, u_acc, 0.5, 0.5, kernels=kind)
        return sl * scale + sh, sg[0] * scale + sg[1], sg[2]

    counts = sorted({ref_default, phys})
    per = budget_s * 0.8 / len(counts)
    results = {}
    for threads in counts:
        if gomp is not None:
            gomp.omp_set_num_threads(threads)
        run_c()  # warm-up
        tot, ker, acc, reps = 0.0, 0.0, 0.0, 0
        t_end = time.perf_counter() + per
        while time.perf_counter() < t_end or reps == 0:
            a, b, c = run_c()
            tot += a
            ker += b
            acc += c
            reps += 1
        results[threads] = (tot / reps, ker / reps, acc / reps, reps)
        log(f"cpu baseline (C driver) threads={threads}: {tot / reps * 1e3:.1f} ms/step, "
            f"{ker / reps * 1e3:.1f} ms inside the gemv calls, {acc / reps * 1e3:.1f} ms accept ({reps} samples)")

    # the previous driver: the same kernels called from Python with numpy glue
    gemv = (lambda qt, w, v, K, N: O.ref_gemv(qt, w, v, K, N)) if kind == "reference" else \
        (lambda qt, w, v, K, N: O.gemv_q8k(qt, w, v, K, N, phys))  # noqa: E731

    def rms(v, w):
        return (v / np.sqrt((v.astype(np.float64) ** 2).mean() + 1e-6) * w).astype(np.float32)

    def py_step():
        with np.errstate(over="ignore"):
            x = x0.copy()
            t0 = time.perf_counter()
            for m in range(M):  # token-major, as forward_cpu! and the C driver
                for lw in hostw:
                    h = rms(x[m], lw["attn_norm"])
                    q = gemv(F.Q4_K, lw["q"], h, H, NQ)
                    gemv(F.Q4_K, lw["kv"], h, H, 2 * NKV)
                    x[m] += gemv(F.Q4_K, lw["o"], q, NQ, H)
                    h = rms(x[m], lw["ffn_norm"])
                    gu = gemv(F.Q4_K, lw["gu"], h, H, 2 * FF)
                    g, u = gu[:FF], gu[FF:]
                    x[m] += gemv(F.Q6_K, lw["down"], (g / (1 + np.exp(-g)) * u).astype(np.float32), FF, H)
            t1 = time.perf_counter()
            for m in range(M):
                gemv(F.Q6_K, lm, rms(x[m], model.host_out_norm), H, VOCAB)
            return (t1 - t0) * scale + time.perf_counter() - t1

    if gomp is not None:
        gomp.omp_set_num_threads(phys)
    py_step()
    py, reps_py, t_end = 0.0, 0, time.perf_counter() + budget_s * 0.2
    while time.perf_counter() < t_end or reps_py == 0:
        py += py_step()
        reps_py += 1
    py /= reps_py
    log(f"cpu baseline (Python glue) threads={phys}: {py * 1e3:.1f} ms/step without the accept ({reps_py} samples)")
    best = results[phys]
    return {
        "value": round(1.0 / best[0], 4),
        "unit": "verify steps/s",
        "cores": phys,
        "kind": kind,
        "sample": (f"{sample_layers} of {n_layers} layers, M={M} tokens each through every layer in forward_cpu!'s "
                   f"token-major order (q, k, v, o, gate, up, down per token and layer: the reference's C gemv "
                   f"with a preallocated Q8_K buffer; C RMSNorm, SiLU and residual adds), scaled to {n_layers} "
                   f"layers, + final RMSNorm and lm_head x{M} + accept (mode 0, all {k} drafts accepted, bonus draw); "
                   f"one thread count per figure, OpenMP inside the kernels"),
        "threads": {str(t): {"steps_per_s": round(1.0 / r[0], 4), "ms_per_step": round(r[0] * 1e3, 2),
                             "ms_in_gemv": round(r[1] * 1e3, 2), "ms_accept": round(r[2] * 1e3, 2),
                             "samples": r[3]} for t, r in results.items()},
        "reference_default_threads": ref_default,
        "python_glue_ms_per_step_no_accept": round(py * 1e3, 2),
        "host": topo,
    }


def sampler_config(ih):
    """The draft-side sampler (ihip_sample_ex: softmax_sample, src/ModelCPU.jl:
    1123-1200; ihip_apply_penalties: :1202-1225) at the LM head's vocabulary
    V = 151936: microseconds per call for 1 and 64 rows (seeded Gaussian
    logits, sd 3), each call replayed in a HIP graph, every setting but
    top-k 50 + top-p also with one workgroup per row (ihip_sample); beside it the oracle's numpy
    restatement of one row on the host (argsorts for top-k/top-p)."""
    import torch
    import numpy as np
    V = 151936
    settings = {"plain": dict(temperature=1.0), "top_k=40": dict(temperature=0.8, top_k=40),
                "top_k=50,top_p=0.95": dict(temperature=0.7, top_k=50, top_p=0.95),
                "top_p=0.9": dict(temperature=0.8, top_p=0.9), "min_p=0.05": dict(temperature=1.0, min_p=0.05),
                "top_p=0.9,min_p=0.02": dict(temperature=0.8, top_p=0.9, min_p=0.02),
                "top_k=1000": dict(temperature=0.8, top_k=1000),
                "greedy": dict(temperature=0.0)}
    g = torch.Generator(device="cuda").manual_seed(SEED)
    out = {"V": V, "us_per_call": {}}
    for rows in (1, 64):
        L = 3.0 * torch.randn(rows, V, device="cuda", generator=g)
        u = torch.rand(rows, device="cuda", generator=g)
        tok = torch.empty(rows, dtype=torch.int32, device="cuda")
        ws = torch.empty(ih.sample_ws_bytes(rows, V), dtype=torch.uint8, device="cuda")
        for name, kw in settings.items():
            t = graph_time(lambda: [ih.softmax_sample(L, u, out=tok, ws=ws, **kw) for _ in range(10)]) / 10
            out["us_per_call"][f"rows={rows},{name}"] = round(t * 1e6, 1)
        for name in ("plain", "top_k=40", "top_p=0.9", "min_p=0.05", "top_p=0.9,min_p=0.02", "top_k=1000", "greedy"):
            kw = settings[name]
            t = graph_time(lambda: [ih.softmax_sample(L, u, out=tok, spread=False, **kw) for _ in range(10)]) / 10
            out["us_per_call"][f"rows={rows},{name},one_workgroup"] = round(t * 1e6, 1)
        ids = torch.arange(0, 4096, 7, dtype=torch.int32, device="cuda")
        t = graph_time(lambda: [ih.apply_penalties_(L, ids, presence=0.1, repetition=1.1) for _ in range(10)]) / 10
        out["us_per_call"][f"rows={rows},penalties(586 ids)"] = round(t * 1e6, 1)
    # host: the oracle's numpy restatement, one row per setting
    try:
        sys.path.insert(0, ROOT)
        from oracle import oracle as O
        row = (3.0 * np.random.default_rng(SEED).standard_normal(V)).astype(np.float32)
        cpu = {}
        for name, kw in settings.items():
            t0 = time.perf_counter()
            O.softmax_sample(row, 0.5, **kw)
            cpu[name] = round((time.perf_counter() - t0) * 1e3, 2)
        out["cpu_port_ms_per_row"] = cpu
    except Exception as e:  # (the oracle is test infrastructure; absent means no baseline)
        out["cpu_port_ms_per_row"] = f"unavailable: {e}"
    return out


def gguf_config(ih):
    """GGUF file -> device weights (ihip_gguf_upload, the loader of
    src/GGUF.jl + src/LoaderCPU.jl:120-175): a 604 MB file of eight Q4_K
    matrices 16384 x 8192 (seeded bytes) written to local disk, read back
    (page cache warm after one pass) and uploaded plain and packed; GB/s of
    file bytes per second, whole call (host memcpy from the mapping into
    pinned staging, DMA, and for packed the device repack)."""
    import tempfile
    import torch
    import numpy as np
    N, K = 16384, 8192
    rng = np.random.default_rng(SEED)
    nb = N * K // 256 * 144
    blob = rng.integers(0, 256, size=nb, dtype=np.uint8).tobytes()
    out = {"file_bytes": 0}
    with tempfile.TemporaryDirectory(dir=os.environ.get("TMPDIR", "/tmp")) as d:
        path = os.path.join(d, "w.gguf")
        ih.gguf.write_gguf(path, [("general.architecture", ih.gguf.GGUF_TYPE_STRING, "bench")],
                           [(f"blk.{i}.w", (K, N), ih.formats.Q4_K, blob) for i in range(8)])
        out["file_bytes"] = os.path.getsize(path)
        with ih.gguf.read_gguf(path) as f:
            dev = torch.empty(max(nb, ih.quantized_kernels.packed_bytes(ih.formats.Q4_K, N, K)), dtype=torch.uint8,
                              device="cuda")
            for name in f.tensors:  # warm the page cache
                f.upload(name, out=dev)
            for mode, packed in (("plain", False), ("packed", True)):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for name in f.tensors:
                    f.upload(name, packed=packed, out=dev)
                torch.cuda.synchronize()
                dt = time.perf_counter() - t0
                out[f"{mode}_GBps"] = round(8 * nb / dt / 1e9, 2)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--m", type=int, default=5)
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU-baseline work")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--classic", action="store_true",
                    help="time the verify step with an input stage before every matmul (no chained matmuls)")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--profile-kernels", action="store_true",
                    help="only run the roofline kernel and the traffic calibration kernel (for rocprofv3 --pmc)")
    ap.add_argument("--profile-m5", action="store_true",
                    help="only run one layer's four M = 5 matmuls five times each, the plain-read probe and the "
                         "traffic calibration kernel (for rocprofv3 --pmc)")
    ap.add_argument("--profile-chain", action="store_true",
                    help="only run one chained layer's four M = 5 calls five times each, the plain-read probe and "
                         "the traffic calibration kernel (for rocprofv3 --pmc)")
    ap.add_argument("--profile-tall", action="store_true",
                    help="only run the M = 64 gate/up and down matmuls five times each (for rocprofv3 --pmc)")
    ap.add_argument("--configs", type=str, default="",
                    help="instead of the bench line: measure BASELINE configs (comma list of 1,2,3,4,5, 'sampler' "
                         "for the draft-side sampler, 'gguf' for file-to-device loading), one JSON object per config")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(see the sharding design); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    import inferno_hip as ih
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    assert ih.quant_kernels_available(), ih._lib.last_error()
    k, T = 4, 0.8
    t0 = time.time()
    if args.profile_tall:
        profile_tall(ih)
        return
    if args.profile_m5:
        profile_m5(ih)
        return
    if args.profile_chain:
        profile_chain(ih)
        return
    if args.configs:
        want = [c.strip() for c in args.configs.split(",") if c.strip()]
        for c in want:
            if c == "5":
                res = config5(ih, Model(ih, args.layers, keep_gguf=0))
            elif c == "4":
                res = config4(ih, Model(ih, args.layers, keep_gguf=0, gated=not args.classic))
            elif c == "sampler":
                res = sampler_config(ih)
            elif c == "gguf":
                res = gguf_config(ih)
            else:
                res = {"1": config1, "2": config2, "3": config3}[c](ih)
            print(json.dumps({"config": c if c in ("sampler", "gguf") else int(c), **res}), flush=True)
            torch.cuda.empty_cache()
        return
    chained = not args.classic and args.m <= 8
    model = Model(ih, args.layers, keep_gguf=0 if (args.no_cpu or args.profile_kernels) else 4, gated=chained)
    step = ChainStep(ih, model, args.m, k, T) if chained else VerifyStep(ih, model, args.m, k, T)
    log(f"setup {time.time() - t0:.1f}s, weights {model.weight_bytes(args.layers) / 1e9:.3f} GB")
    if args.profile_kernels:
        profile_kernels(ih, model, args.layers, args.m)
        return

    # capture one step in a HIP graph
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step.run()
        step.run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        step.run()
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    ms = e0.elapsed_time(e1) / args.steps
    log(f"verify step: {ms:.3f} ms (wall {wall / args.steps * 1e3:.3f} ms), accepted n={int(step.out_n[0])}")

    hist = step.accept_histogram()
    log(f"accepted lengths over 256 draws on the step's logits: {hist}")
    acc_us, acc_us_spread, hist_spread = accept_cost(ih, step)
    log(f"accept alone: {acc_us} us on the step's logits, {acc_us_spread} us on spread rows "
        f"(accepted lengths there over 256 draws: {hist_spread})")
    t_op, alg = gemm_roofline(ih, model, args.layers, args.m)
    achieved = alg / t_op / 1e9
    peaks = read_peak(ih)
    log(f"plain-read ceiling (GB/s by buffer bytes): {peaks}")
    sweep = None if args.no_sweep else gemm_sweep(ih, model, args.layers)
    cpu = None if args.no_cpu else cpu_baseline(ih, model, args.layers, args.m, k, args.cpu_budget)

    out = {
        "metric": METRIC,
        "value": round(1000.0 / ms, 3),
        "unit": "verify steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (split-f16 MFMA operands, f32 accumulate)",
        "data": "synthetic (seeded GGUF blocks and activations, random-init, no checkpoint offline)",
        "config": {
            "workload": "configs[3]: full verify step, 32 layers hidden 4096 (Q4_K q/k/v/o/gate/up, "
                        "Q6_K down), Q6_K lm_head 151936x4096, M=5, k=4 accept at T=0.8",
            "layers": args.layers, "hidden": H, "vocab": VOCAB, "M": args.m, "k": k,
            "weight_bytes_per_step": model.weight_bytes(args.layers),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": read_traffic(model.gated),
            "kernel": ("gemm_v_kernel<Q4_K, chained input>: packed Q4_K [gate; up] dequant-matmul 24576x4096, "
                       "M=5, fp32-accurate, operand written by its producer (rescaled per unit in registers), "
                       "h = silu(gate) up and down's operand out"
                       if model.gated else
                       "gemm_v_kernel<Q4_K>: packed Q4_K dequant-matmul 24576x4096, M=5, fp32-accurate "
                       "(activations prepared once)") +
                      "; per launch in a replayed graph of 64 launches over cold "
                      "weights, median of 15 replays, HIP events (dispatch gap included, as in a kernel trace)",
            "step_composition": "chained (one input stage per layer)" if chained else "classic (input stage per matmul)",
            "us_per_launch": round(t_op * 1e6, 2),
            "algorithmic_bytes": alg,
            "measured_peak": max(peaks.values()),
            "measured_peak_by_bytes": peaks,
            "frac_of_measured_peak": round(achieved / max(peaks.values()), 4),
            "step_frac": round(model.weight_bytes(args.layers) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
            "step_GBps": round(model.weight_bytes(args.layers) / (ms * 1e-3) / 1e9, 1),
        },
        "accept": {"timed_step_accepted": int(step.out_n[0]),
                   "accepted_length_histogram_256_draws": hist,
                   "draft_logits": "target + N(0, 1.5^2)",
                   "us_per_accept_step_logits": acc_us,
                   "us_per_accept_spread_logits": acc_us_spread,
                   "spread_logits": "target ~ N(0, 4^2), draft = target + N(0, 1.5^2), same M, k, V, T",
                   "accepted_length_histogram_256_draws_spread": hist_spread},
        "cpu_baseline": cpu,
        "gemm_gbps_by_M": sweep,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
