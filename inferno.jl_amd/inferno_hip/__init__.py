"""inferno_hip: MI355X (gfx950) speculative-verify hot path of Inferno.jl.

Host mirror of the reference's QuantizedKernels (quantized GEMV) and
SpeculativeDecoding (verify / accept) interfaces over the C ABI in
include/inferno_hip.h, implemented by hand-written HIP kernels in
lib/libinferno_hip.so. There is no CPU fallback.
"""
from . import formats, gguf, synth
from ._lib import HipError, load
from .quantized_kernels import (ACT_PLAIN, ACT_RMSNORM, ACT_SILU_MUL, EPI_GATE, EPI_RESID, EPI_STATS, EPI_STORE,
                                GEMM_ACCUM, GEMM_AUTO, GEMM_F32, GEMM_HALF, GEMM_DEFER, GEMM_PACKED, GEMM_REUSE, GEMM_SUM_OUT,
                                chain_buffers, chain_in, chain_operand_bytes, chain_out, dequant, gemm_partials, gemm_q, gemm_q_chain,
                                gemm_q_ex, pack_weights_gated,
                                mlp_forward_, mlp_ws_bytes, pack_weights, packed_bytes, q4_k_gemv_, q5_k_gemv_, q6_k_gemv_, q8_0_gemv_,
                                quant_kernels_available, rmsnorm)
from .sampler import apply_penalties_, sample_ws_bytes, softmax_sample
from .speculative import (MODE_REFERENCE, MODE_STANDARD, SpeculativeStats, advance_len_, commit_state_, greedy_verify,
                          mtp_verify_step, n_tokens, softmax_stats, spec_accept, tree_accept)

__all__ = [
    "formats", "gguf", "synth", "HipError", "load", "GEMM_ACCUM", "GEMM_AUTO", "GEMM_F32", "GEMM_HALF",
    "GEMM_PACKED", "GEMM_REUSE", "GEMM_DEFER", "GEMM_SUM_OUT", "gemm_partials", "ACT_PLAIN", "ACT_RMSNORM", "ACT_SILU_MUL", "dequant", "gemm_q", "gemm_q_ex",
    "mlp_forward_", "mlp_ws_bytes", "pack_weights", "packed_bytes", "q4_k_gemv_", "q5_k_gemv_", "q6_k_gemv_", "q8_0_gemv_",
    "quant_kernels_available", "rmsnorm", "EPI_STORE", "EPI_STATS", "EPI_RESID", "EPI_GATE", "chain_in",
    "chain_out", "chain_buffers", "chain_operand_bytes", "gemm_q_chain", "pack_weights_gated", "MODE_REFERENCE", "MODE_STANDARD", "SpeculativeStats",
    "greedy_verify", "mtp_verify_step", "n_tokens", "softmax_stats", "spec_accept", "tree_accept",
    "softmax_sample", "sample_ws_bytes", "apply_penalties_", "commit_state_", "advance_len_",
]
