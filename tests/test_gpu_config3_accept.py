"""GPU parity of configs[2]'s 4096 independent verify steps at the real
vocabulary: Q6_K lm_head 151936 x 2048 target logits from seeded hidden
states (the fp32-accurate matmul, six steps per 30-row call, as the
benchmark batches them), draft logits = target + N(0, 1.5^2), k = 4 drafts
drawn from the draft softmax at T = 0.8, explicit uniforms; every step
through ihip_spec_accept in both modes against the oracle's accept
(src/SpeculativeDecoding.jl:37-107) on the same logits, streamed to the host
in batches of 256 steps. accepted lengths identical on
>= 99.9 % of steps; the resampled / bonus tokens are compared too."""
import numpy as np
import pytest

import oracle as O
from inferno_hip import formats as F

pytestmark = pytest.mark.gpu

STEPS, K, T, V, HD = 4096, 4, 0.8, 151936, 2048
BATCH = 256


@pytest.fixture(scope="module")
def ih():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import inferno_hip
    assert inferno_hip.quant_kernels_available(), inferno_hip._lib.last_error()
    return inferno_hip


@pytest.fixture(scope="module")
def case(ih):
    """Device-resident inputs of the 4096 steps (20 GB of logits in HBM)."""
    import torch
    q = ih.quantized_kernels
    st = ih.synth.stream_for
    seed = 0x1F3E0003
    lm = ih.pack_weights(F.Q6_K, q.synth_blocks(F.Q6_K, st(seed, "acc4096.lm"), V * HD // 256), V, HD)
    rows = STEPS * (K + 1)
    Hs = q.synth_gaussian(st(seed, "acc4096.h"), rows * HD).view(rows, HD)
    Lt = torch.empty((rows, V), device="cuda")
    fl = ih.GEMM_F32 | ih.GEMM_PACKED
    m = 6 * (K + 1)
    ws = torch.empty(q.gemm_ws_bytes(F.Q6_K, m, V, HD, fl), dtype=torch.uint8, device="cuda")
    for r0 in range(0, rows, m):
        mm = min(m, rows - r0)
        ih.gemm_q_ex(F.Q6_K, lm, Hs[r0:r0 + mm], V, HD, flags=fl, out=Lt[r0:r0 + mm], ws=ws)
    del Hs, lm, ws
    L3 = Lt.view(STEPS, K + 1, V)
    Ld = torch.empty((STEPS, K, V), device="cuda")
    g = torch.Generator(device="cuda").manual_seed(seed + 4096)
    draft = torch.empty((STEPS, K), dtype=torch.int32, device="cuda")
    for s0 in range(0, STEPS, BATCH):
        blk = L3[s0:s0 + BATCH, :K].contiguous()
        q.synth_gaussian(st(seed, f"acc4096.d{s0}"), blk.numel(), 1.5, add=blk, out=Ld[s0:s0 + BATCH].view(-1))
        p = torch.softmax(Ld[s0:s0 + BATCH].view(-1, V).double() / T, -1)
        draft[s0:s0 + BATCH] = torch.multinomial(p, 1, generator=g).view(-1, K).to(torch.int32)
        del p, blk
    u_acc = torch.rand((STEPS, K), generator=g, device="cuda")
    u_res = torch.rand(STEPS, generator=g, device="cuda")
    u_bon = torch.rand(STEPS, generator=g, device="cuda")
    torch.cuda.synchronize()
    print(f"config 3 accept case: {STEPS} steps of logits generated", flush=True)
    return L3, Ld, draft, u_acc, u_res, u_bon


@pytest.mark.parametrize("mode", [0, 1])
def test_config3_4096_steps(ih, case, mode):
    L3, Ld, draft, u_acc, u_res, u_bon = case
    tok, n = ih.spec_accept(L3, Ld, draft, T, u_acc, u_res, u_bon, mode=mode)
    tok, n = tok.cpu().numpy(), n.cpu().numpy()
    dr, ua, ur, ub = (t.cpu().numpy() for t in (draft, u_acc, u_res, u_bon))
    same_len = same_tok = 0
    lengths = np.zeros(K + 1, dtype=np.int64)
    for s0 in range(0, STEPS, BATCH):
        sl = slice(s0, s0 + BATCH)
        rtok, rn = O.spec_accept_batch(L3[sl].cpu().numpy(), Ld[sl].cpu().numpy(), dr[sl], T, ua[sl], ur[sl],
                                       ub[sl], mode)
        for i in range(rn.shape[0]):
            s = s0 + i
            nt = O.n_tokens(int(rn[i]), K, mode)
            ok_len = int(n[s]) == int(rn[i])
            same_len += ok_len
            same_tok += ok_len and tok[s, :nt].tolist() == rtok[i, :nt].tolist()
        lengths += np.bincount(rn[rn >= 0], minlength=K + 1)
        print(f"mode {mode}: steps {s0 + BATCH}/{STEPS}, lengths agree {same_len}, tokens agree {same_tok}",
              flush=True)
    print(f"config 3 mode {mode}: accepted lengths identical on {same_len}/{STEPS} steps, tokens on "
          f"{same_tok}/{STEPS}; oracle length histogram {lengths.tolist()}", flush=True)
    assert same_len >= 0.999 * STEPS
    assert same_tok >= 0.999 * STEPS
