"""GPU: ihip_gguf_upload. A GGUF file's tensors reach the device byte for
byte (through the pinned staging, including a tensor several staging chunks
long), and a packed upload equals ihip_pack_weights of the same bytes, so a
matmul on it equals the one on weights uploaded any other way."""
import numpy as np
import pytest

from inferno_hip import HipError
from inferno_hip import formats as F
from inferno_hip import gguf as G
from inferno_hip import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ih():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import inferno_hip
    assert inferno_hip.quant_kernels_available(), inferno_hip._lib.last_error()
    return inferno_hip


def test_upload_plain_and_packed(ih, tmp_path):
    import torch
    mats = {"q4": (F.Q4_K, 96, 512), "q5": (F.Q5_K, 40, 768), "q6": (F.Q6_K, 64, 1024), "q8": (F.Q8_0, 33, 256)}
    data = {k: synth.matrix(qt, N, K, synth.stream_for(N + K, k)) for k, (qt, N, K) in mats.items()}
    vec = np.linspace(-1, 1, 100).astype(np.float32)
    tensors = [(k, (K, N), qt, data[k].tobytes()) for k, (qt, N, K) in mats.items()] + [("v", (100,), 0, vec.tobytes())]
    G.write_gguf(str(tmp_path / "m.gguf"), [("general.architecture", G.GGUF_TYPE_STRING, "test")], tensors)
    x = torch.randn(5, 1024, device="cuda")
    with G.read_gguf(str(tmp_path / "m.gguf")) as f:
        for k, (qt, N, K) in mats.items():
            raw = f.upload(k)
            assert torch.equal(raw.cpu(), torch.from_numpy(data[k].reshape(-1)))
            packed = f.upload(k, packed=True)
            ref = ih.pack_weights(qt, torch.from_numpy(data[k].reshape(-1)).cuda(), N, K)
            assert torch.equal(packed, ref), k
            fl = ih.GEMM_F32
            y1 = ih.gemm_q(qt, packed, x[:, :K].contiguous(), N, K, flags=fl | ih.GEMM_PACKED)
            y2 = ih.gemm_q(qt, raw, x[:, :K].contiguous(), N, K, flags=fl)
            assert torch.equal(y1, y2), k
        assert torch.equal(f.upload("v").cpu().view(torch.float32), torch.from_numpy(vec))
        with pytest.raises(HipError):
            f.upload("v", packed=True)  # only quantized matrices pack
        small = torch.empty(16, dtype=torch.uint8, device="cuda")
        with pytest.raises(HipError, match="device bytes"):
            f.upload("q4", out=small)


def test_upload_spans_staging_chunks(ih, tmp_path):
    import torch
    N, K = 16384, 16384  # 151 MB of Q4_K: three 64 MiB staging chunks
    rng = np.random.default_rng(7)
    blob = rng.integers(0, 256, size=N * K // 256 * 144, dtype=np.uint8)
    G.write_gguf(str(tmp_path / "big.gguf"), [], [("w", (K, N), F.Q4_K, blob.tobytes())])
    with G.read_gguf(str(tmp_path / "big.gguf")) as f:
        d = f.upload("w")
        assert d.numel() == blob.size
        # whole-buffer equality in slices (host copies of 151 MB are fine on the box)
        h = d.cpu().numpy()
        assert np.array_equal(h, blob)
