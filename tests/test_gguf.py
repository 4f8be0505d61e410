"""The GGUF loader (ihip_gguf_*, csrc/gguf.cpp; Python inferno_hip.gguf) on
the CPU: the byte-level cases of the reference's own GGUF tests
(tests/unit/test_gguf.jl: strings with the 1 MiB limit, every value type,
arrays, an unknown type, a bad magic), alignment and tensor placement as
src/GGUF.jl:152-165 computes them, tensor sizes as src/LoaderCPU.jl:131-175
takes them, and every truncation of a valid file rejected without a crash.
Files are written byte by byte here (struct), independent of write_gguf,
except where write_gguf itself is under test."""
import struct

import numpy as np
import pytest

from inferno_hip import HipError
from inferno_hip import gguf as G
from inferno_hip import synth
from inferno_hip import formats as F


def _s(x: str | bytes) -> bytes:
    b = x.encode() if isinstance(x, str) else x
    return struct.pack("<Q", len(b)) + b


def _file(tmp_path, kv: list[bytes], tensors: list[bytes] = (), data: bytes = b"", magic=G.GGUF_MAGIC,
          version=3, align=32, name="t.gguf"):
    head = struct.pack("<IIQQ", magic, version, len(tensors), len(kv)) + b"".join(kv) + b"".join(tensors)
    head += b"\0" * ((-len(head)) % align)
    p = tmp_path / name
    p.write_bytes(head + data)
    return str(p)


def _kv(key, vt, payload: bytes) -> bytes:
    return _s(key) + struct.pack("<I", vt) + payload


def test_constants():
    assert G.GGUF_MAGIC == 0x46554747 and struct.pack("<I", G.GGUF_MAGIC) == b"GGUF"
    assert G.GGUF_VERSION == 3
    assert (G.GGUF_TYPE_UINT8, G.GGUF_TYPE_STRING, G.GGUF_TYPE_ARRAY, G.GGUF_TYPE_FLOAT64) == (0, 8, 9, 12)


def test_strings(tmp_path):
    kv = [_kv("a", 8, _s("Hello")), _kv("b", 8, _s("")), _kv("c", 8, _s("Hello 世界!")),
          _kv("d", 8, _s("a" * 1048575)), _kv("e", 8, _s("b" * 1048576))]
    with G.read_gguf(_file(tmp_path, kv)) as f:
        m = f.metadata
        assert m["a"] == "Hello" and m["b"] == "" and m["c"] == "Hello 世界!"
        assert len(m["d"]) == 1048575 and len(m["e"]) == 1048576
    for n in (1048577, 100 * 1048576, 2**64 - 1):  # over the limit: an error, never a read past the end
        bad = _s("k") + struct.pack("<I", 8) + struct.pack("<Q", n)
        with pytest.raises(HipError, match="1MB"):
            G.read_gguf(_file(tmp_path, [bad], name=f"s{n}.gguf"))


def test_value_types(tmp_path):
    vals = [(0, "<B", 42), (1, "<b", -42), (2, "<H", 1000), (3, "<h", -1000), (4, "<I", 100000), (5, "<i", -100000),
            (10, "<Q", 10000000000), (11, "<q", -10000000000), (6, "<f", 3.14159), (12, "<d", 3.14159265358979),
            (7, "<?", True), (7, "<?", False)]
    kv = [_kv(f"v{i}", vt, struct.pack(fmt, v)) for i, (vt, fmt, v) in enumerate(vals)]
    with G.read_gguf(_file(tmp_path, kv)) as f:
        for i, (vt, fmt, v) in enumerate(vals):
            got = f.metadata[f"v{i}"]
            if vt == 6:
                assert abs(got - 3.14159) < 1e-5
            elif vt == 12:
                assert abs(got - 3.14159265358979) < 1e-14
            else:
                assert got == v and type(got) is type(v), (vt, got)


def test_arrays(tmp_path):
    kv = [_kv("ints", 9, struct.pack("<IQ", 5, 3) + struct.pack("<iii", 1, 2, 3)),
          _kv("strs", 9, struct.pack("<IQ", 8, 2) + _s("Hi") + _s("World")),
          _kv("empty", 9, struct.pack("<IQ", 5, 0)),
          _kv("f32", 9, struct.pack("<IQ", 6, 2) + struct.pack("<ff", 0.5, -2.0))]
    with G.read_gguf(_file(tmp_path, kv)) as f:
        assert f.metadata["ints"] == [1, 2, 3]
        assert f.metadata["strs"] == ["Hi", "World"]
        assert f.metadata["empty"] == []
        assert f.metadata["f32"] == [0.5, -2.0]


def test_unknown_type_and_bad_magic(tmp_path):
    with pytest.raises(HipError, match="Unknown GGUF type"):
        G.read_gguf(_file(tmp_path, [_kv("x", 999, b"\0" * 8)]))
    with pytest.raises(HipError, match="Not a valid GGUF file"):
        G.read_gguf(_file(tmp_path, [], magic=0x12345678, name="m.gguf"))
    p = tmp_path / "tiny.gguf"
    p.write_bytes(b"GG")
    with pytest.raises(HipError, match="Not a valid GGUF file"):
        G.read_gguf(str(p))


def _tensor_info(name, dims, ty, off):
    return _s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) + \
        struct.pack("<IQ", ty, off)


@pytest.mark.parametrize("align", [32, 64])
def test_tensor_table_and_alignment(tmp_path, align):
    K, N = 512, 48
    q4 = synth.matrix(F.Q4_K, N, K, 11).tobytes()
    q6 = synth.matrix(F.Q6_K, N, K, 12).tobytes()
    f32 = np.arange(10, dtype=np.float32).tobytes()
    kv = [_kv("general.architecture", 8, _s("qwen35"))]
    if align != 32:
        kv.append(_kv("general.alignment", 4, struct.pack("<I", align)))
    o1 = 0
    o2 = (len(q4) + align - 1) // align * align
    o3 = (o2 + len(q6) + align - 1) // align * align
    tens = [_tensor_info("blk.0.ffn_up.weight", (K, N), 12, o1), _tensor_info("blk.0.ffn_down.weight", (K, N), 14, o2),
            _tensor_info("token_embd_norm", (10,), 0, o3)]
    data = bytearray(o3 + len(f32))
    data[o1:o1 + len(q4)] = q4
    data[o2:o2 + len(q6)] = q6
    data[o3:] = f32
    path = _file(tmp_path, kv, tens, bytes(data), align=align)
    with G.read_gguf(path) as f:
        assert f.version == 3 and f.alignment == align and f.data_offset % align == 0
        assert f.metadata["general.architecture"] == "qwen35"
        t = f.tensors["blk.0.ffn_up.weight"]
        assert t.dimensions == (K, N) and t.type == 12 and t.nbytes == N * K // 256 * 144
        assert f.tensors["blk.0.ffn_down.weight"].nbytes == N * K // 256 * 210
        assert f.tensors["token_embd_norm"].nbytes == 40
        assert f.tensor_bytes("blk.0.ffn_up.weight").tobytes() == q4
        assert f.tensor_bytes("blk.0.ffn_down.weight").tobytes() == q6
        np.testing.assert_array_equal(f.tensor_bytes("token_embd_norm").view(np.float32), np.arange(10))
        with pytest.raises(KeyError, match="Tensor not found"):
            f.index("missing")


def test_write_gguf_round_trip(tmp_path):
    K, N = 256, 32
    q8 = synth.matrix(F.Q8_0, N, K, 5).tobytes()
    meta = [("general.architecture", G.GGUF_TYPE_STRING, "qwen35"), ("general.alignment", G.GGUF_TYPE_UINT32, 128),
            ("qwen35.block_count", G.GGUF_TYPE_UINT32, 2),
            ("tokenizer.ggml.tokens", G.GGUF_TYPE_ARRAY, (G.GGUF_TYPE_STRING, ["<s>", "a", "ü"])),
            ("rope.freq", G.GGUF_TYPE_FLOAT32, 1.5e6)]
    G.write_gguf(str(tmp_path / "w.gguf"), meta, [("a.weight", (K, N), 8, q8), ("b", (7,), 0, b"\1" * 28)])
    with G.read_gguf(str(tmp_path / "w.gguf")) as f:
        assert f.alignment == 128 and f.data_offset % 128 == 0
        assert f.metadata["tokenizer.ggml.tokens"] == ["<s>", "a", "ü"] and f.metadata["qwen35.block_count"] == 2
        assert f.tensors["a.weight"].offset == 0 and f.tensors["b"].offset % 128 == 0
        assert f.tensor_bytes("a.weight").tobytes() == q8 and f.tensor_bytes("b").tobytes() == b"\1" * 28


def test_truncations_and_bad_tables_are_errors(tmp_path):
    K, N = 256, 16
    q4 = synth.matrix(F.Q4_K, N, K, 3).tobytes()
    G.write_gguf(str(tmp_path / "ok.gguf"), [("k", G.GGUF_TYPE_ARRAY, (G.GGUF_TYPE_STRING, ["x", "yz"]))],
                 [("w", (K, N), 12, q4)])
    full = (tmp_path / "ok.gguf").read_bytes()
    for n in list(range(0, 200)) + [len(full) - 1]:
        p = tmp_path / f"cut{n}.gguf"
        p.write_bytes(full[:n])
        with pytest.raises(HipError):
            G.read_gguf(str(p))
    # data past the end, non-whole blocks, a zero dimension, 5 dimensions
    for dims, ty, off in (((K, N), 12, 64), ((100, 2), 12, 0), ((0, 4), 0, 0), ((1, 1, 1, 1, 1), 0, 0)):
        path = _file(tmp_path, [], [_tensor_info("w", dims, ty, off)], q4, name=f"bad{len(dims)}{ty}{off}.gguf")
        with pytest.raises(HipError):
            G.read_gguf(path)
    # an unknown GGML type parses (size unknown) but has no bytes to hand out
    path = _file(tmp_path, [], [_tensor_info("iq", (256,), 23, 0)], b"\0" * 256, name="iq.gguf")
    with G.read_gguf(path) as f:
        assert f.tensors["iq"].nbytes == 0
        with pytest.raises(ValueError):
            f.tensor_bytes("iq")
