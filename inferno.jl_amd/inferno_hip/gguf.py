"""Host mirror of the reference's GGUF reader (src/GGUF.jl:119-186) and of
keep_quantized tensor extraction (src/LoaderCPU.jl:120-175) over the
library's loader (ihip_gguf_*): the file is memory-mapped and parsed in C++,
tensors come back as host byte views or are uploaded to the GPU, optionally
straight into the packed matmul layout."""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib

GGUF_MAGIC = 0x46554747
GGUF_VERSION = 3
# value types (src/GGUF.jl:8-22)
(GGUF_TYPE_UINT8, GGUF_TYPE_INT8, GGUF_TYPE_UINT16, GGUF_TYPE_INT16, GGUF_TYPE_UINT32, GGUF_TYPE_INT32,
 GGUF_TYPE_FLOAT32, GGUF_TYPE_BOOL, GGUF_TYPE_STRING, GGUF_TYPE_ARRAY, GGUF_TYPE_UINT64, GGUF_TYPE_INT64,
 GGUF_TYPE_FLOAT64) = range(13)
_FLOAT_TYPES = (GGUF_TYPE_FLOAT32, GGUF_TYPE_FLOAT64)


@dataclass(frozen=True)
class TensorInfo:
    """TensorInfo (src/GGUF.jl:62-67); dims innermost first; nbytes 0 when the
    GGML type's layout is unknown to the library."""
    name: str
    dimensions: tuple
    type: int
    offset: int
    nbytes: int


class GGUFFile:
    """read_gguf: metadata dict, tensors dict, data_offset; tensor_bytes()
    is a zero-copy view into the mapping, upload() copies to the GPU."""

    def __init__(self, path: str):
        L = _lib.load()
        h = C.c_void_p()
        _lib.check(L.ihip_gguf_open(str(path).encode(), C.byref(h)))
        self._h, self._L, self.path = h, L, str(path)
        ver, nt, nkv, al, do = C.c_uint32(), C.c_int64(), C.c_int64(), C.c_uint64(), C.c_uint64()
        _lib.check(L.ihip_gguf_info(h, C.byref(ver), C.byref(nt), C.byref(nkv), C.byref(al), C.byref(do)))
        self.version, self.alignment, self.data_offset = ver.value, al.value, do.value
        self.metadata = {}
        for i in range(nkv.value):
            self.metadata.update([self._kv(i)])
        self.tensors = {}
        for i in range(nt.value):
            name, ty, nd = C.c_char_p(), C.c_int(), C.c_int()
            dims, off, nb = (C.c_int64 * 4)(), C.c_uint64(), C.c_uint64()
            _lib.check(L.ihip_gguf_tensor(h, i, C.byref(name), C.byref(ty), C.byref(nd), dims, C.byref(off),
                                          C.byref(nb)))
            nm = name.value.decode("utf-8", errors="replace")
            self.tensors[nm] = TensorInfo(nm, tuple(dims[: nd.value]), ty.value, off.value, nb.value)

    def _str(self, i, j=0):
        p, n = C.c_void_p(), C.c_uint64()
        _lib.check(self._L.ihip_gguf_kv_string(self._h, i, j, C.byref(p), C.byref(n)))
        return C.string_at(p.value, n.value).decode("utf-8", errors="replace") if n.value else ""

    def _num(self, i, j, vtype):
        iv, fv = C.c_int64(), C.c_double()
        _lib.check(self._L.ihip_gguf_kv_number(self._h, i, j, C.byref(iv), C.byref(fv)))
        if vtype in _FLOAT_TYPES:
            return float(fv.value)
        if vtype == GGUF_TYPE_BOOL:
            return bool(iv.value)
        if vtype == GGUF_TYPE_UINT64:
            return iv.value % (1 << 64)
        return int(iv.value)

    def _kv(self, i):
        key, vt, at, cnt = C.c_char_p(), C.c_int(), C.c_int(), C.c_uint64()
        _lib.check(self._L.ihip_gguf_kv(self._h, i, C.byref(key), C.byref(vt), C.byref(at), C.byref(cnt)))
        k = key.value.decode("utf-8", errors="replace")
        if vt.value == GGUF_TYPE_STRING:
            return k, self._str(i)
        if vt.value == GGUF_TYPE_ARRAY:
            if at.value == GGUF_TYPE_STRING:
                return k, [self._str(i, j) for j in range(cnt.value)]
            return k, [self._num(i, j, at.value) for j in range(cnt.value)]
        return k, self._num(i, 0, vt.value)

    def index(self, name: str) -> int:
        i = self._L.ihip_gguf_find_tensor(self._h, name.encode())
        if i < 0:
            raise KeyError(f"Tensor not found: {name}")
        return i

    def tensor_bytes(self, name: str) -> np.ndarray:
        """The tensor's bytes in the file (read-only view; keep the file open)."""
        info = self.tensors[name]
        if info.nbytes == 0:
            raise ValueError(f"{name}: GGML type {info.type} has no known layout")
        p = self._L.ihip_gguf_tensor_data(self._h, self.index(name))
        return np.ctypeslib.as_array((C.c_uint8 * info.nbytes).from_address(p))

    def upload(self, name: str, packed: bool = False, out=None, stream=None):
        """The tensor on the GPU as a uint8 tensor: GGUF bytes, or (packed) the
        layout of pack_weights for a 2-D Q4_K/Q5_K/Q6_K/Q8_0 matrix."""
        import torch
        from .quantized_kernels import _stream, packed_bytes
        info = self.tensors[name]
        if packed:
            if len(info.dimensions) > 2:
                raise ValueError(f"{name}: only 2-D matrices pack")
            K = info.dimensions[0]
            N = info.dimensions[1] if len(info.dimensions) > 1 else 1
            nb = packed_bytes(info.type, N, K)
        else:
            nb = info.nbytes
        if out is None:
            out = torch.empty(max(nb, 1), dtype=torch.uint8, device="cuda")
        _lib.check(self._L.ihip_gguf_upload(self._h, self.index(name), out.data_ptr(), out.numel(),
                                            1 if packed else 0, _stream(stream)))
        return out

    def close(self):
        if self._h:
            self._L.ihip_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def read_gguf(path: str) -> GGUFFile:
    """src/GGUF.jl:119 read_gguf."""
    return GGUFFile(path)


_SCALAR_FMT = {GGUF_TYPE_UINT8: "<B", GGUF_TYPE_INT8: "<b", GGUF_TYPE_UINT16: "<H", GGUF_TYPE_INT16: "<h",
               GGUF_TYPE_UINT32: "<I", GGUF_TYPE_INT32: "<i", GGUF_TYPE_FLOAT32: "<f", GGUF_TYPE_BOOL: "<?",
               GGUF_TYPE_UINT64: "<Q", GGUF_TYPE_INT64: "<q", GGUF_TYPE_FLOAT64: "<d"}


def _pack_value(vtype: int, value, atype: int | None = None) -> bytes:
    import struct
    if vtype == GGUF_TYPE_STRING:
        b = value.encode("utf-8") if isinstance(value, str) else bytes(value)
        return struct.pack("<Q", len(b)) + b
    if vtype == GGUF_TYPE_ARRAY:
        return struct.pack("<IQ", atype, len(value)) + b"".join(_pack_value(atype, v) for v in value)
    return struct.pack(_SCALAR_FMT[vtype], value)


def write_gguf(path: str, metadata, tensors, version: int = GGUF_VERSION) -> None:
    """Writes a GGUF file in the layout read_gguf reads (src/GGUF.jl:119-165):
    metadata = [(key, vtype, value) or (key, GGUF_TYPE_ARRAY, (atype, values))],
    tensors = [(name, dims innermost first, ggml_type, bytes)]. Tensor data
    is laid out in order, each at a multiple of the alignment
    (general.alignment if given, else 32)."""
    import struct
    align = 32
    for k, vt, v in metadata:
        if k == "general.alignment" and vt != GGUF_TYPE_ARRAY:
            align = int(v)
    head = [struct.pack("<IIQQ", GGUF_MAGIC, version, len(tensors), len(metadata))]
    for k, vt, v in metadata:
        head.append(_pack_value(GGUF_TYPE_STRING, k) + struct.pack("<I", vt))
        head.append(_pack_value(vt, v[1], v[0]) if vt == GGUF_TYPE_ARRAY else _pack_value(vt, v))
    off, blobs = 0, []
    for name, dims, ty, data in tensors:
        off = (off + align - 1) // align * align
        head.append(_pack_value(GGUF_TYPE_STRING, name) + struct.pack("<I", len(dims)) +
                    b"".join(struct.pack("<Q", int(d)) for d in dims) + struct.pack("<IQ", ty, off))
        blobs.append((off, bytes(data)))
        off += len(data)
    h = b"".join(head)
    pad = (-len(h)) % align
    with open(path, "wb") as f:
        f.write(h + b"\0" * pad)
        base = f.tell()
        for o, b in blobs:
            f.seek(base + o)
            f.write(b)
