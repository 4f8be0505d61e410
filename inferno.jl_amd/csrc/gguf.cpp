// GGUF file -> device weights (host side of libinferno_hip).
//
// The file format as src/GGUF.jl:119-165 reads it: magic "GGUF" (u32
// 0x46554747), version (u32; 3 expected, others accepted), tensor count and
// metadata count (u64 each), the metadata key/value pairs (key string =
// u64 length + bytes, at most 1 MiB; u32 value type; the value: scalars
// little-endian, strings as keys, arrays as u32 element type + u64 count +
// elements), the tensor infos (name string, u32 ndim, ndim u64 dims with the
// innermost first, u32 GGML type, u64 offset into the data section), zero
// padding to general.alignment (default 32), then the data section. Tensor
// bytes per type as src/LoaderCPU.jl:131-175 takes them (blocks of 256 for
// the K-quants, 32 for Q8_0, elements for the float types).
//
// The file is memory-mapped read-only; every read is bounds-checked, and a
// malformed file is an error (IHIP_EINVAL with the reason), never a crash.
// ihip_gguf_upload copies one tensor to device memory through two pinned
// staging buffers (hipHostMalloc, copies overlapped with the next chunk's
// memcpy out of the mapping), optionally repacking a quantized matrix into
// the matmul's packed layout on the device.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/inferno_hip.h"

extern "C" int ihip_internal_fail(int code, const char *fmt, ...);  // (status reporting, capi.cpp)
extern "C" int ihip_internal_ok();
size_t packed_bytes(int qt, int N, int K);
hipError_t launch_pack(int qt, const void *W, void *P, int N, int K, hipStream_t st, int gated);

namespace {

constexpr uint32_t GGUF_MAGIC = 0x46554747u;
constexpr uint64_t MAX_STRING = 1048576;  // src/GGUF.jl:83-85

enum VType : uint32_t {
    VT_U8 = 0, VT_I8 = 1, VT_U16 = 2, VT_I16 = 3, VT_U32 = 4, VT_I32 = 5, VT_F32 = 6, VT_BOOL = 7,
    VT_STRING = 8, VT_ARRAY = 9, VT_U64 = 10, VT_I64 = 11, VT_F64 = 12
};

int scalar_size(uint32_t t) {
    switch (t) {
    case VT_U8: case VT_I8: case VT_BOOL: return 1;
    case VT_U16: case VT_I16: return 2;
    case VT_U32: case VT_I32: case VT_F32: return 4;
    case VT_U64: case VT_I64: case VT_F64: return 8;
    }
    return 0;
}

// (block elements, block bytes) of the GGML types whose layout is known
// here; 0 elements: unknown (the tensor's size is not derived)
void ggml_block(int type, int &elems, int &bytes) {
    elems = 0;
    bytes = 0;
    switch (type) {
    case 0: elems = 1; bytes = 4; break;     // F32
    case 1: elems = 1; bytes = 2; break;     // F16
    case 30: elems = 1; bytes = 2; break;    // BF16
    case 8: elems = 32; bytes = 34; break;   // Q8_0
    case 12: elems = 256; bytes = 144; break;  // Q4_K
    case 13: elems = 256; bytes = 176; break;  // Q5_K
    case 14: elems = 256; bytes = 210; break;  // Q6_K
    case 24: elems = 1; bytes = 1; break;    // I8
    case 25: elems = 1; bytes = 2; break;    // I16
    case 26: elems = 1; bytes = 4; break;    // I32
    case 27: elems = 1; bytes = 8; break;    // I64
    case 28: elems = 1; bytes = 8; break;    // F64
    }
}

struct Value {  // one metadata value (arrays: elements in the mapping)
    uint32_t type = 0, atype = 0;
    uint64_t count = 1;          // array elements (1 for scalars)
    const uint8_t *data = nullptr;  // scalar bytes, string bytes, or the first array element
    uint64_t len = 0;            // string length
    std::vector<const uint8_t *> elem;  // string arrays: each element's length field
};

struct Tensor {
    std::string name;
    int type = 0, ndim = 0;
    int64_t dims[4] = {1, 1, 1, 1};
    uint64_t offset = 0, nbytes = 0;
};

constexpr size_t STAGE = (size_t)64 << 20;  // bytes per pinned staging buffer

struct File {
    int fd = -1;
    uint8_t *base = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32, data_offset = 0;
    std::vector<std::string> keys;
    std::vector<Value> values;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, int64_t> by_name, by_key;
    // pinned staging for uploads, allocated by the first one and kept until close
    void *pin[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    ~File() {
        for (int b = 0; b < 2; b++) {
            if (done[b]) (void)hipEventDestroy(done[b]);
            if (pin[b]) (void)hipHostFree(pin[b]);
        }
        if (base) munmap(base, size);
        if (fd >= 0) close(fd);
    }
};

// memcpy of n bytes split over up to 8 host threads (one chunk of staging)
void copy_parallel(void *dst, const void *src, size_t n) {
    const unsigned hw = std::thread::hardware_concurrency();
    const int T = (int)std::max(1u, std::min(8u, hw ? hw : 1u));
    if (n < ((size_t)4 << 20) || T == 1) {
        memcpy(dst, src, n);
        return;
    }
    std::vector<std::thread> th;
    const size_t per = (n / T + 4095) & ~(size_t)4095;
    for (int k = 0; k < T; k++) {
        const size_t o = (size_t)k * per;
        if (o >= n) break;
        const size_t m = std::min(per, n - o);
        th.emplace_back([=] { memcpy((uint8_t *)dst + o, (const uint8_t *)src + o, m); });
    }
    for (auto &t : th) t.join();
}

struct Reader {
    const uint8_t *p, *end;
    std::string err;
    bool need(uint64_t n) {
        if ((uint64_t)(end - p) < n) {
            if (err.empty()) err = "truncated file";
            return false;
        }
        return true;
    }
    template <class T> bool get(T &v) {
        if (!need(sizeof(T))) return false;
        memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return true;
    }
    bool str(const uint8_t *&s, uint64_t &len) {
        if (!get(len)) return false;
        if (len > MAX_STRING) {
            err = "string length exceeds maximum allowed length of 1MB";
            return false;
        }
        if (!need(len)) return false;
        s = p;
        p += len;
        return true;
    }
    bool skip_value(uint32_t t, Value *out, int depth) {
        if (t == VT_STRING) {
            const uint8_t *s;
            uint64_t len;
            if (!str(s, len)) return false;
            if (out) {
                out->data = s;
                out->len = len;
            }
            return true;
        }
        if (t == VT_ARRAY) {
            if (depth > 0) {
                err = "nested array";
                return false;
            }
            uint32_t at;
            uint64_t n;
            if (!get(at) || !get(n)) return false;
            if (at != VT_STRING && scalar_size(at) == 0) {
                err = "unknown GGUF array element type " + std::to_string(at);
                return false;
            }
            if (out) {
                out->atype = at;
                out->count = n;
                out->data = p;
            }
            if (at == VT_STRING) {
                if (n > (uint64_t)(end - p) / 8) {
                    err = "truncated file";
                    return false;
                }
                if (out) out->elem.reserve(n);
                for (uint64_t i = 0; i < n; i++) {
                    if (out) out->elem.push_back(p);
                    const uint8_t *s;
                    uint64_t len;
                    if (!str(s, len)) return false;
                }
                return true;
            }
            const uint64_t sz = (uint64_t)scalar_size(at);
            if (n > (uint64_t)(end - p) / sz) {
                err = "truncated file";
                return false;
            }
            p += n * sz;
            return true;
        }
        const int sz = scalar_size(t);
        if (sz == 0) {
            err = "Unknown GGUF type: " + std::to_string(t);
            return false;
        }
        if (!need(sz)) return false;
        if (out) out->data = p;
        p += sz;
        return true;
    }
};

int parse(File &f, std::string &err) {
    Reader r{f.base, f.base + f.size, {}};
    uint32_t magic;
    uint64_t nt, nkv;
    if (!r.get(magic) || magic != GGUF_MAGIC) {
        err = "Not a valid GGUF file";
        return IHIP_EINVAL;
    }
    if (!r.get(f.version) || !r.get(nt) || !r.get(nkv)) {
        err = r.err;
        return IHIP_EINVAL;
    }
    if (nkv > f.size || nt > f.size) {
        err = "counts exceed the file size";
        return IHIP_EINVAL;
    }
    for (uint64_t i = 0; i < nkv; i++) {
        const uint8_t *k;
        uint64_t klen;
        uint32_t t;
        Value v;
        if (!r.str(k, klen) || !r.get(t)) {
            err = r.err;
            return IHIP_EINVAL;
        }
        v.type = t;
        if (!r.skip_value(t, &v, 0)) {
            err = r.err;
            return IHIP_EINVAL;
        }
        std::string key((const char *)k, klen);
        f.by_key[key] = (int64_t)f.keys.size();  // (a repeated key: the last one, as a Dict keeps it)
        f.keys.push_back(std::move(key));
        f.values.push_back(std::move(v));
    }
    for (uint64_t i = 0; i < nt; i++) {
        Tensor T;
        const uint8_t *s;
        uint64_t len;
        uint32_t nd, ty;
        if (!r.str(s, len) || !r.get(nd)) {
            err = r.err;
            return IHIP_EINVAL;
        }
        T.name.assign((const char *)s, len);
        if (nd < 1 || nd > 4) {
            err = "tensor " + T.name + ": ndim " + std::to_string(nd) + " outside 1..4";
            return IHIP_EINVAL;
        }
        T.ndim = (int)nd;
        uint64_t n_el = 1;
        for (uint32_t d = 0; d < nd; d++) {
            uint64_t v;
            if (!r.get(v)) {
                err = r.err;
                return IHIP_EINVAL;
            }
            if (v == 0 || v > (1ull << 40) || n_el > (1ull << 50) / v) {
                err = "tensor " + T.name + ": bad dimension";
                return IHIP_EINVAL;
            }
            T.dims[d] = (int64_t)v;
            n_el *= v;
        }
        if (!r.get(ty) || !r.get(T.offset)) {
            err = r.err;
            return IHIP_EINVAL;
        }
        T.type = (int)ty;
        int be, bb;
        ggml_block(T.type, be, bb);
        if (be > 0) {
            if (n_el % (uint64_t)be) {
                err = "tensor " + T.name + ": " + std::to_string(n_el) + " elements, not whole blocks";
                return IHIP_EINVAL;
            }
            T.nbytes = n_el / be * bb;
        }
        f.by_name[T.name] = (int64_t)f.tensors.size();
        f.tensors.push_back(std::move(T));
    }
    // alignment (src/GGUF.jl:152-156): general.alignment when it is an integer
    auto it = f.by_key.find("general.alignment");
    if (it != f.by_key.end()) {
        const Value &v = f.values[it->second];
        uint64_t a = 0;
        if (v.type == VT_U32 || v.type == VT_I32) {
            uint32_t x;
            memcpy(&x, v.data, 4);
            a = x;
        } else if (v.type == VT_U64 || v.type == VT_I64) {
            memcpy(&a, v.data, 8);
        } else if (v.type == VT_U16 || v.type == VT_I16) {
            uint16_t x;
            memcpy(&x, v.data, 2);
            a = x;
        } else if (v.type == VT_U8 || v.type == VT_I8) {
            a = v.data[0];
        }
        if (a == 0 || a > (1u << 20)) {
            err = "general.alignment " + std::to_string(a) + " unusable";
            return IHIP_EINVAL;
        }
        f.alignment = a;
    }
    const uint64_t pos = (uint64_t)(r.p - f.base);
    const uint64_t pad = f.alignment - pos % f.alignment;
    f.data_offset = pos + (pad != f.alignment ? pad : 0);
    if (f.data_offset > f.size) {
        err = "truncated file (data section)";
        return IHIP_EINVAL;
    }
    for (const Tensor &T : f.tensors) {
        if (T.nbytes && (T.offset > f.size - f.data_offset || T.nbytes > f.size - f.data_offset - T.offset)) {
            err = "tensor " + T.name + ": data past the end of the file";
            return IHIP_EINVAL;
        }
    }
    return IHIP_OK;
}

File *as_file(void *h) { return static_cast<File *>(h); }

int check_tensor(File *f, int64_t i, const char *what) {
    if (!f) return ihip_internal_fail(IHIP_EFAULT, "%s: NULL handle", what);
    if (i < 0 || i >= (int64_t)f->tensors.size())
        return ihip_internal_fail(IHIP_EINVAL, "%s: tensor index %lld of %zu", what, (long long)i, f->tensors.size());
    return IHIP_OK;
}

int check_kv(File *f, int64_t i, const char *what) {
    if (!f) return ihip_internal_fail(IHIP_EFAULT, "%s: NULL handle", what);
    if (i < 0 || i >= (int64_t)f->keys.size())
        return ihip_internal_fail(IHIP_EINVAL, "%s: key index %lld of %zu", what, (long long)i, f->keys.size());
    return IHIP_OK;
}

}  // namespace

int ihip_gguf_open(const char *path, void **handle) {
    if (!path || !handle) return ihip_internal_fail(IHIP_EFAULT, "ihip_gguf_open: NULL pointer");
    *handle = nullptr;
    File *f = new File();
    f->fd = open(path, O_RDONLY);
    if (f->fd < 0) {
        delete f;
        return ihip_internal_fail(IHIP_EINVAL, "ihip_gguf_open: cannot open %s", path);
    }
    struct stat st;
    if (fstat(f->fd, &st) != 0 || st.st_size < 4) {
        delete f;
        return ihip_internal_fail(IHIP_EINVAL, "ihip_gguf_open: %s: Not a valid GGUF file", path);
    }
    f->size = (size_t)st.st_size;
    void *m = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
    if (m == MAP_FAILED) {
        delete f;
        return ihip_internal_fail(IHIP_ENOMEM, "ihip_gguf_open: mmap of %s failed", path);
    }
    f->base = (uint8_t *)m;
    std::string err;
    const int rc = parse(*f, err);
    if (rc != IHIP_OK) {
        delete f;
        return ihip_internal_fail(rc, "ihip_gguf_open: %s: %s", path, err.c_str());
    }
    *handle = f;
    return ihip_internal_ok();
}

int ihip_gguf_close(void *handle) {
    delete as_file(handle);
    return ihip_internal_ok();
}

int ihip_gguf_info(void *handle, uint32_t *version, int64_t *n_tensors, int64_t *n_kv, uint64_t *alignment,
                   uint64_t *data_offset) {
    File *f = as_file(handle);
    if (!f) return ihip_internal_fail(IHIP_EFAULT, "ihip_gguf_info: NULL handle");
    if (version) *version = f->version;
    if (n_tensors) *n_tensors = (int64_t)f->tensors.size();
    if (n_kv) *n_kv = (int64_t)f->keys.size();
    if (alignment) *alignment = f->alignment;
    if (data_offset) *data_offset = f->data_offset;
    return ihip_internal_ok();
}

int ihip_gguf_tensor(void *handle, int64_t i, const char **name, int *ggml_type, int *ndim, int64_t *dims,
                     uint64_t *offset, uint64_t *nbytes) {
    File *f = as_file(handle);
    const int rc = check_tensor(f, i, "ihip_gguf_tensor");
    if (rc != IHIP_OK) return rc;
    const Tensor &T = f->tensors[i];
    if (name) *name = T.name.c_str();
    if (ggml_type) *ggml_type = T.type;
    if (ndim) *ndim = T.ndim;
    if (dims)
        for (int d = 0; d < 4; d++) dims[d] = T.dims[d];
    if (offset) *offset = T.offset;
    if (nbytes) *nbytes = T.nbytes;
    return ihip_internal_ok();
}

int64_t ihip_gguf_find_tensor(void *handle, const char *name) {
    File *f = as_file(handle);
    if (!f || !name) return -1;
    auto it = f->by_name.find(name);
    return it == f->by_name.end() ? -1 : it->second;
}

int64_t ihip_gguf_find_key(void *handle, const char *key) {
    File *f = as_file(handle);
    if (!f || !key) return -1;
    auto it = f->by_key.find(key);
    return it == f->by_key.end() ? -1 : it->second;
}

int ihip_gguf_kv(void *handle, int64_t i, const char **key, int *vtype, int *atype, uint64_t *count) {
    File *f = as_file(handle);
    const int rc = check_kv(f, i, "ihip_gguf_kv");
    if (rc != IHIP_OK) return rc;
    const Value &v = f->values[i];
    if (key) *key = f->keys[i].c_str();
    if (vtype) *vtype = (int)v.type;
    if (atype) *atype = v.type == VT_ARRAY ? (int)v.atype : -1;
    if (count) *count = v.count;
    return ihip_internal_ok();
}

int ihip_gguf_kv_number(void *handle, int64_t i, uint64_t index, int64_t *as_int, double *as_float) {
    File *f = as_file(handle);
    const int rc = check_kv(f, i, "ihip_gguf_kv_number");
    if (rc != IHIP_OK) return rc;
    const Value &v = f->values[i];
    const uint32_t t = v.type == VT_ARRAY ? v.atype : v.type;
    if (t == VT_STRING || scalar_size(t) == 0)
        return ihip_internal_fail(IHIP_EINVAL, "ihip_gguf_kv_number: %s is not numeric", f->keys[i].c_str());
    if (index >= v.count)
        return ihip_internal_fail(IHIP_EINVAL, "ihip_gguf_kv_number: %s: element %llu of %llu", f->keys[i].c_str(),
                                  (unsigned long long)index, (unsigned long long)v.count);
    const uint8_t *p = v.data + index * (uint64_t)scalar_size(t);
    int64_t iv = 0;
    double fv = 0.0;
    switch (t) {
    case VT_U8: iv = p[0]; break;
    case VT_BOOL: iv = p[0] != 0; break;
    case VT_I8: iv = (int8_t)p[0]; break;
    case VT_U16: { uint16_t x; memcpy(&x, p, 2); iv = x; break; }
    case VT_I16: { int16_t x; memcpy(&x, p, 2); iv = x; break; }
    case VT_U32: { uint32_t x; memcpy(&x, p, 4); iv = x; break; }
    case VT_I32: { int32_t x; memcpy(&x, p, 4); iv = x; break; }
    case VT_U64: { uint64_t x; memcpy(&x, p, 8); iv = (int64_t)x; break; }
    case VT_I64: { int64_t x; memcpy(&x, p, 8); iv = x; break; }
    case VT_F32: { float x; memcpy(&x, p, 4); fv = x; break; }
    case VT_F64: { double x; memcpy(&x, p, 8); fv = x; break; }
    }
    if (t != VT_F32 && t != VT_F64) fv = (double)iv;
    else iv = (int64_t)fv;
    if (as_int) *as_int = iv;
    if (as_float) *as_float = fv;
    return ihip_internal_ok();
}

int ihip_gguf_kv_string(void *handle, int64_t i, uint64_t index, const char **str, uint64_t *len) {
    File *f = as_file(handle);
    const int rc = check_kv(f, i, "ihip_gguf_kv_string");
    if (rc != IHIP_OK) return rc;
    const Value &v = f->values[i];
    if (v.type == VT_STRING) {
        if (index != 0) return ihip_internal_fail(IHIP_EINVAL, "ihip_gguf_kv_string: element %llu of a string",
                                                  (unsigned long long)index);
        if (str) *str = (const char *)v.data;
        if (len) *len = v.len;
        return ihip_internal_ok();
    }
    if (v.type != VT_ARRAY || v.atype != VT_STRING)
        return ihip_internal_fail(IHIP_EINVAL, "ihip_gguf_kv_string: %s is not a string", f->keys[i].c_str());
    if (index >= v.count)
        return ihip_internal_fail(IHIP_EINVAL, "ihip_gguf_kv_string: %s: element %llu of %llu", f->keys[i].c_str(),
                                  (unsigned long long)index, (unsigned long long)v.count);
    const uint8_t *e = v.elem[index];
    uint64_t l;
    memcpy(&l, e, 8);
    if (str) *str = (const char *)(e + 8);
    if (len) *len = l;
    return ihip_internal_ok();
}

const void *ihip_gguf_tensor_data(void *handle, int64_t i) {
    File *f = as_file(handle);
    if (!f || i < 0 || i >= (int64_t)f->tensors.size()) return nullptr;
    return f->base + f->data_offset + f->tensors[i].offset;
}

int ihip_gguf_upload(void *handle, int64_t i, void *dev, size_t dev_bytes, int flags, void *stream) {
    File *f = as_file(handle);
    int rc = check_tensor(f, i, "ihip_gguf_upload");
    if (rc != IHIP_OK) return rc;
    if (!dev) return ihip_internal_fail(IHIP_EFAULT, "ihip_gguf_upload: NULL device pointer");
    if (flags & ~IHIP_GGUF_PACKED) return ihip_internal_fail(IHIP_EINVAL, "ihip_gguf_upload: flags 0x%x", flags);
    const Tensor &T = f->tensors[i];
    if (T.nbytes == 0)
        return ihip_internal_fail(IHIP_EINVAL, "ihip_gguf_upload: %s: GGML type %d has no known layout here",
                                  T.name.c_str(), T.type);
    const bool pack = flags & IHIP_GGUF_PACKED;
    const int qt = T.type;
    const bool quant = qt == IHIP_Q4_K || qt == IHIP_Q5_K || qt == IHIP_Q6_K || qt == IHIP_Q8_0;
    const int64_t K = T.dims[0], N = T.ndim >= 2 ? T.dims[1] : 1;
    if (pack && (!quant || T.ndim > 2 || K > INT32_MAX || N > INT32_MAX))
        return ihip_internal_fail(IHIP_EINVAL, "ihip_gguf_upload: %s: only 2-D Q4_K/Q5_K/Q6_K/Q8_0 matrices pack",
                                  T.name.c_str());
    const size_t need = pack ? packed_bytes(qt, (int)N, (int)K) : (size_t)T.nbytes;
    if (dev_bytes < need)
        return ihip_internal_fail(IHIP_ENOMEM, "ihip_gguf_upload: %s needs %zu device bytes, %zu given",
                                  T.name.c_str(), need, dev_bytes);
    hipStream_t st = (hipStream_t)stream;
    // staging: the GGUF bytes land in dev itself, or in a temporary buffer
    // that the pack kernel reads
    uint8_t *dst = (uint8_t *)dev;
    void *tmp = nullptr;
    hipError_t e = hipSuccess;
    if (pack) {
        e = hipMalloc(&tmp, T.nbytes);
        if (e != hipSuccess)
            return ihip_internal_fail(IHIP_ENOMEM, "ihip_gguf_upload: %s: %s", T.name.c_str(), hipGetErrorString(e));
        dst = (uint8_t *)tmp;
    }
    const uint8_t *src = f->base + f->data_offset + T.offset;
    for (int b = 0; b < 2 && e == hipSuccess; b++) {
        if (!f->pin[b]) e = hipHostMalloc(&f->pin[b], STAGE, hipHostMallocDefault);
        if (e == hipSuccess && !f->done[b]) e = hipEventCreateWithFlags(&f->done[b], hipEventDisableTiming);
        // (a buffer may still feed the previous upload's copy on another stream)
        if (e == hipSuccess) e = hipEventSynchronize(f->done[b]);
    }
    for (size_t o = 0, k = 0; e == hipSuccess && o < T.nbytes; o += STAGE, k++) {
        const int b = (int)(k & 1);
        const size_t n = T.nbytes - o < STAGE ? T.nbytes - o : STAGE;
        if (k >= 2) e = hipEventSynchronize(f->done[b]);  // the copy that last used this buffer
        if (e != hipSuccess) break;
        copy_parallel(f->pin[b], src + o, n);
        e = hipMemcpyAsync(dst + o, f->pin[b], n, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipEventRecord(f->done[b], st);
    }
    if (e == hipSuccess && pack) e = launch_pack(qt, tmp, dev, (int)N, (int)K, st, 0);
    const hipError_t es = hipStreamSynchronize(st);  // tmp is released below
    if (e == hipSuccess) e = es;
    if (tmp) (void)hipFree(tmp);
    if (e != hipSuccess)
        return ihip_internal_fail(IHIP_EHIP, "ihip_gguf_upload: %s: %s", T.name.c_str(), hipGetErrorString(e));
    return ihip_internal_ok();
}
