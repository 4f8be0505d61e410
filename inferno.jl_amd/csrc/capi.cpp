// C ABI of libinferno_hip (declared in include/inferno_hip.h).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>

#include "../../include/inferno_hip.h"
#include "chain.h"

// kernels (gemm.hip, dequant.hip, accept.hip, misc.hip)
hipError_t launch_gemm(int qt, const void *W, const float *X, float *Y, int M, int N, int K, int flags, void *ws,
                       hipStream_t st);
size_t gemm_ws_bytes(int qt, int M, int N, int K, int flags);
size_t packed_bytes(int qt, int N, int K);
hipError_t launch_gemm_ex(int qt, const void *W, const float *X, int ldx, int op, const float *norm_w, float eps,
                          const float *add, int n_add, int64_t add_stride, float *Y, int M, int N, int K, int flags,
                          void *ws, hipStream_t st);
bool gemm_reuse_ok(int M, int flags);
void gemm_partials(int qt, int M, int N, int K, int flags, size_t *offset, int *n_slices);
hipError_t launch_pack(int qt, const void *W, void *P, int N, int K, hipStream_t st, int gated);
hipError_t launch_dequant(int qt, const void *w, float *out, int64_t n_blocks, hipStream_t st);
int accept_nchunk(int V);
size_t accept_part_bytes();
hipError_t launch_stats(const float *L, int rows, int V, float T, float T_last, int period, void *part,
                        hipStream_t st);
hipError_t launch_stats_merge(const void *part, int rows, int V, float *zmax, float *zsum, hipStream_t st);
hipError_t launch_spec_accept(const float *tgt, const float *drf, const int32_t *draft_tok, int steps, int k,
                              int V, float T, const float *u_acc, const float *u_res, const float *u_bonus,
                              int mode, const int32_t *bonus_pre, int32_t *out_tok, int32_t *out_n, void *ws,
                              hipStream_t st);
size_t spec_accept_ws(int steps, int k, int V);
hipError_t launch_argmax_partial(const float *L, int rows, int V, float2 *part, hipStream_t st);
hipError_t launch_greedy(const float2 *part, int V, const int32_t *draft_tok, int steps, int k, int32_t *out_n,
                         int32_t *out_argmax, hipStream_t st);
size_t tree_ws(int n, int V);
hipError_t launch_tree(const float *tgt, const float *drf, const int32_t *tok, const int32_t *parent, int n, int V,
                       float T, const float *u, void *ws, int32_t *out_path, int32_t *out_len, hipStream_t st);
hipError_t launch_rmsnorm(const float *x, const float *w, float *out, int rows, int n, float eps, hipStream_t st);
hipError_t launch_silu_mul(const float *gu, int M, int F, float *out, hipStream_t st);
hipError_t launch_add(float *y, const float *x, int64_t n, hipStream_t st);
hipError_t launch_synth(int qt, uint64_t stream, int64_t first, int64_t nblk, void *out, hipStream_t st);
hipError_t launch_commit_state(void *state, const void *snap, int64_t words, int64_t snap_stride, int k,
                               const int32_t *n_acc, int steps, int64_t state_step, int64_t snap_step,
                               hipStream_t st);
hipError_t launch_advance_len(int32_t *len, const int32_t *n_acc, int steps, hipStream_t st);
int sample_max_v();
hipError_t launch_sample(const float *L, int rows, int V, float T, int top_k, float top_p, float min_p, const float *u,
                         int32_t *out, hipStream_t st);
size_t sample_spread_ws(int rows, int V);
hipError_t launch_sample_spread(const float *L, int rows, int V, float T, int top_k, float top_p, float min_p,
                                const float *u, int32_t *out, void *ws, hipStream_t st);
hipError_t launch_penalties(float *L, int rows, int V, const int32_t *tok, int n_tok, int64_t tok_stride,
                            float presence, float repetition, hipStream_t st);
hipError_t launch_gaussian(uint64_t stream, int64_t n, float scale, const float *add, float *out, hipStream_t st);
hipError_t launch_stream_read(const void *src, int64_t bytes, uint32_t *out, hipStream_t st);
// chained matmuls (gemm.hip)
hipError_t launch_gemm_chain_ex(int qt, const void *W, const float *X, int ldx, int op, const float *norm_w,
                                float eps_in, const float *add, int n_add, int64_t add_stride, const Chain &ch,
                                const float *ssq_in, int n_ssq_in, float eps, float *Y, int M, int N, int K,
                                int flags, void *ws, hipStream_t st);
size_t q8k_block_bytes();
hipError_t launch_quantize_q8k(const float *x, void *y, int64_t k, hipStream_t st);
hipError_t launch_vec_dot_q8k(int qt, const void *x, const void *y, int nb, float *out, hipStream_t st);
size_t noalloc_scratch_bytes();
hipError_t noalloc_scratch(void **out);
hipError_t noalloc_prepare(int device);

namespace {

thread_local std::string t_err;
thread_local int t_status = IHIP_OK;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_err = buf;
    t_status = code;
    return code;
}

int ok() {
    t_err.clear();
    t_status = IHIP_OK;
    return IHIP_OK;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(IHIP_EHIP, "%s: %s", what, hipGetErrorString(e));
}

inline hipStream_t S(void *s) { return (hipStream_t)s; }

bool is_qtype(int qt) { return qt == IHIP_Q4_K || qt == IHIP_Q5_K || qt == IHIP_Q6_K || qt == IHIP_Q8_0; }
int block_elems(int qt) { return qt == IHIP_Q8_0 ? 32 : 256; }
int block_bytes(int qt) {
    return qt == IHIP_Q4_K ? 144 : qt == IHIP_Q5_K ? 176 : qt == IHIP_Q6_K ? 210 : 34;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

int check_gemm_shape(int qt, int M, int N, int K, int flags) {
    if (!is_qtype(qt)) return fail(IHIP_EINVAL, "ihip_gemm_q: unsupported qtype %d", qt);
    if (M < 1 || M > 64) return fail(IHIP_EINVAL, "ihip_gemm_q: M=%d outside 1..64", M);
    if (N < 1) return fail(IHIP_EINVAL, "ihip_gemm_q: N=%d", N);
    if (K < 1 || K % block_elems(qt))
        return fail(IHIP_EINVAL, "ihip_gemm_q: K=%d is not a positive multiple of %d", K, block_elems(qt));
    if ((flags & ~15) || ((flags & 3) == 3)) return fail(IHIP_EINVAL, "ihip_gemm_q: bad flags 0x%x", flags);
    return IHIP_OK;
}

int check_gemm(int qt, const void *w, const float *x, float *y, int M, int N, int K, int flags) {
    if (!w || !x || !y) return fail(IHIP_EFAULT, "ihip_gemm_q: NULL pointer");
    const int rc = check_gemm_shape(qt, M, N, K, flags);
    if (rc != IHIP_OK) return rc;
    if (!aligned16(x)) return fail(IHIP_EINVAL, "ihip_gemm_q: x must be 16-byte aligned");
    if (!aligned16(w)) return fail(IHIP_EINVAL, "ihip_gemm_q: weights must be 16-byte aligned");
    return IHIP_OK;
}

// ---- library state for the host-pointer drop-ins ----
// Device copies of drop-in weights, keyed by (host pointer, bytes, qtype, N,
// K). Each entry keeps a fingerprint of sampled host bytes (first, middle
// and last 256 bytes), checked on every call: a host buffer freed and
// reallocated at the same address with other contents (a garbage-collected
// array) is uploaded again instead of served stale. Entries are evicted
// least recently used first when the cached bytes would pass the cap
// (INFERNO_HIP_WEIGHT_CACHE_BYTES, default three quarters of the device's
// memory).
struct WKey {
    const void *ptr;
    size_t bytes;
    int qt, N, K;
    bool operator<(const WKey &o) const {
        if (ptr != o.ptr) return ptr < o.ptr;
        if (bytes != o.bytes) return bytes < o.bytes;
        if (qt != o.qt) return qt < o.qt;
        if (N != o.N) return N < o.N;
        return K < o.K;
    }
};
struct WEntry {
    void *dev;
    size_t dev_bytes;
    uint64_t fingerprint;
    uint64_t last_use;
};
struct Lib {
    std::mutex mu;
    bool inited = false;
    int init_status = IHIP_ENODEV;
    int device = 0;
    hipStream_t stream = nullptr;
    std::map<WKey, WEntry> wcache;
    size_t wcache_bytes = 0, wcache_cap = 0;
    uint64_t use_clock = 0;
    float *dx = nullptr, *dy = nullptr, *dws = nullptr;
    size_t dx_cap = 0, dy_cap = 0, dws_cap = 0;
};

// FNV-1a over the first, middle and last (up to) 256 bytes of the weights.
uint64_t weight_fingerprint(const uint8_t *p, size_t n) {
    uint64_t h = 1469598103934665603ull;
    const size_t span = n < 256 ? n : 256;
    const size_t starts[3] = {0, (n - span) / 2, n - span};
    for (size_t s : starts)
        for (size_t i = 0; i < span; i++) h = (h ^ p[s + i]) * 1099511628211ull;
    return h ^ n;
}
Lib &lib() {
    static Lib L;
    return L;
}

bool disabled_by_env() {
    const char *v = getenv("INFERNO_NO_QUANT_KERNELS");
    return v && strcmp(v, "0") != 0;
}

int init_locked(Lib &L, int device) {
    if (L.inited) return L.init_status;
    L.inited = true;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= device || device < 0)
        return L.init_status = fail(IHIP_ENODEV, "ihip_init: no HIP device %d (%d found)", device, n);
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess) return L.init_status = hip_fail(e, "ihip_init");
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return L.init_status = fail(IHIP_ENODEV, "ihip_init: device %d is %s, not gfx950", device, prop.gcnArchName);
    if ((e = hipSetDevice(device)) != hipSuccess) return L.init_status = hip_fail(e, "ihip_init");
    if ((e = hipStreamCreateWithFlags(&L.stream, hipStreamNonBlocking)) != hipSuccess)
        return L.init_status = hip_fail(e, "ihip_init");
    L.device = device;
    const char *cap = getenv("INFERNO_HIP_WEIGHT_CACHE_BYTES");
    L.wcache_cap = cap && *cap ? (size_t)strtoull(cap, nullptr, 10) : prop.totalGlobalMem / 4 * 3;
    return L.init_status = IHIP_OK;
}

void wcache_drop(Lib &L, std::map<WKey, WEntry>::iterator it) {
    (void)hipFree(it->second.dev);
    L.wcache_bytes -= it->second.dev_bytes;
    L.wcache.erase(it);
}

// Evicts least-recently-used entries until `need` more bytes fit under the cap.
void wcache_make_room(Lib &L, size_t need) {
    while (!L.wcache.empty() && L.wcache_bytes + need > L.wcache_cap) {
        auto lru = L.wcache.begin();
        for (auto it = L.wcache.begin(); it != L.wcache.end(); ++it)
            if (it->second.last_use < lru->second.last_use) lru = it;
        wcache_drop(L, lru);
    }
}

int grow(float **p, size_t *cap, size_t bytes) {
    if (*cap >= bytes) return IHIP_OK;
    if (*p) (void)hipFree(*p);
    *p = nullptr;
    *cap = 0;
    hipError_t e = hipMalloc((void **)p, bytes);
    if (e != hipSuccess) return hip_fail(e, "drop-in buffer");
    *cap = bytes;
    return IHIP_OK;
}

// Drop-in GEMV: host pointers, synchronous on the library stream. On any
// failure out[0..N) is filled with NaN (the reference's C entry points
// return void, so an unmodified caller never reads the status: NaN makes the
// failure visible downstream instead of leaving stale values).
void dropin_gemv(const char *name, int qt, const uint8_t *weight, const float *x, float *out, int K, int N) {
    Lib &L = lib();
    std::lock_guard<std::mutex> lk(L.mu);
    int rc;
    if (disabled_by_env()) {
        rc = fail(IHIP_ENODEV, "%s: disabled by INFERNO_NO_QUANT_KERNELS", name);
    } else if ((rc = init_locked(L, 0)) != IHIP_OK) {
        // message already set
    } else if (!weight || !x || !out) {
        rc = fail(IHIP_EFAULT, "%s: NULL pointer", name);
    } else if (K < 1 || K % block_elems(qt) || N < 1) {
        rc = fail(IHIP_EINVAL, "%s: inner_dim=%d outer_dim=%d (inner_dim must be a positive multiple of %d)",
                  name, K, N, block_elems(qt));
    } else {
        (void)hipSetDevice(L.device);
        const size_t wbytes = (size_t)N * (K / block_elems(qt)) * block_bytes(qt);
        const WKey key{(const void *)weight, wbytes, qt, N, K};
        const uint64_t fp = weight_fingerprint(weight, wbytes);
        void *dw = nullptr;
        auto it = L.wcache.find(key);
        if (it != L.wcache.end() && it->second.fingerprint != fp) {
            wcache_drop(L, it);  // same address, other contents: upload again
            it = L.wcache.end();
        }
        hipError_t e = hipSuccess;
        if (it != L.wcache.end()) {
            dw = it->second.dev;
            it->second.last_use = ++L.use_clock;
        } else {
            // first call with this matrix: upload, repack once, keep the packed copy
            const size_t pbytes = packed_bytes(qt, N, K);
            wcache_make_room(L, pbytes);
            void *raw = nullptr;
            e = hipMalloc(&raw, wbytes);
            if (e == hipSuccess) e = hipMalloc(&dw, pbytes);
            if (e == hipSuccess) e = hipMemcpy(raw, weight, wbytes, hipMemcpyHostToDevice);
            if (e == hipSuccess) e = launch_pack(qt, raw, dw, N, K, L.stream, 0);
            if (e == hipSuccess) e = hipStreamSynchronize(L.stream);
            if (raw) (void)hipFree(raw);
            if (e == hipSuccess) {
                L.wcache[key] = WEntry{dw, pbytes, fp, ++L.use_clock};
                L.wcache_bytes += pbytes;
            } else if (dw) {
                (void)hipFree(dw);
                dw = nullptr;
            }
        }
        if (e != hipSuccess) {
            rc = hip_fail(e, name);
        } else if ((rc = grow(&L.dx, &L.dx_cap, (size_t)K * 4)) == IHIP_OK &&
                   (rc = grow(&L.dy, &L.dy_cap, (size_t)N * 4)) == IHIP_OK &&
                   (rc = grow(&L.dws, &L.dws_cap, gemm_ws_bytes(qt, 1, N, K, IHIP_GEMM_F32 | IHIP_GEMM_PACKED))) ==
                       IHIP_OK) {
            e = hipMemcpyAsync(L.dx, x, (size_t)K * 4, hipMemcpyHostToDevice, L.stream);
            if (e == hipSuccess)
                e = launch_gemm(qt, dw, L.dx, L.dy, 1, N, K, IHIP_GEMM_F32 | IHIP_GEMM_PACKED, L.dws, L.stream);
            if (e == hipSuccess) e = hipMemcpyAsync(out, L.dy, (size_t)N * 4, hipMemcpyDeviceToHost, L.stream);
            if (e == hipSuccess) e = hipStreamSynchronize(L.stream);
            rc = e == hipSuccess ? ok() : hip_fail(e, name);
        }
    }
    if (rc != IHIP_OK) {
        fprintf(stderr, "inferno_hip: %s\n", t_err.c_str());
        if (out && N > 0)
            for (int i = 0; i < N; i++) out[i] = __builtin_nanf("");
    }
}

// Host-pointer round trip of the Q8_K helpers on the library stream: copies
// `nin` input buffers to scratch device memory, runs `launch`, copies `out_bytes`
// back. The scratch buffers (dx, dws) grow as needed and stay allocated.
template <class F>
int dropin_roundtrip(Lib &L, const char *name, const void *in0, size_t b0, const void *in1, size_t b1, void *out,
                     size_t out_bytes, F launch) {
    int rc;
    if (disabled_by_env()) return fail(IHIP_ENODEV, "%s: disabled by INFERNO_NO_QUANT_KERNELS", name);
    if ((rc = init_locked(L, 0)) != IHIP_OK) return rc;
    (void)hipSetDevice(L.device);
    const size_t a0 = (b0 + 255) & ~(size_t)255, a1 = (b1 + 255) & ~(size_t)255;
    if ((rc = grow(&L.dws, &L.dws_cap, a0 + a1 + out_bytes)) != IHIP_OK) return rc;
    uint8_t *base = (uint8_t *)L.dws;
    hipError_t e = hipMemcpyAsync(base, in0, b0, hipMemcpyHostToDevice, L.stream);
    if (e == hipSuccess && in1) e = hipMemcpyAsync(base + a0, in1, b1, hipMemcpyHostToDevice, L.stream);
    if (e == hipSuccess) e = launch(base, base + a0, base + a0 + a1, L.stream);
    if (e == hipSuccess) e = hipMemcpyAsync(out, base + a0 + a1, out_bytes, hipMemcpyDeviceToHost, L.stream);
    if (e == hipSuccess) e = hipStreamSynchronize(L.stream);
    return e == hipSuccess ? ok() : hip_fail(e, name);
}

float dropin_vec_dot(const char *name, int qt, const void *x, const void *y, int nb) {
    Lib &L = lib();
    std::lock_guard<std::mutex> lk(L.mu);
    float r = __builtin_nanf("");
    int rc;
    if (!x || !y) {
        rc = fail(IHIP_EFAULT, "%s: NULL pointer", name);
    } else if (nb < 0) {
        rc = fail(IHIP_EINVAL, "%s: nb=%d", name, nb);
    } else if (nb == 0) {
        ok();
        return 0.0f;
    } else {
        rc = dropin_roundtrip(L, name, x, (size_t)nb * block_bytes(qt), y, (size_t)nb * q8k_block_bytes(), &r,
                              sizeof(float), [&](uint8_t *dx, uint8_t *dy, uint8_t *dout, hipStream_t st) {
                                  return launch_vec_dot_q8k(qt, dx, dy, nb, (float *)dout, st);
                              });
    }
    if (rc != IHIP_OK) {
        fprintf(stderr, "inferno_hip: %s\n", t_err.c_str());
        return __builtin_nanf("");
    }
    return r;
}

}  // namespace

extern "C" {

void quantize_row_q8_K(const float *x, void *y, int64_t k) {
    Lib &L = lib();
    std::lock_guard<std::mutex> lk(L.mu);
    int rc;
    if (!x || !y) {
        rc = fail(IHIP_EFAULT, "quantize_row_q8_K: NULL pointer");
    } else if (k < 0 || k % 256) {
        rc = fail(IHIP_EINVAL, "quantize_row_q8_K: k=%lld is not a multiple of 256", (long long)k);
    } else if (k == 0) {
        rc = ok();
    } else {
        const size_t nb = (size_t)(k / 256);
        rc = dropin_roundtrip(L, "quantize_row_q8_K", x, (size_t)k * 4, nullptr, 0, y, nb * q8k_block_bytes(),
                              [&](uint8_t *dx, uint8_t *, uint8_t *dout, hipStream_t st) {
                                  return launch_quantize_q8k((const float *)dx, dout, k, st);
                              });
    }
    if (rc != IHIP_OK) {
        fprintf(stderr, "inferno_hip: %s\n", t_err.c_str());
        if (y && k > 0 && k % 256 == 0) {  // d = NaN in every block: downstream dot products show the failure
            const float nan = __builtin_nanf("");
            for (int64_t b = 0; b < k / 256; b++) memcpy((uint8_t *)y + b * q8k_block_bytes(), &nan, 4);
        }
    }
}

float vec_dot_q4_K_q8_K(const void *x, const void *y, int nb) { return dropin_vec_dot("vec_dot_q4_K_q8_K", IHIP_Q4_K, x, y, nb); }
float vec_dot_q5_K_q8_K(const void *x, const void *y, int nb) { return dropin_vec_dot("vec_dot_q5_K_q8_K", IHIP_Q5_K, x, y, nb); }
float vec_dot_q6_K_q8_K(const void *x, const void *y, int nb) { return dropin_vec_dot("vec_dot_q6_K_q8_K", IHIP_Q6_K, x, y, nb); }

const char *ihip_last_error(void) { return t_err.c_str(); }
// status reporting for the other host files of the library (gguf.cpp)
__attribute__((visibility("hidden"))) int ihip_internal_fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return fail(code, "%s", buf);
}
__attribute__((visibility("hidden"))) int ihip_internal_ok() { return ok(); }

int ihip_last_status(void) { return t_status; }

int ihip_init(int device) {
    Lib &L = lib();
    std::lock_guard<std::mutex> lk(L.mu);
    const int rc = init_locked(L, device);
    if (rc != IHIP_OK) return rc;
    // the allocation-free entry point's scratch address on this device, so
    // that a call under graph capture finds it already resolved
    const hipError_t e = noalloc_prepare(device);
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_init: device scratch");
}

int ihip_available(void) {
    if (disabled_by_env()) return 0;
    return ihip_init(0) == IHIP_OK ? 1 : 0;
}

void ihip_weight_cache_clear(void) {
    Lib &L = lib();
    std::lock_guard<std::mutex> lk(L.mu);
    for (auto &kv : L.wcache) (void)hipFree(kv.second.dev);
    L.wcache.clear();
    L.wcache_bytes = 0;
}

void q4_k_gemv(const uint8_t *weight, const float *x, float *out, void *q8_buf, int inner_dim, int outer_dim) {
    (void)q8_buf;
    dropin_gemv("q4_k_gemv", IHIP_Q4_K, weight, x, out, inner_dim, outer_dim);
}
void q5_k_gemv(const uint8_t *weight, const float *x, float *out, void *q8_buf, int inner_dim, int outer_dim) {
    (void)q8_buf;
    dropin_gemv("q5_k_gemv", IHIP_Q5_K, weight, x, out, inner_dim, outer_dim);
}
void q6_k_gemv(const uint8_t *weight, const float *x, float *out, void *q8_buf, int inner_dim, int outer_dim) {
    (void)q8_buf;
    dropin_gemv("q6_k_gemv", IHIP_Q6_K, weight, x, out, inner_dim, outer_dim);
}
void q8_0_gemv(const uint8_t *weight, const float *x, float *out, int inner_dim, int outer_dim) {
    dropin_gemv("q8_0_gemv", IHIP_Q8_0, weight, x, out, inner_dim, outer_dim);
}

int ihip_gemm_q_ws_bytes(int qtype, int M, int N, int K, int flags, size_t *bytes) {
    if (!bytes) return fail(IHIP_EFAULT, "ihip_gemm_q_ws_bytes: NULL");
    int rc = check_gemm_shape(qtype, M, N, K, flags);
    if (rc != IHIP_OK) return rc;
    *bytes = gemm_ws_bytes(qtype, M, N, K, flags);
    return ok();
}

int ihip_gemm_q(int qtype, const void *w_dev, const float *x_dev, float *y_dev, int M, int N, int K, int flags,
                void *ws, size_t ws_bytes, void *stream) {
    int rc = check_gemm(qtype, w_dev, x_dev, y_dev, M, N, K, flags);
    if (rc != IHIP_OK) return rc;
    const size_t need = gemm_ws_bytes(qtype, M, N, K, flags);
    if (!ws) return fail(IHIP_EFAULT, "ihip_gemm_q: NULL workspace (%zu bytes needed)", need);
    if (ws_bytes < need) return fail(IHIP_ENOMEM, "ihip_gemm_q: workspace %zu < %zu bytes", ws_bytes, need);
    if (!aligned16(ws)) return fail(IHIP_EINVAL, "ihip_gemm_q: workspace must be 16-byte aligned");
    hipError_t e = launch_gemm(qtype, w_dev, x_dev, y_dev, M, N, K, flags, ws, S(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_gemm_q");
}

int ihip_gemm_q_noalloc(int qtype, const void *w_dev, const float *x_dev, float *y_dev, int M, int N, int K,
                        int flags, void *stream) {
    int rc = check_gemm(qtype, w_dev, x_dev, y_dev, M, N, K, flags);
    if (rc != IHIP_OK) return rc;
    const size_t need = gemm_ws_bytes(qtype, M, N, K, flags);
    if (need > noalloc_scratch_bytes())
        return fail(IHIP_ENOMEM, "ihip_gemm_q_noalloc: this shape needs %zu bytes of scratch, above the fixed %zu "
                    "(use ihip_gemm_q with a caller workspace)", need, noalloc_scratch_bytes());
    void *scr = nullptr;
    hipError_t e = noalloc_scratch(&scr);
    if (e != hipSuccess) return hip_fail(e, "ihip_gemm_q_noalloc: device scratch");
    e = launch_gemm(qtype, w_dev, x_dev, y_dev, M, N, K, flags, scr, S(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_gemm_q_noalloc");
}

int ihip_pack_weights_gated(int qtype, const void *w_gguf_dev, void *w_packed_dev, int F, int K, void *stream) {
    if (!w_gguf_dev || !w_packed_dev) return fail(IHIP_EFAULT, "ihip_pack_weights_gated: NULL pointer");
    if (!is_qtype(qtype) || F < 8 || F % 8 || K < 1 || K % block_elems(qtype))
        return fail(IHIP_EINVAL, "ihip_pack_weights_gated: qtype %d F=%d K=%d (F a multiple of 8)", qtype, F, K);
    hipError_t e = launch_pack(qtype, w_gguf_dev, w_packed_dev, 2 * F, K, S(stream), F);
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_pack_weights_gated");
}

size_t ihip_chain_operand_bytes(int K) { return K > 0 ? (size_t)chain_operand_bytes(K) : 0; }

int ihip_gemm_q_chain(int qtype, const void *w_packed, const ihip_gemm_input *in, const ihip_chain_in *cin,
                      const ihip_chain_out *cout, int M, int N, int K, int flags, void *ws, size_t ws_bytes,
                      void *stream) {
    const char *fn = "ihip_gemm_q_chain";
    if (!w_packed || !ws) return fail(IHIP_EFAULT, "%s: NULL weights or workspace", fn);
    if ((in == nullptr) == (cin == nullptr)) return fail(IHIP_EINVAL, "%s: pass exactly one of in / cin", fn);
    const bool defer = flags & IHIP_GEMM_DEFER;
    if (flags & ~(IHIP_GEMM_F32 | IHIP_GEMM_PACKED | IHIP_GEMM_DEFER))
        return fail(IHIP_EINVAL, "%s: flags 0x%x (fp32-accurate packed only, IHIP_GEMM_DEFER allowed)", fn, flags);
    int rc = check_gemm_shape(qtype, M, N, K, IHIP_GEMM_F32 | IHIP_GEMM_PACKED);
    if (rc != IHIP_OK) return rc;
    if (M > 8) return fail(IHIP_EINVAL, "%s: M=%d (chained calls hold one token tile: M <= 8)", fn, M);
    if (!aligned16(w_packed) || !aligned16(ws)) return fail(IHIP_EINVAL, "%s: weights/workspace 16-byte aligned", fn);
    const size_t need = gemm_ws_bytes(qtype, M, N, K, IHIP_GEMM_F32 | IHIP_GEMM_PACKED);
    if (ws_bytes < need) return fail(IHIP_ENOMEM, "%s: workspace %zu < %zu bytes", fn, ws_bytes, need);
    Chain ch{};
    ch.epi = IHIP_EPI_STORE;
    ch.ldy = N;
    float *y = nullptr;
    if (cout) {
        const int e = cout->epi;
        if (e < IHIP_EPI_STORE || e > IHIP_EPI_GATE) return fail(IHIP_EINVAL, "%s: epi=%d", fn, e);
        if (!cout->y) return fail(IHIP_EFAULT, "%s: NULL y", fn);
        if (defer) return fail(IHIP_EINVAL, "%s: IHIP_GEMM_DEFER leaves partials: no output descriptor", fn);
        const int width = e == IHIP_EPI_GATE ? N / 2 : N;
        if (cout->ldy < width || (e == IHIP_EPI_GATE && N % 16))
            return fail(IHIP_EINVAL, "%s: ldy=%d (need >= %d; IHIP_EPI_GATE needs N %% 16 == 0)", fn, cout->ldy, width);
        if (e != IHIP_EPI_STORE) {
            // the next matmul's K: whole 256-element units
            const int kn = e == IHIP_EPI_STATS ? cout->stat_rows : width;
            const int tiles = e == IHIP_EPI_GATE ? kn / 8 : kn / 16;
            if (e == IHIP_EPI_STATS && (cout->stat_rows < 256 || cout->stat_rows > N))
                return fail(IHIP_EINVAL, "%s: stat_rows=%d (within N)", fn, cout->stat_rows);
            if (kn % 256) return fail(IHIP_EINVAL, "%s: the operand covers %d values (a multiple of 256)", fn, kn);
            const int cq = cout->consumer_qtype;
            if (cq != IHIP_Q4_K && cq != IHIP_Q5_K && cq != IHIP_Q6_K && cq != IHIP_Q8_0)
                return fail(IHIP_EINVAL, "%s: consumer_qtype=%d", fn, cq);
            if (cout->operand && !aligned16(cout->operand)) return fail(IHIP_EINVAL, "%s: operand 16-byte aligned", fn);
            if (cout->tile_sum && (!aligned16(cout->tile_sum) || (cout->sum_stride & 3) || cout->sum_stride < tiles))
                return fail(IHIP_EINVAL, "%s: tile_sum 16-byte aligned, sum_stride=%d >= %d tiles and a multiple of 4",
                            fn, cout->sum_stride, tiles);
            ch.op_lk = cq == IHIP_Q6_K ? 1 : cq == IHIP_Q8_0 ? 2 : 0;
            ch.yop = (uint8_t *)cout->operand;
            ch.y_units = kn / 256;
            ch.ysum = cout->tile_sum;
            ch.ysum_stride = cout->sum_stride;
            ch.yssq = cout->tile_ssq;
            ch.stat_rows = cout->stat_rows;
        }
        ch.epi = e;
        ch.ldy = cout->ldy;
        ch.yw = cout->norm_w;
        y = cout->y;
    } else if (!defer) {
        return fail(IHIP_EINVAL, "%s: no output descriptor and no IHIP_GEMM_DEFER", fn);
    }
    const float *ssq_in = nullptr;
    int n_ssq = 0;
    float eps = 0.f;
    hipError_t err;
    if (cin) {
        if (K % 256) return fail(IHIP_EINVAL, "%s: a chained input needs K %% 256 == 0", fn);
        const int tpu = cin->tiles_per_unit;
        if (!cin->operand) return fail(IHIP_EFAULT, "%s: NULL operand", fn);
        if (!aligned16(cin->operand)) return fail(IHIP_EINVAL, "%s: operand 16-byte aligned", fn);
        if (tpu != 16 && tpu != 32) return fail(IHIP_EINVAL, "%s: tiles_per_unit=%d (16 or 32)", fn, tpu);
        const bool mins = qtype == IHIP_Q4_K || qtype == IHIP_Q5_K;
        if (mins && (!cin->tile_sum || !aligned16(cin->tile_sum) || (cin->sum_stride & 3) ||
                     cin->sum_stride < (K / 256) * tpu))
            return fail(IHIP_EINVAL, "%s: Q4_K/Q5_K need tile_sum (16-byte aligned, sum_stride=%d >= %d, a multiple "
                                     "of 4)", fn, cin->sum_stride, (K / 256) * tpu);
        if (cin->tile_ssq && (cin->ssq_tiles < 1 || !(cin->eps >= 0.f)))
            return fail(IHIP_EINVAL, "%s: ssq_tiles=%d eps=%g", fn, cin->ssq_tiles, cin->eps);
        ch.xop = (const uint8_t *)cin->operand;
        ch.xsum = cin->tile_sum;
        ch.xsum_stride = cin->sum_stride;
        ch.x_tiles_per_unit = tpu;
        ssq_in = cin->tile_ssq;
        n_ssq = cin->tile_ssq ? cin->ssq_tiles : 0;
        eps = cin->eps;
        err = launch_gemm_chain_ex(qtype, w_packed, nullptr, 0, 0, nullptr, 0.f, nullptr, 0, 0, ch, ssq_in, n_ssq,
                                   eps, y, M, N, K, flags, ws, S(stream));
    } else {
        const int act = in->act;
        if (!in->x) return fail(IHIP_EFAULT, "%s: NULL in->x", fn);
        if (act < IHIP_ACT_PLAIN || act > IHIP_ACT_SILU_MUL) return fail(IHIP_EINVAL, "%s: act=%d", fn, act);
        const int min_ld = act == IHIP_ACT_SILU_MUL ? 2 * K : K;
        if (in->ldx < min_ld || (in->ldx & 3) || !aligned16(in->x))
            return fail(IHIP_EINVAL, "%s: ldx=%d (need >= %d, multiple of 4; x 16-byte aligned)", fn, in->ldx, min_ld);
        if (act == IHIP_ACT_RMSNORM && !(in->eps >= 0.f)) return fail(IHIP_EINVAL, "%s: eps=%g", fn, in->eps);
        if (in->add && (in->n_add < 1 || in->add_stride < (int64_t)M * K || (in->add_stride & 3) || !aligned16(in->add)))
            return fail(IHIP_EINVAL, "%s: add slices n=%d stride=%lld", fn, in->n_add, (long long)in->add_stride);
        err = launch_gemm_chain_ex(qtype, w_packed, in->x, in->ldx, act, act == IHIP_ACT_RMSNORM ? in->norm_w : nullptr,
                                   in->eps, in->add, in->add ? in->n_add : 0, in->add_stride, ch, nullptr, 0, 0.f, y, M,
                                   N, K, flags, ws, S(stream));
    }
    if (err == hipErrorInvalidValue)
        return fail(IHIP_EINVAL, "%s: shape not on the one-tile streaming plan", fn);
    return err == hipSuccess ? ok() : hip_fail(err, fn);
}

int ihip_gemm_q_ex(int qtype, const void *w_dev, const ihip_gemm_input *in, float *y_dev, int M, int N, int K,
                   int flags, void *ws, size_t ws_bytes, void *stream) {
    if (!in) return fail(IHIP_EFAULT, "ihip_gemm_q_ex: NULL input descriptor");
    const int base = flags & ~(IHIP_GEMM_REUSE | IHIP_GEMM_DEFER | IHIP_GEMM_SUM_OUT);
    const bool defer = flags & IHIP_GEMM_DEFER;
    // x absent: the input is the sum of the add slices themselves; with
    // SUM_OUT that sum is also stored into x
    const bool sum_out = flags & IHIP_GEMM_SUM_OUT;
    if (!in->x && !in->add) return fail(IHIP_EFAULT, "ihip_gemm_q_ex: NULL x without add slices");
    if (sum_out && (!in->x || !in->add))
        return fail(IHIP_EFAULT, "ihip_gemm_q_ex: IHIP_GEMM_SUM_OUT needs x (the sum's destination) and add slices");
    const float *xin = in->x ? in->x : in->add;
    int rc = check_gemm(qtype, w_dev, xin, defer ? const_cast<float *>(xin) : y_dev, M, N, K, base);
    if (rc != IHIP_OK) return rc;
    const int act = in->act;
    if (act < IHIP_ACT_PLAIN || act > IHIP_ACT_SILU_MUL) return fail(IHIP_EINVAL, "ihip_gemm_q_ex: act=%d", act);
    const int min_ld = act == IHIP_ACT_SILU_MUL ? 2 * K : K;
    if (in->ldx < min_ld || (in->ldx & 3))
        return fail(IHIP_EINVAL, "ihip_gemm_q_ex: ldx=%d (need >= %d, multiple of 4)", in->ldx, min_ld);
    if ((K & 7) != 0) return fail(IHIP_EINVAL, "ihip_gemm_q_ex: K=%d must be a multiple of 8", K);
    if (act == IHIP_ACT_RMSNORM && !(in->eps >= 0.f)) return fail(IHIP_EINVAL, "ihip_gemm_q_ex: eps=%g", in->eps);
    if (in->norm_w && !aligned16(in->norm_w)) return fail(IHIP_EINVAL, "ihip_gemm_q_ex: norm_w must be 16-byte aligned");
    if (sum_out) {
        if (act == IHIP_ACT_SILU_MUL) return fail(IHIP_EINVAL, "ihip_gemm_q_ex: IHIP_GEMM_SUM_OUT with SILU_MUL");
        if ((K & 255) || (in->ldx & 7))
            return fail(IHIP_EINVAL, "ihip_gemm_q_ex: IHIP_GEMM_SUM_OUT needs K %% 256 == 0 and ldx %% 8 == 0 (K=%d ldx=%d)",
                        K, in->ldx);
        if (!aligned16(in->x)) return fail(IHIP_EINVAL, "ihip_gemm_q_ex: IHIP_GEMM_SUM_OUT x must be 16-byte aligned");
    }
    if (in->add) {
        const int64_t slice = (int64_t)M * (in->x && !sum_out ? K : in->ldx);
        if (in->n_add < 1 || in->add_stride < slice || (in->add_stride & 3) || !aligned16(in->add))
            return fail(IHIP_EINVAL, "ihip_gemm_q_ex: add slices n=%d stride=%lld", in->n_add,
                        (long long)in->add_stride);
        if (act == IHIP_ACT_SILU_MUL && in->x && !sum_out)
            return fail(IHIP_EINVAL, "ihip_gemm_q_ex: add with SILU_MUL needs x = NULL (the slices are the input)");
        if (flags & IHIP_GEMM_REUSE) return fail(IHIP_EINVAL, "ihip_gemm_q_ex: add with IHIP_GEMM_REUSE");
    }
    if ((flags & (IHIP_GEMM_REUSE | IHIP_GEMM_DEFER)) && !gemm_reuse_ok(M, base))
        return fail(IHIP_EINVAL, "ihip_gemm_q_ex: REUSE/DEFER need M <= 32 in fp32-accurate mode");
    if (defer && (flags & IHIP_GEMM_ACCUM)) return fail(IHIP_EINVAL, "ihip_gemm_q_ex: DEFER with ACCUM");
    const size_t need = gemm_ws_bytes(qtype, M, N, K, base);
    if (!ws) return fail(IHIP_EFAULT, "ihip_gemm_q_ex: NULL workspace (%zu bytes needed)", need);
    if (ws_bytes < need) return fail(IHIP_ENOMEM, "ihip_gemm_q_ex: workspace %zu < %zu bytes", ws_bytes, need);
    if (!aligned16(ws)) return fail(IHIP_EINVAL, "ihip_gemm_q_ex: workspace must be 16-byte aligned");
    hipError_t e = launch_gemm_ex(qtype, w_dev, in->x, in->ldx, act, act == IHIP_ACT_RMSNORM ? in->norm_w : nullptr,
                                  in->eps, in->add, in->add ? in->n_add : 0, in->add_stride, y_dev, M, N, K, flags,
                                  ws, S(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_gemm_q_ex");
}

// ---- MLP half of a decoder layer ----
namespace {
size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

int check_mlp(const char *name, int qg, int qd, int M, int H, int F, int flags) {
    if (flags & ~(IHIP_GEMM_F32 | IHIP_GEMM_HALF | IHIP_GEMM_PACKED))
        return fail(IHIP_EINVAL, "%s: flags 0x%x (only F32, HALF, PACKED)", name, flags);
    if (H < 1 || F < 1 || (H & 7) || (F & 7))
        return fail(IHIP_EINVAL, "%s: H=%d F=%d must be positive multiples of 8", name, H, F);
    int rc = check_gemm_shape(qg, M, 2 * F, H, flags);
    if (rc != IHIP_OK) return rc;
    return check_gemm_shape(qd, M, H, F, flags | IHIP_GEMM_ACCUM);
}

size_t mlp_ws(int qg, int qd, int M, int H, int F, int flags) {
    const size_t g = gemm_ws_bytes(qg, M, 2 * F, H, flags);
    const size_t d = gemm_ws_bytes(qd, M, H, F, flags | IHIP_GEMM_ACCUM);
    return align256((size_t)M * 2 * F * sizeof(float)) + (g > d ? g : d);
}
}  // namespace

int ihip_mlp_ws_bytes(int qt_gate_up, int qt_down, int M, int H, int F, int flags, size_t *bytes) {
    if (!bytes) return fail(IHIP_EFAULT, "ihip_mlp_ws_bytes: NULL");
    const int rc = check_mlp("ihip_mlp_ws_bytes", qt_gate_up, qt_down, M, H, F, flags);
    if (rc != IHIP_OK) return rc;
    *bytes = mlp_ws(qt_gate_up, qt_down, M, H, F, flags);
    return ok();
}

int ihip_mlp_forward(int qt_gate_up, const void *w_gate_up, int qt_down, const void *w_down, float *x,
                     const float *norm_w, float eps, int M, int H, int F, int flags, void *ws, size_t ws_bytes,
                     void *stream) {
    if (!w_gate_up || !w_down || !x) return fail(IHIP_EFAULT, "ihip_mlp_forward: NULL pointer");
    int rc = check_mlp("ihip_mlp_forward", qt_gate_up, qt_down, M, H, F, flags);
    if (rc != IHIP_OK) return rc;
    if (!aligned16(x) || !aligned16(w_gate_up) || !aligned16(w_down) || (norm_w && !aligned16(norm_w)))
        return fail(IHIP_EINVAL, "ihip_mlp_forward: x, weights and norm_w must be 16-byte aligned");
    if (!(eps >= 0.f)) return fail(IHIP_EINVAL, "ihip_mlp_forward: eps=%g", eps);
    const size_t need = mlp_ws(qt_gate_up, qt_down, M, H, F, flags);
    if (!ws) return fail(IHIP_EFAULT, "ihip_mlp_forward: NULL workspace (%zu bytes needed)", need);
    if (ws_bytes < need) return fail(IHIP_ENOMEM, "ihip_mlp_forward: workspace %zu < %zu bytes", ws_bytes, need);
    if (!aligned16(ws)) return fail(IHIP_EINVAL, "ihip_mlp_forward: workspace must be 16-byte aligned");
    float *gu = (float *)ws;
    void *gws = (uint8_t *)ws + align256((size_t)M * 2 * F * sizeof(float));
    // [gate; up] of the normalized residual, then x += down(silu(gate) * up)
    hipError_t e = launch_gemm_ex(qt_gate_up, w_gate_up, x, H, IHIP_ACT_RMSNORM, norm_w, eps, nullptr, 0, 0, gu, M,
                                  2 * F, H, flags, gws, S(stream));
    if (e == hipSuccess)
        e = launch_gemm_ex(qt_down, w_down, gu, 2 * F, IHIP_ACT_SILU_MUL, nullptr, 0.f, nullptr, 0, 0, x, M, H, F,
                           flags | IHIP_GEMM_ACCUM, gws, S(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_mlp_forward");
}

int ihip_gemm_q_partials(int qtype, int M, int N, int K, int flags, void *ws, float **slices, int *n_slices,
                         int64_t *stride) {
    if (!ws || !slices || !n_slices || !stride) return fail(IHIP_EFAULT, "ihip_gemm_q_partials: NULL pointer");
    const int base = flags & ~(IHIP_GEMM_REUSE | IHIP_GEMM_DEFER | IHIP_GEMM_SUM_OUT);
    const int rc = check_gemm_shape(qtype, M, N, K, base);
    if (rc != IHIP_OK) return rc;
    size_t off = 0;
    gemm_partials(qtype, M, N, K, base, &off, n_slices);
    *slices = (float *)((uint8_t *)ws + off);
    *stride = (int64_t)M * N;
    return ok();
}

int ihip_packed_bytes(int qtype, int N, int K, size_t *bytes) {
    if (!bytes) return fail(IHIP_EFAULT, "ihip_packed_bytes: NULL");
    const int rc = check_gemm_shape(qtype, 1, N, K, 0);
    if (rc != IHIP_OK) return rc;
    *bytes = packed_bytes(qtype, N, K);
    return ok();
}

int ihip_pack_weights(int qtype, const void *w_gguf_dev, void *w_packed_dev, int N, int K, void *stream) {
    if (!w_gguf_dev || !w_packed_dev) return fail(IHIP_EFAULT, "ihip_pack_weights: NULL pointer");
    const int rc = check_gemm_shape(qtype, 1, N, K, 0);
    if (rc != IHIP_OK) return rc;
    if (!aligned16(w_packed_dev)) return fail(IHIP_EINVAL, "ihip_pack_weights: packed buffer must be 16-byte aligned");
    hipError_t e = launch_pack(qtype, w_gguf_dev, w_packed_dev, N, K, S(stream), 0);
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_pack_weights");
}

int ihip_dequant(int qtype, const void *w_dev, float *out_dev, int64_t n_elems, void *stream) {
    if (!w_dev || !out_dev) return fail(IHIP_EFAULT, "ihip_dequant: NULL pointer");
    if (!is_qtype(qtype)) return fail(IHIP_EINVAL, "ihip_dequant: unsupported qtype %d", qtype);
    if (n_elems < 0 || n_elems % block_elems(qtype))
        return fail(IHIP_EINVAL, "ihip_dequant: n_elems=%lld is not a multiple of %d", (long long)n_elems,
                    block_elems(qtype));
    if (((uintptr_t)out_dev & 15) != 0) return fail(IHIP_EINVAL, "ihip_dequant: out must be 16-byte aligned");
    hipError_t e = launch_dequant(qtype, w_dev, out_dev, n_elems / block_elems(qtype), S(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_dequant");
}

int ihip_rmsnorm(const float *x_dev, const float *w_dev, float *out_dev, int rows, int n, float eps, void *stream) {
    if (!x_dev || !out_dev) return fail(IHIP_EFAULT, "ihip_rmsnorm: NULL pointer");
    if (rows < 0 || n < 1) return fail(IHIP_EINVAL, "ihip_rmsnorm: rows=%d n=%d", rows, n);
    hipError_t e = launch_rmsnorm(x_dev, w_dev, out_dev, rows, n, eps, S(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_rmsnorm");
}

int ihip_silu_mul(const float *gu_dev, int M, int F, float *out_dev, void *stream) {
    if (!gu_dev || !out_dev) return fail(IHIP_EFAULT, "ihip_silu_mul: NULL pointer");
    if (M < 0 || F < 1) return fail(IHIP_EINVAL, "ihip_silu_mul: M=%d F=%d", M, F);
    hipError_t e = launch_silu_mul(gu_dev, M, F, out_dev, S(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_silu_mul");
}

int ihip_add(float *y_dev, const float *x_dev, int64_t n, void *stream) {
    if (!y_dev || !x_dev) return fail(IHIP_EFAULT, "ihip_add: NULL pointer");
    if (n < 0) return fail(IHIP_EINVAL, "ihip_add: n=%lld", (long long)n);
    hipError_t e = launch_add(y_dev, x_dev, n, S(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_add");
}

int ihip_accept_ws_bytes(int rows, int V, size_t *bytes) {
    if (!bytes) return fail(IHIP_EFAULT, "ihip_accept_ws_bytes: NULL");
    if (rows < 0 || V < 1) return fail(IHIP_EINVAL, "ihip_accept_ws_bytes: rows=%d V=%d", rows, V);
    *bytes = (size_t)rows * accept_nchunk(V) * accept_part_bytes() + (size_t)rows * 16 + 256;
    return ok();
}

static int need_ws(const char *name, int rows, int V, void *ws, size_t ws_bytes) {
    size_t need = 0;
    ihip_accept_ws_bytes(rows, V, &need);
    if (!ws) return fail(IHIP_EFAULT, "%s: NULL workspace", name);
    if (ws_bytes < need) return fail(IHIP_ENOMEM, "%s: workspace %zu < %zu bytes", name, ws_bytes, need);
    if (((uintptr_t)ws & 15) != 0) return fail(IHIP_EINVAL, "%s: workspace must be 16-byte aligned", name);
    return IHIP_OK;
}

int ihip_softmax_stats(const float *logits_dev, int rows, int V, float T, float *zmax_dev, float *zsum_dev,
                       void *ws, size_t ws_bytes, void *stream) {
    if (!logits_dev || !zmax_dev || !zsum_dev) return fail(IHIP_EFAULT, "ihip_softmax_stats: NULL pointer");
    if (rows < 1 || V < 1 || !(T > 0.f)) return fail(IHIP_EINVAL, "ihip_softmax_stats: rows=%d V=%d T=%g", rows, V, T);
    int rc = need_ws("ihip_softmax_stats", rows, V, ws, ws_bytes);
    if (rc != IHIP_OK) return rc;
    hipError_t e = launch_stats(logits_dev, rows, V, T, T, 0, ws, S(stream));
    if (e == hipSuccess) e = launch_stats_merge(ws, rows, V, zmax_dev, zsum_dev, S(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_softmax_stats");
}

int ihip_spec_accept_ws_bytes(int steps, int k, int V, size_t *bytes) {
    if (!bytes) return fail(IHIP_EFAULT, "ihip_spec_accept_ws_bytes: NULL");
    if (steps < 1 || k < 0 || V < 1) return fail(IHIP_EINVAL, "ihip_spec_accept_ws_bytes: steps=%d k=%d V=%d", steps, k, V);
    if (V > 1024 * 4096) return fail(IHIP_EINVAL, "ihip_spec_accept_ws_bytes: V=%d above 4194304", V);
    *bytes = spec_accept_ws(steps, k, V);
    return ok();
}

// The bonus draw of a verify step goes through softmax_sample's filters
// (src/SpeculativeDecoding.jl:100-104) when one of them keeps less than the
// whole vocabulary.
static bool bonus_filtered(int V, int top_k, float top_p, float min_p) {
    return (top_k > 0 && top_k < V) || top_p < 1.0f || min_p > 0.f;
}

static size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

// Workspace of a filtered accept: the accept's own, then the steps' bonus
// rows gathered contiguously (steps > 1), the sampler's workspace over them,
// and the drawn bonus tokens.
static size_t spec_accept_ex_ws(int steps, int k, int V, bool filtered) {
    if (!filtered) return spec_accept_ws(steps, k, V);
    size_t b = round256(spec_accept_ws(steps, k, V));
    if (steps > 1) b += round256((size_t)steps * V * sizeof(float));
    return b + round256(sample_spread_ws(steps, V)) + round256((size_t)steps * sizeof(int32_t));
}

int ihip_spec_accept_ex_ws_bytes(int steps, int k, int V, int top_k, float top_p, float min_p, size_t *bytes) {
    if (!bytes) return fail(IHIP_EFAULT, "ihip_spec_accept_ex_ws_bytes: NULL");
    if (steps < 1 || k < 0 || V < 1 || top_k < 0)
        return fail(IHIP_EINVAL, "ihip_spec_accept_ex_ws_bytes: steps=%d k=%d V=%d top_k=%d", steps, k, V, top_k);
    if (V > 1024 * 4096) return fail(IHIP_EINVAL, "ihip_spec_accept_ex_ws_bytes: V=%d above 4194304", V);
    *bytes = spec_accept_ex_ws(steps, k, V, bonus_filtered(V, top_k, top_p, min_p));
    return ok();
}

static int spec_accept_impl(const char *name, const float *tgt_dev, const float *drf_dev,
                            const int32_t *draft_tok_dev, int steps, int k, int V, float T, int top_k, float top_p,
                            float min_p, const float *u_acc_dev, const float *u_res_dev, const float *u_bonus_dev,
                            int mode, int32_t *out_tok_dev, int32_t *out_n_dev, void *ws, size_t ws_bytes,
                            size_t need, bool filtered, void *stream) {
    if (!tgt_dev || !u_res_dev || !u_bonus_dev || !out_tok_dev || !out_n_dev)
        return fail(IHIP_EFAULT, "%s: NULL pointer", name);
    if (k > 0 && (!drf_dev || !draft_tok_dev || !u_acc_dev)) return fail(IHIP_EFAULT, "%s: NULL pointer", name);
    if (steps < 1 || k < 0 || V < 1) return fail(IHIP_EINVAL, "%s: steps=%d k=%d V=%d", name, steps, k, V);
    if (!(T > 0.f)) return fail(IHIP_EINVAL, "%s: T=%g must be > 0 (greedy: ihip_greedy_verify)", name, T);
    if (mode != 0 && mode != 1) return fail(IHIP_EINVAL, "%s: mode=%d", name, mode);
    if (V > 1024 * 4096) return fail(IHIP_EINVAL, "%s: V=%d above 4194304", name, V);
    if (k > 127) return fail(IHIP_EINVAL, "%s: k=%d above 127", name, k);
    if (top_k < 0 || top_p != top_p || min_p != min_p)
        return fail(IHIP_EINVAL, "%s: top_k=%d top_p=%g min_p=%g", name, top_k, top_p, min_p);
    if (!ws) return fail(IHIP_EFAULT, "%s: NULL workspace", name);
    if (ws_bytes < need) return fail(IHIP_ENOMEM, "%s: workspace %zu < %zu bytes", name, ws_bytes, need);
    if (((uintptr_t)ws & 15) != 0) return fail(IHIP_EINVAL, "%s: workspace must be 16-byte aligned", name);
    const int32_t *bonus = nullptr;
    hipError_t e = hipSuccess;
    if (filtered) {
        const int kk = top_k >= V ? 0 : top_k;
        uint8_t *w = (uint8_t *)ws + round256(spec_accept_ws(steps, k, V));
        const float *rows = tgt_dev + (size_t)k * V;  // step 0's bonus row; steps apart by (k + 1) V
        if (steps > 1) {
            float *g = (float *)w;
            w += round256((size_t)steps * V * sizeof(float));
            e = hipMemcpy2DAsync(g, (size_t)V * sizeof(float), rows, (size_t)(k + 1) * V * sizeof(float),
                                 (size_t)V * sizeof(float), steps, hipMemcpyDeviceToDevice, S(stream));
            rows = g;
        }
        void *sws = w;
        int32_t *btok = (int32_t *)(w + round256(sample_spread_ws(steps, V)));
        if (e == hipSuccess)
            e = launch_sample_spread(rows, steps, V, T, kk, top_p, min_p, u_bonus_dev, btok, sws, S(stream));
        bonus = btok;
    }
    if (e == hipSuccess)
        e = launch_spec_accept(tgt_dev, drf_dev, draft_tok_dev, steps, k, V, T, u_acc_dev, u_res_dev, u_bonus_dev,
                               mode, bonus, out_tok_dev, out_n_dev, ws, S(stream));
    return e == hipSuccess ? ok() : hip_fail(e, name);
}

int ihip_spec_accept(const float *tgt_dev, const float *drf_dev, const int32_t *draft_tok_dev, int steps, int k,
                     int V, float T, const float *u_acc_dev, const float *u_res_dev, const float *u_bonus_dev,
                     int mode, int32_t *out_tok_dev, int32_t *out_n_dev, void *ws, size_t ws_bytes, void *stream) {
    const size_t need = steps >= 1 && k >= 0 && V >= 1 ? spec_accept_ws(steps, k, V) : 0;
    return spec_accept_impl("ihip_spec_accept", tgt_dev, drf_dev, draft_tok_dev, steps, k, V, T, 0, 1.0f, 0.f,
                            u_acc_dev, u_res_dev, u_bonus_dev, mode, out_tok_dev, out_n_dev, ws, ws_bytes, need,
                            false, stream);
}

int ihip_spec_accept_ex(const float *tgt_dev, const float *drf_dev, const int32_t *draft_tok_dev, int steps, int k,
                        int V, float T, int top_k, float top_p, float min_p, const float *u_acc_dev,
                        const float *u_res_dev, const float *u_bonus_dev, int mode, int32_t *out_tok_dev,
                        int32_t *out_n_dev, void *ws, size_t ws_bytes, void *stream) {
    const bool filtered = V >= 1 && bonus_filtered(V, top_k, top_p, min_p);
    const size_t need = steps >= 1 && k >= 0 && V >= 1 ? spec_accept_ex_ws(steps, k, V, filtered) : 0;
    return spec_accept_impl("ihip_spec_accept_ex", tgt_dev, drf_dev, draft_tok_dev, steps, k, V, T, top_k, top_p,
                            min_p, u_acc_dev, u_res_dev, u_bonus_dev, mode, out_tok_dev, out_n_dev, ws, ws_bytes,
                            need, filtered, stream);
}

int ihip_greedy_verify(const float *logits_dev, const int32_t *draft_tok_dev, int steps, int k, int V,
                       int32_t *out_n_dev, int32_t *out_argmax_dev, void *ws, size_t ws_bytes, void *stream) {
    if (!logits_dev || !out_n_dev || (k > 0 && !draft_tok_dev)) return fail(IHIP_EFAULT, "ihip_greedy_verify: NULL pointer");
    if (steps < 1 || k < 0 || V < 1) return fail(IHIP_EINVAL, "ihip_greedy_verify: steps=%d k=%d V=%d", steps, k, V);
    int rc = need_ws("ihip_greedy_verify", steps * (k + 1), V, ws, ws_bytes);
    if (rc != IHIP_OK) return rc;
    float2 *part = (float2 *)ws;
    hipError_t e = launch_argmax_partial(logits_dev, steps * (k + 1), V, part, S(stream));
    if (e == hipSuccess) e = launch_greedy(part, V, draft_tok_dev, steps, k, out_n_dev, out_argmax_dev, S(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_greedy_verify");
}

int ihip_tree_accept(const float *tgt_dev, const float *drf_dev, const int32_t *tok_dev, const int32_t *parent_dev,
                     int n, int V, float T, const float *u_dev, int32_t *out_path_dev, int32_t *out_len_dev,
                     void *ws, size_t ws_bytes, void *stream) {
    if (!tgt_dev || !drf_dev || !tok_dev || !parent_dev || !u_dev || !out_path_dev || !out_len_dev)
        return fail(IHIP_EFAULT, "ihip_tree_accept: NULL pointer");
    if (n < 1 || V < 1 || !(T > 0.f)) return fail(IHIP_EINVAL, "ihip_tree_accept: n=%d V=%d T=%g", n, V, T);
    int rc = need_ws("ihip_tree_accept", 3 * n, V, ws, ws_bytes);
    if (rc != IHIP_OK) return rc;
    if (ws_bytes < tree_ws(n, V))  // (ihip_accept_ws_bytes(3 n, V) covers it)
        return fail(IHIP_ENOMEM, "ihip_tree_accept: workspace %zu < %zu bytes", ws_bytes, tree_ws(n, V));
    hipError_t e = launch_tree(tgt_dev, drf_dev, tok_dev, parent_dev, n, V, T, u_dev, ws, out_path_dev,
                               out_len_dev, S(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_tree_accept");
}

int ihip_spec_commit_state(void *state_dev, const void *snap_dev, size_t bytes, int64_t snap_stride_bytes, int k,
                           const int32_t *n_accepted_dev, int steps, int64_t state_step_bytes,
                           int64_t snap_step_bytes, void *stream) {
    if (!state_dev || !snap_dev || !n_accepted_dev) return fail(IHIP_EFAULT, "ihip_spec_commit_state: NULL pointer");
    if (k < 0 || steps < 1 || bytes == 0 || (bytes & 3) || (snap_stride_bytes & 3) || (state_step_bytes & 3) ||
        (snap_step_bytes & 3) || ((uintptr_t)state_dev & 3) || ((uintptr_t)snap_dev & 3))
        return fail(IHIP_EINVAL, "ihip_spec_commit_state: sizes, strides and pointers must be multiples of 4 bytes "
                                 "(k=%d steps=%d)", k, steps);
    if ((k > 0 && snap_stride_bytes < (int64_t)bytes) || (steps > 1 && state_step_bytes < (int64_t)bytes) ||
        (steps > 1 && snap_step_bytes < (int64_t)(k + 1) * snap_stride_bytes))
        return fail(IHIP_EINVAL, "ihip_spec_commit_state: overlapping strides");
    hipError_t e = launch_commit_state(state_dev, snap_dev, (int64_t)(bytes / 4), snap_stride_bytes / 4, k,
                                       n_accepted_dev, steps, state_step_bytes / 4, snap_step_bytes / 4, S(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_spec_commit_state");
}

int ihip_spec_advance_len(int32_t *len_dev, const int32_t *n_accepted_dev, int steps, void *stream) {
    if (!len_dev || !n_accepted_dev) return fail(IHIP_EFAULT, "ihip_spec_advance_len: NULL pointer");
    if (steps < 1) return fail(IHIP_EINVAL, "ihip_spec_advance_len: steps=%d", steps);
    hipError_t e = launch_advance_len(len_dev, n_accepted_dev, steps, S(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_spec_advance_len");
}

int ihip_sample(const float *logits_dev, int rows, int V, float T, int top_k, float top_p, float min_p,
                const float *u_dev, int32_t *out_tok_dev, void *stream) {
    if (!logits_dev || !u_dev || !out_tok_dev) return fail(IHIP_EFAULT, "ihip_sample: NULL pointer");
    if (rows < 1 || V < 1 || V > sample_max_v())
        return fail(IHIP_EINVAL, "ihip_sample: rows=%d V=%d (V in [1, %d])", rows, V, sample_max_v());
    if (!(T >= 0.f) || T > 3.0e38f) return fail(IHIP_EINVAL, "ihip_sample: temperature %g", T);
    if (top_k < 0) return fail(IHIP_EINVAL, "ihip_sample: top_k=%d", top_k);
    if (top_k >= V) top_k = 0;  // keeps every token (sorted_indices[1:min(top_k, V)])
    if (top_p != top_p || min_p != min_p) return fail(IHIP_EINVAL, "ihip_sample: NaN top_p/min_p");
    hipError_t e = launch_sample(logits_dev, rows, V, T, top_k, top_p, min_p, u_dev, out_tok_dev, S(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_sample");
}

int ihip_sample_ws_bytes(int rows, int V, size_t *bytes) {
    if (!bytes) return fail(IHIP_EFAULT, "ihip_sample_ws_bytes: NULL pointer");
    if (rows < 1 || V < 1 || V > sample_max_v())
        return fail(IHIP_EINVAL, "ihip_sample_ws_bytes: rows=%d V=%d", rows, V);
    *bytes = sample_spread_ws(rows, V);
    return ok();
}

int ihip_sample_ex(const float *logits_dev, int rows, int V, float T, int top_k, float top_p, float min_p,
                   const float *u_dev, int32_t *out_tok_dev, void *ws, size_t ws_bytes, void *stream) {
    if (!logits_dev || !u_dev || !out_tok_dev || !ws) return fail(IHIP_EFAULT, "ihip_sample_ex: NULL pointer");
    if (rows < 1 || V < 1 || V > sample_max_v())
        return fail(IHIP_EINVAL, "ihip_sample_ex: rows=%d V=%d (V in [1, %d])", rows, V, sample_max_v());
    if (!aligned16(ws)) return fail(IHIP_EINVAL, "ihip_sample_ex: workspace must be 16-byte aligned");
    if (ws_bytes < sample_spread_ws(rows, V))
        return fail(IHIP_ENOMEM, "ihip_sample_ex: workspace %zu < %zu bytes", ws_bytes, sample_spread_ws(rows, V));
    if (!(T >= 0.f) || T > 3.0e38f) return fail(IHIP_EINVAL, "ihip_sample_ex: temperature %g", T);
    if (top_k < 0) return fail(IHIP_EINVAL, "ihip_sample_ex: top_k=%d", top_k);
    if (top_k >= V) top_k = 0;
    if (top_p != top_p || min_p != min_p) return fail(IHIP_EINVAL, "ihip_sample_ex: NaN top_p/min_p");
    hipError_t e = launch_sample_spread(logits_dev, rows, V, T, top_k, top_p, min_p, u_dev, out_tok_dev, ws,
                                        S(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_sample_ex");
}

int ihip_apply_penalties(float *logits_dev, int rows, int V, const int32_t *tok_dev, int n_tok, int64_t tok_stride,
                         float presence, float repetition, void *stream) {
    if (!logits_dev || (n_tok > 0 && !tok_dev)) return fail(IHIP_EFAULT, "ihip_apply_penalties: NULL pointer");
    if (rows < 1 || V < 1 || n_tok < 0 || (tok_stride != 0 && tok_stride < n_tok))
        return fail(IHIP_EINVAL, "ihip_apply_penalties: rows=%d V=%d n_tok=%d stride=%lld", rows, V, n_tok,
                    (long long)tok_stride);
    if (presence != presence || repetition != repetition)
        return fail(IHIP_EINVAL, "ihip_apply_penalties: NaN penalty");
    hipError_t e = launch_penalties(logits_dev, rows, V, tok_dev, n_tok, tok_stride, presence, repetition, S(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_apply_penalties");
}

int ihip_synth_blocks(int qtype, uint64_t stream, int64_t first_block, int64_t n_blocks, void *out_dev,
                      void *stream_handle) {
    if (!out_dev) return fail(IHIP_EFAULT, "ihip_synth_blocks: NULL pointer");
    if (!is_qtype(qtype) || n_blocks < 0 || first_block < 0)
        return fail(IHIP_EINVAL, "ihip_synth_blocks: qtype=%d n_blocks=%lld", qtype, (long long)n_blocks);
    hipError_t e = launch_synth(qtype, stream, first_block, n_blocks, out_dev, S(stream_handle));
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_synth_blocks");
}

int ihip_synth_gaussian(uint64_t stream, int64_t n, float scale, const float *add_dev, float *out_dev,
                        void *stream_handle) {
    if (!out_dev) return fail(IHIP_EFAULT, "ihip_synth_gaussian: NULL pointer");
    if (n < 0) return fail(IHIP_EINVAL, "ihip_synth_gaussian: n=%lld", (long long)n);
    hipError_t e = launch_gaussian(stream, n, scale, add_dev, out_dev, S(stream_handle));
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_synth_gaussian");
}

int ihip_stream_read(const void *src_dev, size_t bytes, uint32_t *out_dev, void *stream) {
    if (!src_dev || !out_dev) return fail(IHIP_EFAULT, "ihip_stream_read: NULL pointer");
    if (!aligned16(src_dev) || (bytes & 15))
        return fail(IHIP_EINVAL, "ihip_stream_read: src must be 16-byte aligned and bytes a multiple of 16");
    hipError_t e = launch_stream_read(src_dev, (int64_t)bytes, out_dev, S(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "ihip_stream_read");
}

}  // extern "C"
