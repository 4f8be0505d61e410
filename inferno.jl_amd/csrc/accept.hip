// LM-head softmax statistics and speculative acceptance on gfx950.
//
// Softmax statistics are two-level: a grid of (V-chunk, row) workgroups
// writes a partial (max, sum exp(z - max)) per chunk; consumers merge the
// partials in chunk order (deterministic). z = L / T as the reference
// computes logits ./ temperature (src/ModelCPU.jl:1130-1132).
//
// Acceptance (src/SpeculativeDecoding.jl:75-104 with explicit uniforms):
// one workgroup per verify step merges the statistics of its rows, runs the
// ratio tests, and draws the residual or bonus token with an inverse CDF
// over V: per-thread contiguous slices, a block scan of the slice sums, and
// a sequential scan inside the one slice that holds u*S.
#include "common.h"

namespace {

constexpr int CHUNK = 4096;      // V elements per partial
constexpr int NT = 256;          // threads per workgroup

__device__ __forceinline__ void merge_ms(float &m, float &s, float m2, float s2) {
    if (m2 == -__builtin_huge_valf()) return;
    if (m == -__builtin_huge_valf()) { m = m2; s = s2; return; }
    const float M = fmaxf(m, m2);
    s = s * __expf(m - M) + s2 * __expf(m2 - M);
    m = M;
}

// Block-wide (max, sum) merge of per-thread pairs.
__device__ void block_merge_ms(float &m, float &s, float *sh) {
    // wave level
    for (int o = 32; o > 0; o >>= 1) {
        const float m2 = __shfl_xor(m, o), s2 = __shfl_xor(s, o);
        merge_ms(m, s, m2, s2);
    }
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    if (l == 0) { sh[2 * w] = m; sh[2 * w + 1] = s; }
    __syncthreads();
    if (threadIdx.x == 0) {
        float M = sh[0], S = sh[1];
        for (int i = 1; i < (int)(blockDim.x >> 6); i++) merge_ms(M, S, sh[2 * i], sh[2 * i + 1]);
        sh[0] = M;
        sh[1] = S;
    }
    __syncthreads();
    m = sh[0];
    s = sh[1];
    __syncthreads();
}

// partial[row][chunk] = (max z, sum exp(z - max)). Row r uses T_last when period > 0 and r % period == period - 1 (the bonus
// row of a verify step), T otherwise.
__global__ __launch_bounds__(NT) void stats_partial_kernel(const float *__restrict__ L, int V, int nchunk,
                                                           float T, float T_last, int period,
                                                           float2 *__restrict__ part) {
    __shared__ float sh[2 * NT / 64];
    const int chunk = blockIdx.x, row = blockIdx.y;
    const float Tr = (period > 0 && row % period == period - 1) ? T_last : T;
    const float *src = L + (size_t)row * V;
    const int j0 = chunk * CHUNK, j1 = min(V, j0 + CHUNK);
    float m = -__builtin_huge_valf();
    for (int j = j0 + threadIdx.x; j < j1; j += NT) m = fmaxf(m, src[j] / Tr);
    float s = 0.f;
    for (int j = j0 + threadIdx.x; j < j1; j += NT) s += __expf(src[j] / Tr - m);
    block_merge_ms(m, s, sh);
    if (threadIdx.x == 0) part[(size_t)row * nchunk + chunk] = make_float2(m, s);
}

__device__ __forceinline__ float2 merge_row(const float2 *part, int nchunk) {
    float m = -__builtin_huge_valf(), s = 0.f;
    for (int c = 0; c < nchunk; c++) merge_ms(m, s, part[c].x, part[c].y);
    return make_float2(m, s);
}

__global__ void stats_merge_kernel(const float2 *__restrict__ part, int rows, int nchunk,
                                   float *__restrict__ zmax, float *__restrict__ zsum) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const float2 ms = merge_row(part + (size_t)r * nchunk, nchunk);
    zmax[r] = ms.x;
    zsum[r] = ms.y;
}

// Weight of entry j of the sampling distribution:
//   kind 0: p_j (row lt at T)                       bonus / fallback draw
//   kind 1: max(0, p_j - q_j)  (q from row ld)      standard residual
//   kind 2: max(0, p_j - qs)   (qs scalar)          reference residual
struct Dist {
    const float *lt, *ld;
    float Tp, mp, sp, Tq, mq, sq, qs;
    int kind;
    __device__ __forceinline__ float w(int j) const {
        const float p = __expf(lt[j] / Tp - mp) / sp;
        if (kind == 0) return p;
        const float q = kind == 1 ? __expf(ld[j] / Tq - mq) / sq : qs;
        return fmaxf(p - q, 0.f);
    }
};

// First j with u*S <= C_j (C inclusive prefix of w), or V-1. Also returns S.
__device__ int block_inv_cdf(const Dist &D, int V, float u, float *sh, float &S_out) {
    const int t = threadIdx.x;
    const int per = (V + NT - 1) / NT;
    const int j0 = min(V, t * per), j1 = min(V, j0 + per);
    float loc = 0.f;
    for (int j = j0; j < j1; j++) loc += D.w(j);
    // inclusive block scan of loc over threads (Hillis-Steele in LDS)
    sh[t] = loc;
    __syncthreads();
    for (int o = 1; o < NT; o <<= 1) {
        const float v = t >= o ? sh[t - o] : 0.f;
        __syncthreads();
        sh[t] += v;
        __syncthreads();
    }
    const float S = sh[NT - 1];
    const float before = t > 0 ? sh[t - 1] : 0.f;
    const float target = u * S;
    __shared__ int found;
    if (t == 0) found = V - 1;
    __syncthreads();
    // the first thread whose inclusive range reaches target scans its slice
    const bool mine = (target <= sh[t]) && (t == 0 || target > before) && j1 > j0;
    if (mine) {
        float c = before;
        int res = j1 - 1;
        for (int j = j0; j < j1; j++) {
            c += D.w(j);
            if (target <= c) { res = j; break; }
        }
        atomicMin(&found, res);
    }
    __syncthreads();
    S_out = S;
    const int r = found;
    __syncthreads();
    return r;
}

// One workgroup per verify step.
__global__ __launch_bounds__(NT) void spec_accept_kernel(
    const float *__restrict__ tgt, const float *__restrict__ drf, const int32_t *__restrict__ draft_tok,
    int k, int V, float T, const float *__restrict__ u_acc, const float *__restrict__ u_res,
    const float *__restrict__ u_bonus, int mode, const float2 *__restrict__ part, int nchunk,
    int32_t *__restrict__ out_tok, int32_t *__restrict__ out_n) {
    __shared__ float sh[NT];
    __shared__ int s_n, s_rej;
    __shared__ float s_qs;
    const int step = blockIdx.x;
    const float *Lt = tgt + (size_t)step * (k + 1) * V;
    const float *Ld = drf + (size_t)step * k * V;
    const int32_t *dt = draft_tok + (size_t)step * k;
    // partials: target rows [steps*(k+1)][nchunk], then draft rows [steps*k][nchunk]
    const float2 *Pt = part + (size_t)step * (k + 1) * nchunk;
    const float2 *Pd = part + ((size_t)gridDim.x * (k + 1) + (size_t)step * k) * nchunk;
    const float Tr = mode == 0 ? T : 1.0f;
    if (threadIdx.x == 0) {
        int n = 0, rej = -1;
        float qs = 0.f;
        for (int i = 0; i < k; i++) {
            const float2 pt = merge_row(Pt + (size_t)i * nchunk, nchunk);
            const float2 pd = merge_row(Pd + (size_t)i * nchunk, nchunk);
            const int x = dt[i];
            if (x < 0 || x >= V) {  // invalid draft id: reported as out_n = -1
                n = -1;
                break;
            }
            const float p = __expf(Lt[(size_t)i * V + x] / Tr - pt.x) / pt.y;
            const float q = __expf(Ld[(size_t)i * V + x] / Tr - pd.x) / pd.y;
            const float ratio = q > 0.f ? fminf(1.0f, p / q) : 1.0f;
            if (u_acc[(size_t)step * k + i] < ratio) {
                out_tok[(size_t)step * (k + 1) + n] = x;
                n++;
            } else {
                rej = i;
                qs = q;
                break;
            }
        }
        s_n = n;
        s_rej = rej;
        s_qs = qs;
    }
    __syncthreads();
    const int n = s_n, rej = s_rej;
    if (n < 0) {
        if (threadIdx.x == 0) out_n[step] = -1;
        return;
    }
    Dist D;
    int tok;
    float S;
    if (rej >= 0) {
        const float2 pt = merge_row(Pt + (size_t)rej * nchunk, nchunk);
        const float2 pd = merge_row(Pd + (size_t)rej * nchunk, nchunk);
        D.lt = Lt + (size_t)rej * V;
        D.ld = Ld + (size_t)rej * V;
        D.Tp = Tr; D.mp = pt.x; D.sp = pt.y;
        D.Tq = Tr; D.mq = pd.x; D.sq = pd.y;
        D.qs = s_qs;
        D.kind = mode == 0 ? 1 : 2;
        const float u = u_res[step];
        tok = block_inv_cdf(D, V, u, sh, S);
        if (!(S > 0.f)) {
            if (mode == 0) {  // p == q: sample from p
                D.kind = 0;
                tok = block_inv_cdf(D, V, u, sh, S);
            } else {
                tok = V - 1;  // all-NaN residual in the reference returns length(probs)
            }
        }
    } else {
        const float2 pt = merge_row(Pt + (size_t)k * nchunk, nchunk);
        D.lt = Lt + (size_t)k * V;
        D.ld = nullptr;
        D.Tp = T; D.mp = pt.x; D.sp = pt.y;
        D.Tq = T; D.mq = 0.f; D.sq = 1.f; D.qs = 0.f;
        D.kind = 0;
        tok = block_inv_cdf(D, V, u_bonus[step], sh, S);
    }
    if (threadIdx.x == 0) {
        out_tok[(size_t)step * (k + 1) + n] = tok;
        out_n[step] = n;
    }
}

// Partial first-index argmax per (chunk, row).
__global__ __launch_bounds__(NT) void argmax_partial_kernel(const float *__restrict__ L, int V, int nchunk,
                                                            float2 *__restrict__ part) {
    __shared__ float sv[NT / 64];
    __shared__ int si[NT / 64];
    const int chunk = blockIdx.x, row = blockIdx.y;
    const float *src = L + (size_t)row * V;
    const int j0 = chunk * CHUNK, j1 = min(V, j0 + CHUNK);
    float bv = -__builtin_huge_valf();
    int bi = 0x7fffffff;
    for (int j = j0 + threadIdx.x; j < j1; j += NT) {
        const float v = src[j];
        if (v > bv) { bv = v; bi = j; }  // strided: first j per thread wins ties
    }
    for (int o = 32; o > 0; o >>= 1) {
        const float v2 = __shfl_xor(bv, o);
        const int i2 = __shfl_xor(bi, o);
        if (v2 > bv || (v2 == bv && i2 < bi)) { bv = v2; bi = i2; }
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { sv[w] = bv; si[w] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < NT / 64; i++)
            if (sv[i] > bv || (sv[i] == bv && si[i] < bi)) { bv = sv[i]; bi = si[i]; }
        part[(size_t)row * nchunk + chunk] = make_float2(bv, __int_as_float(bi));
    }
}

__global__ void greedy_kernel(const float2 *__restrict__ part, int nchunk, const int32_t *__restrict__ draft_tok,
                              int steps, int k, int32_t *__restrict__ out_n, int32_t *__restrict__ out_argmax) {
    const int step = blockIdx.x * blockDim.x + threadIdx.x;
    if (step >= steps) return;
    int n = 0;
    bool go = true;
    for (int i = 0; i <= k; i++) {
        const float2 *p = part + ((size_t)step * (k + 1) + i) * nchunk;
        float bv = p[0].x;
        int bi = __float_as_int(p[0].y);
        for (int c = 1; c < nchunk; c++)
            if (p[c].x > bv) { bv = p[c].x; bi = __float_as_int(p[c].y); }  // chunks ascend: strict > keeps first
        if (out_argmax) out_argmax[(size_t)step * (k + 1) + i] = bi;
        if (i < k && go) {
            if (bi == draft_tok[(size_t)step * k + i]) n++;
            else go = false;
        }
    }
    out_n[step] = n;
}

// Tree walk: one thread, nodes in index order (parent[i] < i).
__global__ void tree_kernel(const float *__restrict__ tgt, const float *__restrict__ drf,
                            const int32_t *__restrict__ tok, const int32_t *__restrict__ parent, int n, int V,
                            float T, const float *__restrict__ u, const float2 *__restrict__ part, int nchunk,
                            int32_t *__restrict__ out_path, int32_t *__restrict__ out_len, int32_t *__restrict__ wsi) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    int32_t *acc = wsi, *depth = wsi + n;
    acc[0] = 1;
    depth[0] = 0;
    int best = 0;
    for (int i = 1; i < n; i++) {
        const int p = parent[i];
        const int x = tok[i];
        acc[i] = 0;
        if (p < 0 || p >= i || x < 0 || x >= V) {  // malformed node: reported as out_len = -1
            *out_len = -1;
            return;
        }
        depth[i] = depth[p] + 1;
        if (!acc[p]) continue;
        const float2 pt = merge_row(part + (size_t)p * nchunk, nchunk);
        const float2 pd = merge_row(part + (size_t)(n + p) * nchunk, nchunk);
        const float pp = __expf(tgt[(size_t)p * V + x] / T - pt.x) / pt.y;
        const float qq = __expf(drf[(size_t)p * V + x] / T - pd.x) / pd.y;
        const float ratio = qq > 0.f ? fminf(1.0f, pp / qq) : 1.0f;
        if (u[i] < ratio) {
            acc[i] = 1;
            if (depth[i] > depth[best]) best = i;
        }
    }
    const int len = depth[best] + 1;
    int v = best;
    for (int d = len - 1; d >= 0; d--) {
        out_path[d] = v;
        v = d > 0 ? parent[v] : 0;
    }
    *out_len = len;
}

}  // namespace

int accept_nchunk(int V) { return (V + CHUNK - 1) / CHUNK; }

hipError_t launch_stats(const float *L, int rows, int V, float T, float T_last, int period, float2 *part,
                        hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    const int nc = accept_nchunk(V);
    stats_partial_kernel<<<dim3(nc, rows), NT, 0, st>>>(L, V, nc, T, T_last, period, part);
    return hipGetLastError();
}

hipError_t launch_stats_merge(const float2 *part, int rows, int V, float *zmax, float *zsum, hipStream_t st) {
    const int nc = accept_nchunk(V);
    stats_merge_kernel<<<(rows + 63) / 64, 64, 0, st>>>(part, rows, nc, zmax, zsum);
    return hipGetLastError();
}

// part: float2 [steps*(k+1) + steps*k][nchunk].
hipError_t launch_spec_accept(const float *tgt, const float *drf, const int32_t *draft_tok, int steps, int k,
                              int V, float T, const float *u_acc, const float *u_res, const float *u_bonus,
                              int mode, int32_t *out_tok, int32_t *out_n, float2 *part, hipStream_t st) {
    const int nc = accept_nchunk(V);
    const float Tr = mode == 0 ? T : 1.0f;
    hipError_t e = launch_stats(tgt, steps * (k + 1), V, Tr, T, k + 1, part, st);
    if (e != hipSuccess) return e;
    e = launch_stats(drf, steps * k, V, Tr, Tr, 0, part + (size_t)steps * (k + 1) * nc, st);
    if (e != hipSuccess) return e;
    spec_accept_kernel<<<steps, NT, 0, st>>>(tgt, drf, draft_tok, k, V, T, u_acc, u_res, u_bonus, mode, part, nc,
                                             out_tok, out_n);
    return hipGetLastError();
}

hipError_t launch_argmax_partial(const float *L, int rows, int V, float2 *part, hipStream_t st) {
    const int nc = accept_nchunk(V);
    argmax_partial_kernel<<<dim3(nc, rows), NT, 0, st>>>(L, V, nc, part);
    return hipGetLastError();
}

hipError_t launch_greedy(const float2 *part, int V, const int32_t *draft_tok, int steps, int k, int32_t *out_n,
                         int32_t *out_argmax, hipStream_t st) {
    const int nc = accept_nchunk(V);
    greedy_kernel<<<(steps + 63) / 64, 64, 0, st>>>(part, nc, draft_tok, steps, k, out_n, out_argmax);
    return hipGetLastError();
}

// part: float2 [2n][nchunk] (target rows then draft rows); wsi: int32 [2n].
hipError_t launch_tree(const float *tgt, const float *drf, const int32_t *tok, const int32_t *parent, int n, int V,
                       float T, const float *u, float2 *part, int32_t *out_path, int32_t *out_len,
                       int32_t *wsi, hipStream_t st) {
    const int nc = accept_nchunk(V);
    hipError_t e = launch_stats(tgt, n, V, T, T, 0, part, st);
    if (e != hipSuccess) return e;
    e = launch_stats(drf, n, V, T, T, 0, part + (size_t)n * nc, st);
    if (e != hipSuccess) return e;
    tree_kernel<<<1, 64, 0, st>>>(tgt, drf, tok, parent, n, V, T, u, part, nc, out_path, out_len, wsi);
    return hipGetLastError();
}
