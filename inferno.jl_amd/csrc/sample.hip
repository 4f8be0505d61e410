// Draft-side sampler on gfx950: softmax_sample (src/ModelCPU.jl:1123-1200)
// with temperature, top-k, top-p and min-p, and the presence / repetition
// penalties the generation loop applies to the logits first
// (apply_presence_penalty!, apply_repetition_penalty!,
// src/ModelCPU.jl:1202-1225).
//
// One workgroup of 1024 threads per row. Every pass over a row reads it in
// rounds of 4096 logits (one float4 per thread, coalesced), so after the
// first pass the row (600 KB at V = 151936) is served from L2.
//
//  * T = 0: Julia's argmax (the first NaN above every number, +0.0 above
//    -0.0, the first of equals) by an integer key.
//  * top-k (1 <= k <= 4096, k < V): exact radix select of the k-th largest
//    z = L / T (8 bits a pass on an order-preserving key), ties at the
//    threshold kept lowest index first (the stable descending sortperm);
//    the k candidates are compacted into LDS in index order, and softmax,
//    top-p (a bitonic sort by probability, then a scan), min-p and the draw
//    run there.
//  * no top-k: softmax statistics by full passes; top-p finds the nucleus by
//    a radix select over the same keys whose buckets carry the probability
//    mass in 2^-40 fixed point (integer LDS atomics: deterministic); min-p
//    is a threshold; the draw sums each round, picks the round, then scans
//    it, the rounds' sums taken from per-wave parts kept by the pass before
//    it (statistics, nucleus mass or min-p mass) where V <= 262144.
//  * the threshold's refinement passes run over the first pass's bucket
//    gathered into LDS when it holds at most 4096 elements.
//  * with a workspace, every setting spreads each row over workgroups of
//    one round (chunk statistics, each chunk's argmax, top-k candidates,
//    threshold histograms, kept sums or kept entries), and one workgroup
//    per row finishes each stage from them.
// Sums and scans are trees, where the reference accumulates sequentially:
// the drawn token can differ only where u falls within rounding of a CDF
// step.
#include "common.h"

#include <climits>

namespace {

constexpr int SNT = 1024;
constexpr int SNW = SNT / 64;
constexpr int SROUND = 4 * SNT;
constexpr int SK_MAX = 4096;
constexpr int SMAX_ROUNDS = 1024;  // V <= 4194304
constexpr int SPART_ROUNDS = 64;   // plain draws by per-wave parts: V <= 262144

struct SampleArgs {
    float T;       // 0: argmax
    int top_k;     // 0: off (the host maps k >= V to 0)
    float top_p;   // >= 1: off
    float min_p;   // <= 0: off
};

// Order-preserving 32-bit key of a float (larger float, larger key).
__device__ __forceinline__ uint32_t okey(float z) {
    const uint32_t b = __float_as_uint(z);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float okey_inv(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// ---- block primitives (16 waves), fixed reduction trees
__device__ __forceinline__ float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ int wave_min_i(int v) {
    for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o));
    return v;
}
__device__ float block_sum(float v, float *red) {
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    v = wave_sum(v);
    __syncthreads();  // (red may still be read by the previous call)
    if (l == 0) red[w] = v;
    __syncthreads();
    return wave_sum(l < SNW ? red[l] : 0.f);
}
__device__ float block_max(float v, float *red) {
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    v = wave_max(v);
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    return wave_max(l < SNW ? red[l] : -__builtin_huge_valf());
}
__device__ int block_min_i(int v, int *red) {
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    v = wave_min_i(v);
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    return wave_min_i(l < SNW ? red[l] : INT_MAX);
}
// exclusive scan over the block in thread order; *total = block sum
__device__ uint32_t block_excl_scan_u(uint32_t v, uint32_t *red, uint32_t &total) {
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    uint32_t inc = v;
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(inc, o);
        if (l >= o) inc += y;
    }
    __syncthreads();
    if (l == 63) red[w] = inc;
    __syncthreads();
    uint32_t base = 0, tot = 0;
    for (int i = 0; i < SNW; i++) {
        const uint32_t x = red[i];
        base += i < w ? x : 0u;
        tot += x;
    }
    total = tot;
    return base + inc - v;
}
__device__ float block_excl_scan_f(float v, float *red, float &total) {
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    float inc = v;
    for (int o = 1; o < 64; o <<= 1) {
        const float y = __shfl_up(inc, o);
        if (l >= o) inc += y;
    }
    __syncthreads();
    if (l == 63) red[w] = inc;
    __syncthreads();
    float base = 0.f, tot = 0.f;
    for (int i = 0; i < SNW; i++) {
        const float x = red[i];
        if (i < w) base += x;
        tot += x;
    }
    total = tot;
    return base + (inc - v);
}

// Round r of a row: this thread's 4 logits z = L * (1 / T) (within an ulp
// of the reference's L / T, the same order and the same ties), in false past
// V. One 16-byte load where the 4 lie inside the row at an aligned address,
// else 4-byte loads; an entry past V reads -Inf, which no draw can select
// (probability 0, below every kept entry, the last in index order among
// ties), so a row of any length or alignment is drawn as the reference
// draws it (the tokens are clamped to V - 1).
__device__ __forceinline__ void load_round(const float *__restrict__ row, int V, int r, float invT, float (&z)[4],
                                           bool &in) {
    const int base = r * SROUND + 4 * (int)threadIdx.x;
    in = base < V;
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (in) {
        if (base + 4 <= V && ((uintptr_t)(row + base) & 15) == 0) {
            x = *(const float4 *)(row + base);
        } else {
            const float ninf = -__builtin_huge_valf();
            x.x = row[base];
            x.y = base + 1 < V ? row[base + 1] : ninf;
            x.z = base + 2 < V ? row[base + 2] : ninf;
            x.w = base + 3 < V ? row[base + 3] : ninf;
        }
    }
    z[0] = x.x; z[1] = x.y; z[2] = x.z; z[3] = x.w;
    if (invT != 1.0f) {
#pragma unroll
        for (int e = 0; e < 4; e++) z[e] = z[e] * invT;
    }
}

// A pass over the row: the loads of RB rounds are in flight together, then
// f(z, in, r) runs for each round in order (uniformly, so f may hold
// barriers).
constexpr int RB = 8;
template <class F>
__device__ __forceinline__ void for_rounds(const float *__restrict__ row, int V, int nround, float T, F &&f) {
    for (int r0 = 0; r0 < nround; r0 += RB) {
        float z[RB][4];
        bool in[RB];
#pragma unroll
        for (int b = 0; b < RB; b++) load_round(row, V, r0 + b, T, z[b], in[b]);
#pragma unroll
        for (int b = 0; b < RB; b++)
            if (r0 + b < nround) f(z[b], in[b], r0 + b);
    }
}

// exp for the probabilities (the hardware exp2 after a multiply by log2 e:
// ~1e-6 relative, the same value in every pass)
__device__ __forceinline__ float pexp(float x) { return __expf(x); }

// (m, s) = (max, sum exp(z - max)) merged; symmetric, so both partners of a
// butterfly get the same bits
__device__ __forceinline__ void merge_ms2(float &m, float &s, float m2, float s2) {
    const float mm = fmaxf(m, m2);
    if (mm == -__builtin_huge_valf()) {  // (both sums 0, or NaN from a NaN entry: kept)
        s = s + s2;
        return;
    }
    s = s * pexp(m - mm) + s2 * pexp(m2 - mm);
    m = mm;
}
__device__ void block_ms(float &m, float &s, float *red) {
    for (int o = 32; o > 0; o >>= 1) {
        const float m2 = __shfl_xor(m, o), s2 = __shfl_xor(s, o);
        merge_ms2(m, s, m2, s2);
    }
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    __syncthreads();
    if (l == 0) {
        red[w] = m;
        red[SNW + w] = s;
    }
    __syncthreads();
    m = l < SNW ? red[l] : -__builtin_huge_valf();
    s = l < SNW ? red[SNW + l] : 0.f;
    for (int o = 32; o > 0; o >>= 1) {
        const float m2 = __shfl_xor(m, o), s2 = __shfl_xor(s, o);
        merge_ms2(m, s, m2, s2);
    }
}

// First j in [0, n) of this thread's 4 values (slot 4t + e) with u <= the
// inclusive prefix; the block's scan total goes to *total.
__device__ int first_cdf_hit(const float (&v)[4], int n_here, float before, float u, float *redf, float &total) {
    float c[4], run = 0.f;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        run += v[e];
        c[e] = run;
    }
    const float ex = block_excl_scan_f(run, redf, total);
    int hit = INT_MAX;
#pragma unroll
    for (int e = 3; e >= 0; e--)
        if (e < n_here && u <= before + (ex + c[e])) hit = 4 * (int)threadIdx.x + e;
    return hit;
}

// Julia's findmax order as an unsigned key: the order-preserving key of the
// float (+0.0 above -0.0), every NaN the largest (NaNs equal: the first
// wins). A real float's key is at least 1.
__device__ __forceinline__ uint32_t jl_key(float z) { return isnan(z) ? 0xffffffffu : okey(z); }
__device__ __forceinline__ uint32_t wave_max_u(uint32_t v) {
    for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o));
    return v;
}
// The block's first index holding the largest key (INT_MAX when none: all
// keys 0); *best_k gets that key.
__device__ int block_argmax_key(uint32_t k, int i, uint32_t *s_k, int *s_i, uint32_t *best_k = nullptr) {
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    uint32_t m = wave_max_u(k);
    __syncthreads();
    if (l == 0) s_k[w] = m;
    __syncthreads();
    m = wave_max_u(l < SNW ? s_k[l] : 0u);
    if (best_k) *best_k = m;
    return block_min_i(k == m && m != 0u ? i : INT_MAX, s_i);
}

// Threshold selection counted from the top (the k-th largest z, or the z
// where the probability mass from the top reaches top_p). Pass A buckets
// w = zmax - z linearly, 8 buckets per unit of log-probability (bucket 255:
// the tail), which spreads real logits over many buckets; then 4 passes of
// 8 key bits each refine inside the chosen bucket, over its few elements.
// With MASS the buckets also carry each element's probability in 2^-40
// fixed point (integer atomics: the same sums in any order).
__device__ __forceinline__ uint32_t zbin(float z, float zmax) {
    const float w = (zmax - z) * 8.0f;
    return w < 255.0f ? (uint32_t)w : 255u;  // (-Inf and NaN: the tail)
}

struct Select {
    uint32_t zb;             // the bucket of pass A
    uint32_t tau;            // key of the threshold element inside it
    unsigned long long rem;  // units still to reach among the elements equal to tau
    uint32_t cnt;            // elements equal to tau
    bool all;                // (MASS) the total ran short of the target: keep every element
};

// Wave 0 finds, over the 256 buckets (descending or ascending index), the
// one holding the rem-th unit (~0ull in *selm when the total is short).
template <bool MASS>
__device__ void pick_bucket(const uint32_t *hist, const unsigned long long *mass, unsigned long long rem,
                            uint32_t *sel, unsigned long long *selm, bool descending) {
    const int t = threadIdx.x;
    if (t >= 64) return;
    unsigned long long c[4], sum = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int b = descending ? 255 - 4 * t - j : 4 * t + j;
        c[j] = MASS ? mass[b] : (unsigned long long)hist[b];
        sum += c[j];
    }
    unsigned long long inc = sum;
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned long long y = __shfl_up(inc, o);
        if (t >= o) inc += y;
    }
    const unsigned long long before = inc - sum;
    const bool found = before < rem && rem <= inc;
    if (found) {
        unsigned long long cum = before;
        for (int j = 0; j < 4; j++) {
            if (cum + c[j] >= rem) {
                sel[0] = descending ? 255u - 4u * t - j : 4u * t + j;
                selm[0] = cum;
                break;
            }
            cum += c[j];
        }
    }
    if (__ballot(found) == 0ull && t == 0) {
        sel[0] = 0u;
        selm[0] = ~0ull;
    }
}

// Fixed-point probability mass of z: p = exp(z - zmax) / S in units of 2^-40.
__device__ __forceinline__ unsigned long long mass_fx(float z, float zmax, float invS) {
    return (unsigned long long)(pexp(z - zmax) * invS * 1099511627776.0f);
}

// Passes B: the exact key inside bucket R.zb, 8 bits a pass from the top,
// R.rem units still to reach; over the nzb gathered keys and values (ck, cz)
// when gathered, else over the row. R.tau, R.rem and R.cnt on return, or
// R.all when (MASS) truncated masses fall just short of the target. At most
// SPAIR_MAX gathered elements are ranked directly instead: tau is the key
// whose larger keys hold less than R.rem units and which with its equals
// reaches it (integer sums: the key the passes would find; MASS: the
// elements' units staged in mass[], which holds 256).
constexpr int SPAIR_MAX = 128;
template <bool MASS>
__device__ void refine_threshold(const float *__restrict__ row, int V, int nround, float T, float zmax, float S,
                                 bool gathered, int nzb, uint32_t *hist, unsigned long long *mass, uint32_t *sel,
                                 unsigned long long *selm, const uint32_t *ck, const float *cz, Select &R) {
    const int t = threadIdx.x;
    const uint32_t zb = R.zb;
    const float invS = 1.0f / S;
    if (gathered && nzb <= SPAIR_MAX) {
        if (t == 0) {
            sel[0] = 0u;
            sel[1] = 0u;
            selm[0] = ~0ull;
        }
        if (MASS && t < nzb) mass[t] = mass_fx(cz[t], zmax, invS);  // (each element's units, once)
        __syncthreads();
        // element i = t / P compared with every P-th element from t % P (at
        // most 16 comparisons a lane); the P lanes of an element (adjacent,
        // in one wave) then add their sums
        int lp = 0;
        while (nzb > (16 << lp)) lp++;  // (nzb <= SPAIR_MAX: P = 2^lp <= 8)
        const int P = 1 << lp, i = t >> lp;
        const bool act = i < nzb;
        const uint32_t ki = act ? ck[i] : 0u;
        unsigned long long gt = 0, eq = 0;
        uint32_t ne = 0;
        if (act)
            for (int j = t & (P - 1); j < nzb; j += P) {
                const uint32_t kj = ck[j];
                const unsigned long long mj = MASS ? mass[j] : 1ull;
                if (kj > ki) {
                    gt += mj;
                } else if (kj == ki) {
                    eq += mj;
                    ne++;
                }
            }
        for (int o = 1; o < P; o <<= 1) {
            gt += __shfl_xor(gt, o);
            eq += __shfl_xor(eq, o);
            ne += __shfl_xor(ne, o);
        }
        if (act && (t & (P - 1)) == 0 && gt < R.rem && R.rem <= gt + eq) {  // (every element of key ki writes the same)
            sel[0] = ki;
            sel[1] = ne;
            selm[0] = gt;
        }
        __syncthreads();
        const uint32_t tau = sel[0], cnt = sel[1];
        const unsigned long long above = selm[0];
        __syncthreads();
        if (above == ~0ull) {
            R.all = true;
            return;
        }
        R.rem -= above;
        R.cnt = cnt;
        R.tau = tau;
        return;
    }
    uint32_t prefix = 0, pmask = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        if (t < 256) {
            hist[t] = 0;
            if (MASS) mass[t] = 0;
        }
        __syncthreads();
        if (gathered) {
            for (int i = t; i < nzb; i += SNT) {
                const uint32_t k = ck[i];
                if ((k & pmask) != prefix) continue;
                const uint32_t b = (k >> shift) & 255u;
                atomicAdd(&hist[b], 1u);
                if (MASS) atomicAdd(&mass[b], mass_fx(cz[i], zmax, invS));
            }
        } else {
            for_rounds(row, V, nround, T, [&](const float (&z)[4], bool in, int) {
                if (!in) return;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint32_t k = okey(z[e]);
                    if ((k & pmask) != prefix || zbin(z[e], zmax) != zb) continue;
                    const uint32_t b = (k >> shift) & 255u;
                    atomicAdd(&hist[b], 1u);
                    if (MASS) atomicAdd(&mass[b], mass_fx(z[e], zmax, invS));
                }
            });
        }
        __syncthreads();
        pick_bucket<MASS>(hist, mass, R.rem, sel, selm, true);
        __syncthreads();
        const uint32_t b = sel[0];
        const unsigned long long above = selm[0];
        const uint32_t cb = hist[b];
        __syncthreads();
        if (above == ~0ull) {  // (MASS: truncated masses just short of the target)
            R.all = true;
            return;
        }
        R.rem -= above;
        prefix |= b << shift;
        pmask |= 255u << shift;
        R.cnt = cb;
    }
    R.tau = prefix;
}

// The B passes read only the elements of bucket zb: when it holds at most
// SK_MAX of them, one more pass gathers their keys and values into LDS
// (ck, cz; any order: the passes only count) and the B passes run there
// instead of over the row.
template <bool MASS>
__device__ void select_threshold(const float *__restrict__ row, int V, int nround, float T, float zmax, float S,
                                 unsigned long long target, uint32_t *hist, unsigned long long *mass, uint32_t *sel,
                                 unsigned long long *selm, uint32_t *ck, float *cz, int *ncnt, Select &R) {
    const int t = threadIdx.x;
    R.zb = 255u;
    R.tau = 0u;
    R.rem = target;
    R.cnt = 0;
    R.all = false;
    const float invS = 1.0f / S;
    // pass A: buckets of w = zmax - z, largest z first = bucket 0 first
    if (t < 256) {
        hist[t] = 0;
        if (MASS) mass[t] = 0;
    }
    __syncthreads();
    for_rounds(row, V, nround, T, [&](const float (&z)[4], bool in, int) {
        if (!in) return;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t b = zbin(z[e], zmax);
            atomicAdd(&hist[b], 1u);
            if (MASS) atomicAdd(&mass[b], mass_fx(z[e], zmax, invS));
        }
    });
    __syncthreads();
    pick_bucket<MASS>(hist, mass, R.rem, sel, selm, false);
    __syncthreads();
    const uint32_t zb = sel[0];
    const unsigned long long aboveA = selm[0];
    const uint32_t nzb = hist[zb];
    __syncthreads();
    if (aboveA == ~0ull) {
        R.all = true;
        return;
    }
    R.rem -= aboveA;
    R.zb = zb;
    const bool gathered = nzb <= (uint32_t)SK_MAX;
    if (gathered) {
        if (t == 0) *ncnt = 0;
        __syncthreads();
        for_rounds(row, V, nround, T, [&](const float (&z)[4], bool in, int) {
            if (!in) return;
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (zbin(z[e], zmax) == zb) {
                    const int p = atomicAdd(ncnt, 1);  // < nzb: the predicate pass A counted
                    ck[p] = okey(z[e]);
                    cz[p] = z[e];
                }
        });
        __syncthreads();
    }
    refine_threshold<MASS>(row, V, nround, T, zmax, S, gathered, (int)nzb, hist, mass, sel, selm, ck, cz, R);
}

// Kept by a threshold: a larger z than the bucket (smaller bucket index), or
// inside it a larger key, or an equal key before index tie_lim.
__device__ __forceinline__ bool above_threshold(float z, int j, float zmax, uint32_t zb, uint32_t tau, int tie_lim) {
    const uint32_t b = zbin(z, zmax);
    if (b != zb) return b < zb;
    const uint32_t k = okey(z);
    return k > tau || (k == tau && j < tie_lim);
}

// The draw over n top-k candidates in LDS in index order (s_cidx: token
// ids, s_cp: z = L / T; s_sort: scratch), shared by draft_sample_kernel and
// the spread top-k draw: softmax over the candidates (the rest are
// exp(-Inf) = 0), top-p by a bitonic sort of their probabilities, min-p,
// then the inverse CDF in index order.
__device__ void draw_candidates(int n, const SampleArgs &a, float ur, int V, int *s_cidx, float *s_cp, int *s_sort,
                                float *s_redf, int *s_redi, int32_t *out_row) {
    const int t = threadIdx.x;
    // softmax over the candidates (the rest are exp(-Inf) = 0)
    float lm = -__builtin_huge_valf();
    for (int i = t; i < n; i += SNT) lm = fmaxf(lm, s_cp[i]);
    const float zmax = block_max(lm, s_redf);
    float ls = 0.f;
    for (int i = t; i < n; i += SNT) {
        const float w = pexp(s_cp[i] - zmax);
        s_cp[i] = w;
        ls += w;
    }
    const float S = block_sum(ls, s_redf);
    for (int i = t; i < n; i += SNT) s_cp[i] = s_cp[i] / S;
    __syncthreads();
    if (a.top_p < 1.0f) {
        // sort the slots by (p descending, slot ascending) = the stable
        // descending sortperm of the probabilities
        int P2 = 1;
        while (P2 < n) P2 <<= 1;
        for (int i = t; i < P2; i += SNT) s_sort[i] = i < n ? i : -1;
        __syncthreads();
        for (int size = 2; size <= P2; size <<= 1)
            for (int stride = size >> 1; stride > 0; stride >>= 1) {
                for (int i = t; i < P2 / 2; i += SNT) {
                    const int lo = ((i & ~(stride - 1)) << 1) | (i & (stride - 1));
                    const int hi = lo + stride;
                    const int A = s_sort[lo], B = s_sort[hi];
                    bool a_first;
                    if (A < 0) a_first = false;
                    else if (B < 0) a_first = true;
                    else {
                        const float pa = s_cp[A], pb = s_cp[B];
                        a_first = pa > pb || (pa == pb && A < B);
                    }
                    if (a_first != ((lo & size) == 0)) {
                        s_sort[lo] = B;
                        s_sort[hi] = A;
                    }
                }
                __syncthreads();
            }
        // the shortest sorted prefix whose mass reaches top_p
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int j = 4 * t + e;
            v[e] = j < n ? s_cp[s_sort[j]] : 0.f;
        }
        float tot;
        const int hit = first_cdf_hit(v, n - 4 * t, 0.f, a.top_p, s_redf, tot);
        const int cut = block_min_i(hit, s_redi);
        const int n_keep = cut == INT_MAX ? n : cut + 1;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int j = 4 * t + e;
            if (j < n && j >= n_keep) s_cp[s_sort[j]] = 0.f;
        }
        __syncthreads();
        float lt = 0.f;
        for (int i = t; i < n; i += SNT) lt += s_cp[i];
        const float total = block_sum(lt, s_redf);
        if (total > 0.f)
            for (int i = t; i < n; i += SNT) s_cp[i] = s_cp[i] / total;
        __syncthreads();
    }
    if (a.min_p > 0.f) {
        float lm2 = 0.f;
        for (int i = t; i < n; i += SNT) lm2 = fmaxf(lm2, s_cp[i]);
        const float thr = block_max(lm2, s_redf) * a.min_p;
        float lt = 0.f;
        for (int i = t; i < n; i += SNT) {
            float p = s_cp[i];
            if (p < thr) p = 0.f;
            s_cp[i] = p;
            lt += p;
        }
        const float total = block_sum(lt, s_redf);
        if (total > 0.f)
            for (int i = t; i < n; i += SNT) s_cp[i] = s_cp[i] / total;
        __syncthreads();
    }
    // inverse CDF in index order over the candidates
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int j = 4 * t + e;
        v[e] = j < n ? s_cp[j] : 0.f;
    }
    float tot;
    const int hit = first_cdf_hit(v, n - 4 * t, 0.f, ur, s_redf, tot);
    const int slot = block_min_i(hit, s_redi);
    if (t == 0) *out_row = slot == INT_MAX ? V - 1 : s_cidx[slot];
}

__global__ __launch_bounds__(SNT) void draft_sample_kernel(const float *__restrict__ L, int V, SampleArgs a,
                                                           const float *__restrict__ u, int32_t *__restrict__ out) {
    __shared__ float s_redf[2 * SNW];
    __shared__ float s_redv[SNW][RB];
    __shared__ uint32_t s_redu[SNW];
    __shared__ int s_redi[SNW];
    __shared__ uint32_t s_hist[256];
    __shared__ unsigned long long s_mass[256];
    __shared__ uint32_t s_sel[2];
    __shared__ unsigned long long s_selm[2];
    __shared__ float s_round[SMAX_ROUNDS];
    __shared__ float s_before;
    __shared__ int s_cidx[SK_MAX];
    __shared__ float s_cp[SK_MAX];
    __shared__ int s_sort[SK_MAX];
    __shared__ int s_ncnt;
    __shared__ float s_pm[SPART_ROUNDS][SNW], s_ps[SPART_ROUNDS][SNW];
    const int row = blockIdx.x, t = threadIdx.x;
    const float *Lr = L + (size_t)row * V;
    const int nround = (V + SROUND - 1) / SROUND;
    const float ur = u[row];
    const float invT = a.T > 0.f ? 1.0f / a.T : 1.0f;

    if (a.T == 0.0f) {
        // Julia's argmax: findmax order (the first NaN above every number,
        // +0.0 above -0.0), the first index among equals; each thread sees
        // its indices in increasing order
        uint32_t bk = 0u;
        int bi = INT_MAX;
        for_rounds(Lr, V, nround, 1.0f, [&](const float (&z)[4], bool in, int r) {
            if (!in) return;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t k = jl_key(z[e]);
                if (k > bk) {
                    bk = k;
                    bi = r * SROUND + 4 * t + e;
                }
            }
        });
        const int first = block_argmax_key(bk, bi, s_redu, s_redi);
        if (t == 0) out[row] = first == INT_MAX ? 0 : first;
        return;
    }
    const int K = a.top_k;
    if (K > 0 && K <= SK_MAX) {
        // ---- top-k: the k-th largest z, then the k candidates in index order
        float lmax = -__builtin_huge_valf(), nan = 0.f;
        for_rounds(Lr, V, nround, invT, [&](const float (&z)[4], bool in, int) {
            if (in)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    lmax = fmaxf(lmax, z[e]);
                    if (z[e] != z[e]) nan = 1.f;
                }
        });
        const float zm = block_max(lmax, s_redf);
        // a degenerate row (the reference's top-k keeps a NaN, its maximum is
        // then NaN; or no finite maximum) has NaN probabilities: last index
        if (block_max(nan, s_redf) > 0.f || !(zm > -__builtin_huge_valf() && zm < __builtin_huge_valf()) ||
            ur != ur) {
            if (t == 0) out[row] = V - 1;
            return;
        }
        // the reference's draw returns index 1 (here 0) when r <= 0: cumsum >= 0
        if (!(ur > 0.f)) {
            if (t == 0) out[row] = 0;
            return;
        }
        Select R;
        select_threshold<false>(Lr, V, nround, invT, zm, 1.f, (unsigned long long)K, s_hist, s_mass, s_sel, s_selm,
                                (uint32_t *)s_cidx, s_cp, &s_ncnt, R);
        const uint32_t zb = R.zb, tau = R.tau;
        const int rem = (int)R.rem;  // elements equal to tau that are kept, lowest index first
        int run_kept = 0, run_eq = 0;
        for_rounds(Lr, V, nround, invT, [&](const float (&z)[4], bool in, int r) {
            bool g[4], q[4];
            uint32_t ng = 0, nq = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t b = zbin(z[e], zm);
                const uint32_t k = okey(z[e]);
                g[e] = in && (b < zb || (b == zb && k > tau));
                q[e] = in && b == zb && k == tau;
                ng += g[e];
                nq += q[e];
            }
            uint32_t tot;
            const uint32_t ex = block_excl_scan_u(ng | (nq << 16), s_redu, tot);
            const int eq_before = (int)(ex >> 16);
            int pos = run_kept + (int)(ex & 0xffffu) + min(max(rem - run_eq, 0), eq_before);
            int er = run_eq + eq_before;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if (g[e] || (q[e] && er < rem)) {
                    if (pos < SK_MAX) {
                        s_cidx[pos] = r * SROUND + 4 * t + e;
                        s_cp[pos] = z[e];
                    }
                    pos++;
                }
                if (q[e]) er++;
            }
            run_kept += (int)(tot & 0xffffu) + min(max(rem - run_eq, 0), (int)(tot >> 16));
            run_eq += (int)(tot >> 16);
        });
        __syncthreads();
        const int n = min(run_kept, SK_MAX);  // == K
        draw_candidates(n, a, ur, V, s_cidx, s_cp, s_sort, s_redf, s_redi, out + row);
        return;
    }

    // ---- whole-row path: softmax statistics in one pass
    float zmax = -__builtin_huge_valf(), S = 0.f;
    // plain draws (no top-p, no min-p) over at most SPART_ROUNDS rounds:
    // every wave keeps the (max, sum exp(z - max)) of its part of each round,
    // so the rounds' sums for the draw need no second pass over the row
    bool by_parts = K == 0 && a.top_p >= 1.0f && a.min_p <= 0.f && nround <= SPART_ROUNDS;
    if (by_parts) {
        const int w = t >> 6;
        for_rounds(Lr, V, nround, invT, [&](const float (&z)[4], bool in, int r) {
            float m = -__builtin_huge_valf();
            if (in)
#pragma unroll
                for (int e = 0; e < 4; e++) m = fmaxf(m, z[e]);
            m = wave_max(m);
            float sw = 0.f;
            if (in)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    if (z[e] != z[e]) sw = __builtin_nanf("");  // (a NaN entry flags the row)
                    else if (m > -__builtin_huge_valf()) sw += pexp(z[e] - m);
                }
            sw = wave_sum(sw);
            if ((t & 63) == 0) {
                s_pm[r][w] = m;
                s_ps[r][w] = sw;
            }
        });
        __syncthreads();
        const int np = nround * SNW;
        float lm = -__builtin_huge_valf(), nan = 0.f;
        for (int i = t; i < np; i += SNT) {
            lm = fmaxf(lm, s_pm[i / SNW][i % SNW]);
            if (s_ps[i / SNW][i % SNW] != s_ps[i / SNW][i % SNW]) nan = 1.f;
        }
        zmax = block_max(lm, s_redf);
        const bool has_nan = block_max(nan, s_redf) > 0.f;
        float ls = 0.f;
        if (zmax > -__builtin_huge_valf())
            for (int i = t; i < np; i += SNT) {
                const float m = s_pm[i / SNW][i % SNW];
                if (m > -__builtin_huge_valf()) ls += s_ps[i / SNW][i % SNW] * pexp(m - zmax);
            }
        S = block_sum(ls, s_redf);
        if (has_nan) S = __builtin_nanf("");
        // rows without a finite maximum or sum (all -Inf, NaN) take the
        // online pass below, as every other draw does
        by_parts = zmax > -__builtin_huge_valf() && S > 0.f && S < __builtin_huge_valf();
    }
    if (!by_parts) {
        zmax = -__builtin_huge_valf();
        S = 0.f;
        for_rounds(Lr, V, nround, invT, [&](const float (&z)[4], bool in, int) {
            if (!in) return;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if (z[e] != z[e]) {
                    S = __builtin_nanf("");  // (a NaN entry: the row is degenerate)
                } else if (z[e] > zmax) {
                    S = S * pexp(zmax - z[e]) + 1.0f;
                    zmax = z[e];
                } else if (zmax > -__builtin_huge_valf()) {
                    S += pexp(z[e] - zmax);
                }
            }
        });
        block_ms(zmax, S, s_redf);
    }
    // a degenerate row (no finite maximum, or a NaN entry: the reference's
    // maximum is NaN then) has NaN probabilities: the draw returns the last
    // index; otherwise r <= 0 returns the first (cumsum >= 0)
    if (!(zmax > -__builtin_huge_valf() && zmax < __builtin_huge_valf()) || !(S > 0.f && S < __builtin_huge_valf()) ||
        ur != ur) {
        if (t == 0) out[row] = V - 1;
        return;
    }
    if (!(ur > 0.f)) {
        if (t == 0) out[row] = 0;
        return;
    }
    // the index limit of the ties at a threshold: the first n_eq of the
    // elements in bucket zb with key tau are kept (index order)
    auto tie_limit = [&](uint32_t zb, uint32_t tau, unsigned long long n_eq) {
        int run = 0, lim = V;
        for_rounds(Lr, V, nround, invT, [&](const float (&z)[4], bool in, int r) {
            bool q[4];
            uint32_t nq = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                q[e] = in && zbin(z[e], zmax) == zb && okey(z[e]) == tau;
                nq += q[e];
            }
            uint32_t tot;
            const uint32_t ex = block_excl_scan_u(nq, s_redu, tot);
            int cand = INT_MAX;
            int c = run + (int)ex;
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (q[e]) {
                    c++;
                    if (c == (int)n_eq && cand == INT_MAX) cand = r * SROUND + 4 * t + e + 1;
                }
            const int got = block_min_i(cand, s_redi);
            if (lim == V && got != INT_MAX) lim = got;
            run += (int)tot;
        });
        return lim;
    };
    // top-k above the candidate limit: the k-th largest z by count (the
    // candidate path's threshold), kept by comparison; the softmax is over
    // the kept entries (S their sum), and top-p / min-p act on it below
    uint32_t zbK = 256u, tauK = 0u;
    int tieK = V;
    if (K > 0) {
        Select RK;
        select_threshold<false>(Lr, V, nround, invT, zmax, 1.f, (unsigned long long)K, s_hist, s_mass, s_sel, s_selm,
                                (uint32_t *)s_cidx, s_cp, &s_ncnt, RK);
        if (!RK.all) {
            zbK = RK.zb;
            tauK = RK.tau;
            if (RK.rem < RK.cnt) tieK = tie_limit(zbK, tauK, RK.rem);
        }
        float ls = 0.f;
        for_rounds(Lr, V, nround, invT, [&](const float (&z)[4], bool in, int r) {
            if (in)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (zbK == 256u || above_threshold(z[e], r * SROUND + 4 * t + e, zmax, zbK, tauK, tieK))
                        ls += pexp(z[e] - zmax);
        });
        S = block_sum(ls, s_redf);
    }
    auto keptK = [&](float z, int j) { return zbK == 256u || above_threshold(z, j, zmax, zbK, tauK, tieK); };
    // kept: above_threshold(zb, tau, tie_lim); everything without top-p
    uint32_t zb = 256u, tau = 0u;
    int tie_lim = V;
    bool div_total = false;  // top-p renormalizes by the nucleus mass
    float total_p = 1.0f;
    // rounds' sums of the final probabilities from the last pass's per-wave
    // parts (s_ps, times parts_scale) instead of a pass of their own
    bool round_parts = false;
    float parts_scale = 1.0f;
    const float invS = 1.0f / S;  // (probabilities by reciprocals: within an ulp of the divisions)
    if (a.top_p < 1.0f) {
        const float tp = fmaxf(a.top_p, 0.f) * 1099511627776.0f;
        const unsigned long long target = tp < 1.0f ? 1ull : (unsigned long long)ceilf(tp);
        Select R;
        select_threshold<true>(Lr, V, nround, invT, zmax, S, target, s_hist, s_mass, s_sel, s_selm,
                               (uint32_t *)s_cidx, s_cp, &s_ncnt, R);
        if (!R.all) {
            zb = R.zb;
            tau = R.tau;
            // ties at tau share one probability: keep the first n_eq of them
            const float ptau = pexp(okey_inv(tau) - zmax) * invS;
            const unsigned long long mt = (unsigned long long)(ptau * 1099511627776.0f);
            unsigned long long n_eq = mt ? (R.rem + mt - 1) / mt : (unsigned long long)R.cnt;
            if (n_eq < 1) n_eq = 1;
            if (n_eq < R.cnt) tie_lim = tie_limit(zb, tau, n_eq);  // index of the n_eq-th tie
        }
        // mass of the nucleus, then p' = p / total (without min-p, the
        // rounds' sums of the draw come from this pass's per-wave parts)
        const bool parts = a.min_p <= 0.f && nround <= SPART_ROUNDS;
        float lt = 0.f;
        for_rounds(Lr, V, nround, invT, [&](const float (&z)[4], bool in, int r) {
            float c = 0.f;
            if (in)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int j = r * SROUND + 4 * t + e;
                    if (keptK(z[e], j) && (zb == 256u || above_threshold(z[e], j, zmax, zb, tau, tie_lim)))
                        c += pexp(z[e] - zmax) * invS;
                }
            lt += c;
            if (parts) {
                c = wave_sum(c);
                if ((t & 63) == 0) s_ps[r][t >> 6] = c;
            }
        });
        total_p = block_sum(lt, s_redf);
        div_total = total_p > 0.f;
        if (parts) {
            round_parts = true;
            parts_scale = div_total ? 1.0f / total_p : 1.0f;
        }
    }
    const float inv_total = div_total ? 1.0f / total_p : 1.0f;
    auto prob = [&](float z) {
        float p = pexp(z - zmax) * invS;
        if (div_total) p = p * inv_total;
        return p;
    };
    auto kept = [&](float z, int j) {
        return keptK(z, j) && (zb == 256u || above_threshold(z, j, zmax, zb, tau, tie_lim));
    };
    // min-p: the largest probability is the argmax's, exp(0) / S (renormalized)
    float thr = 0.f;
    bool div_total2 = false;
    float total2 = 1.0f;
    if (a.min_p > 0.f) {
        float pmax = invS;
        if (div_total) pmax = pmax * inv_total;
        thr = pmax * a.min_p;
        const bool parts = nround <= SPART_ROUNDS;
        float lt = 0.f;
        for_rounds(Lr, V, nround, invT, [&](const float (&z)[4], bool in, int r) {
            float c = 0.f;
            if (in)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (kept(z[e], r * SROUND + 4 * t + e)) {
                        const float p = prob(z[e]);
                        if (!(p < thr)) c += p;
                    }
            lt += c;
            if (parts) {
                c = wave_sum(c);
                if ((t & 63) == 0) s_ps[r][t >> 6] = c;
            }
        });
        total2 = block_sum(lt, s_redf);
        div_total2 = total2 > 0.f;
        if (parts) {
            round_parts = true;
            parts_scale = div_total2 ? 1.0f / total2 : 1.0f;
        }
    }
    const float inv_total2 = div_total2 ? 1.0f / total2 : 1.0f;
    auto final_p = [&](float z, int j) {
        if (!kept(z, j)) return 0.f;
        float p = prob(z);
        if (a.min_p > 0.f) {
            if (p < thr) return 0.f;
            if (div_total2) p = p * inv_total2;
        }
        return p;
    };
    // the draw: each round's sum (from the waves' parts, or batched: one
    // block reduction per RB rounds), the round, then the index inside it
    if (by_parts) {
        if (t < nround) {
            float sum = 0.f;
            for (int w = 0; w < SNW; w++) {
                const float m = s_pm[t][w];
                if (m > -__builtin_huge_valf()) sum += s_ps[t][w] * pexp(m - zmax);
            }
            s_round[t] = sum * invS;
        }
    } else if (round_parts) {
        if (t < nround) {
            float sum = 0.f;
            for (int w = 0; w < SNW; w++) sum += s_ps[t][w];
            s_round[t] = sum * parts_scale;
        }
    }
    for (int r0 = 0; r0 < (by_parts || round_parts ? 0 : nround); r0 += RB) {
        float part[RB];
#pragma unroll
        for (int b = 0; b < RB; b++) {
            float z[4];
            bool in;
            load_round(Lr, V, r0 + b, invT, z, in);
            float c = 0.f;
#pragma unroll
            for (int e = 0; e < 4; e++) c += in ? final_p(z[e], (r0 + b) * SROUND + 4 * t + e) : 0.f;
            part[b] = wave_sum(c);
        }
        __syncthreads();
        if ((t & 63) == 0)
#pragma unroll
            for (int b = 0; b < RB; b++) s_redv[t >> 6][b] = part[b];
        __syncthreads();
        if (t < RB && r0 + t < nround) {
            float sum = 0.f;
            for (int w = 0; w < SNW; w++) sum += s_redv[w][t];
            s_round[r0 + t] = sum;
        }
    }
    __syncthreads();
    if (t == 0) {
        float cum = 0.f;
        int rr = -1;
        for (int r = 0; r < nround; r++) {
            const float nc = cum + s_round[r];
            if (ur <= nc) {
                rr = r;
                break;
            }
            cum = nc;
        }
        s_sel[0] = (uint32_t)rr;
        s_before = cum;
    }
    __syncthreads();
    const int rr = (int)s_sel[0];
    const float before = s_before;
    __syncthreads();
    if (rr < 0) {
        if (t == 0) out[row] = V - 1;
        return;
    }
    float z[4], v[4];
    bool in;
    load_round(Lr, V, rr, invT, z, in);
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = in ? final_p(z[e], rr * SROUND + 4 * t + e) : 0.f;
    float tot;
    const int hit = first_cdf_hit(v, in ? 4 : 0, before, ur, s_redf, tot);
    const int local = block_min_i(hit, s_redi);
    // (the scan inside the round can end a rounding step below the round's
    // sum that selected it: then the round's last kept entry)
    int last = INT_MAX;
#pragma unroll
    for (int e = 0; e < 4; e++)
        if (v[e] > 0.f) last = INT_MAX - (4 * t + e);
    const int lastk = block_min_i(last, s_redi);
    if (t == 0) {
        int tok = local != INT_MAX ? rr * SROUND + local : lastk != INT_MAX ? rr * SROUND + (INT_MAX - lastk) : V - 1;
        out[row] = min(tok, V - 1);
    }
}

// Workspace of the spread draws: float2 part[rows][nround] (each round's
// (max, sum exp(z - max))), then a slot of SLOT_BYTES per round of each row
// (top-k: float cz[SK_SPREAD], int32 ci[SK_SPREAD], int32 cn; top-p: uint32
// hist[256], uint64 mass[256]; top-p / min-p: float csum at SLOT_CSUM), then
// ROW_BYTES per row (top-p: the selection state and the gathered threshold
// bucket: uint32 keys, float z, int32 index, SK_MAX each).
constexpr int SLOT_BYTES = 4096;
constexpr int SLOT_CSUM = 3072;
constexpr int ROW_GATHER = 256;
constexpr size_t ROW_BYTES = ROW_GATHER + (size_t)SK_MAX * 12;
struct SpreadWs {
    float2 *part;
    uint8_t *slots, *rows;
    int nround;
    __device__ uint8_t *slot(int row, int c) const { return slots + ((size_t)row * nround + c) * SLOT_BYTES; }
    __device__ uint8_t *rowb(int row) const { return rows + (size_t)row * ROW_BYTES; }
};

// The row's softmax statistics from its rounds' partials (a fixed order: the
// same bits in every kernel); false for a degenerate row, whose reference
// probabilities are all NaN (the draw returns the last index): no finite
// maximum (all -Inf, or a +Inf) or a NaN entry anywhere (a round's sum is
// NaN then). The reference's top-k keeps a NaN (its descending sortperm
// puts NaN first) and its maximum is then NaN, so this holds with top-k
// too. count (a top-k threshold, whose softmax is over the kept entries
// only): S = 1.
__device__ bool row_stats(const float2 *pr, int nround, float *s_redf, float &zmax, float &S, bool count = false) {
    const int t = threadIdx.x;
    float lm = -__builtin_huge_valf(), nan = 0.f;
    for (int i = t; i < nround; i += SNT) {
        const float2 p = pr[i];
        lm = fmaxf(lm, p.x);
        if (p.y != p.y) nan = 1.f;
    }
    zmax = block_max(lm, s_redf);
    const bool has_nan = block_max(nan, s_redf) > 0.f;
    float ls = 0.f;
    if (zmax > -__builtin_huge_valf())
        for (int i = t; i < nround; i += SNT) {
            const float2 p = pr[i];
            if (p.x > -__builtin_huge_valf()) ls += p.y * pexp(p.x - zmax);
        }
    S = block_sum(ls, s_redf);
    const bool finite_max = zmax > -__builtin_huge_valf() && zmax < __builtin_huge_valf();
    if (count) {
        S = 1.0f;
        return finite_max && !has_nan;
    }
    return finite_max && !has_nan && S > 0.f && S < __builtin_huge_valf();
}

// (max, sum exp(z - max)) of round blockIdx.x of row blockIdx.y: part[row][round].
__global__ __launch_bounds__(SNT) void chunk_stats_kernel(const float *__restrict__ L, int V, float invT,
                                                          float2 *__restrict__ part) {
    __shared__ float s_red[2 * SNW];
    const int r = blockIdx.x, row = blockIdx.y, nround = gridDim.x;
    float z[4];
    bool in;
    load_round(L + (size_t)row * V, V, r, invT, z, in);
    float m = -__builtin_huge_valf();
    if (in)
#pragma unroll
        for (int e = 0; e < 4; e++) m = fmaxf(m, z[e]);
    m = block_max(m, s_red);
    float sw = 0.f;
    if (in)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            if (z[e] != z[e]) sw = __builtin_nanf("");  // (flags the row even when m is -Inf)
            else if (m > -__builtin_huge_valf()) sw += pexp(z[e] - m);
        }
    sw = block_sum(sw, s_red);
    if (threadIdx.x == 0) part[(size_t)row * nround + r] = make_float2(m, sw);
}

// The draw of row blockIdx.x from its rounds' statistics: the row's max and
// sum, each round's probability mass, the round holding u (first with u <=
// the running sum), then the index inside it. A row without a finite maximum
// or sum (all -Inf, NaN, +Inf) draws V - 1, as the reference's NaN
// probabilities do; otherwise u <= 0 draws 0.
__global__ __launch_bounds__(SNT) void chunk_draw_kernel(const float *__restrict__ L, int V, float invT,
                                                         const float2 *__restrict__ part, const float *__restrict__ u,
                                                         int32_t *__restrict__ out) {
    __shared__ float s_redf[2 * SNW];
    __shared__ int s_redi[SNW];
    __shared__ float s_round[SMAX_ROUNDS];
    __shared__ float s_before;
    __shared__ int s_rr;
    const int row = blockIdx.x, t = threadIdx.x;
    const int nround = (V + SROUND - 1) / SROUND;
    const float ur = u[row];
    const float2 *pr = part + (size_t)row * nround;
    float zmax, S;
    if (!row_stats(pr, nround, s_redf, zmax, S) || ur != ur) {
        if (t == 0) out[row] = V - 1;
        return;
    }
    if (!(ur > 0.f)) {  // the reference's draw returns index 1 (here 0) when r <= 0
        if (t == 0) out[row] = 0;
        return;
    }
    const float invS = 1.0f / S;
    for (int i = t; i < nround; i += SNT) {
        const float2 p = pr[i];
        s_round[i] = p.x > -__builtin_huge_valf() ? p.y * pexp(p.x - zmax) * invS : 0.f;
    }
    __syncthreads();
    if (t == 0) {
        float cum = 0.f;
        int rr = -1;
        for (int r = 0; r < nround; r++) {
            const float nc = cum + s_round[r];
            if (ur <= nc) {
                rr = r;
                break;
            }
            cum = nc;
        }
        s_rr = rr;
        s_before = cum;
    }
    __syncthreads();
    const int rr = s_rr;
    const float before = s_before;
    if (rr < 0) {
        if (t == 0) out[row] = V - 1;
        return;
    }
    float z[4], v[4];
    bool in;
    load_round(L + (size_t)row * V, V, rr, invT, z, in);
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = in ? pexp(z[e] - zmax) * invS : 0.f;
    float tot;
    const int hit = first_cdf_hit(v, in ? 4 : 0, before, ur, s_redf, tot);
    const int local = block_min_i(hit, s_redi);
    // (the scan inside the round can end a rounding step below the round's
    // sum that selected it: then the round's last nonzero entry)
    int last = INT_MAX;
#pragma unroll
    for (int e = 0; e < 4; e++)
        if (v[e] > 0.f) last = INT_MAX - (4 * t + e);
    const int lastk = block_min_i(last, s_redi);
    if (t == 0) {
        const int tok =
            local != INT_MAX ? rr * SROUND + local : lastk != INT_MAX ? rr * SROUND + (INT_MAX - lastk) : V - 1;
        out[row] = min(tok, V - 1);
    }
}

// Spread greedy draws (T = 0): each chunk's first argmax in Julia's order
// (its key and index as float bits) into part[row][chunk], then one
// workgroup per row takes the first of those; an exact order, so the
// tokens are the one-workgroup kernel's.
__global__ __launch_bounds__(SNT) void chunk_argmax_kernel(const float *__restrict__ L, int V,
                                                           float2 *__restrict__ part) {
    __shared__ uint32_t s_k[SNW];
    __shared__ int s_i[SNW];
    const int c = blockIdx.x, row = blockIdx.y, t = threadIdx.x, nround = gridDim.x;
    float z[4];
    bool in;
    load_round(L + (size_t)row * V + (size_t)c * SROUND, min(SROUND, V - c * SROUND), 0, 1.0f, z, in);
    uint32_t bk = 0u;
    int bi = INT_MAX;
    if (in)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t k = jl_key(z[e]);
            if (k > bk) {
                bk = k;
                bi = c * SROUND + 4 * t + e;
            }
        }
    uint32_t best;
    const int first = block_argmax_key(bk, bi, s_k, s_i, &best);
    if (t == 0) part[(size_t)row * nround + c] = make_float2(__uint_as_float(best), __int_as_float(first));
}

__global__ __launch_bounds__(SNT) void argmax_draw_kernel(int V, const float2 *__restrict__ part,
                                                          int32_t *__restrict__ out) {
    __shared__ uint32_t s_k[SNW];
    __shared__ int s_i[SNW];
    const int row = blockIdx.x, t = threadIdx.x;
    const int nround = (V + SROUND - 1) / SROUND;
    uint32_t bk = 0u;
    int bi = INT_MAX;
    for (int c = t; c < nround; c += SNT) {  // (chunks in index order: the first best stays)
        const float2 p = part[(size_t)row * nround + c];
        const uint32_t k = __float_as_uint(p.x);
        if (k > bk) {
            bk = k;
            bi = __float_as_int(p.y);
        }
    }
    const int first = block_argmax_key(bk, bi, s_k, s_i);
    if (t == 0) out[row] = first == INT_MAX ? 0 : first;
}

// Spread top-k (1 <= K <= SK_SPREAD, V <= SPART_ROUNDS rounds): every
// chunk's own top-K by the one-row kernel's order (the row maximum's bucket,
// then the key; ties lowest index first), then one workgroup per row picks
// the row's top-K from the chunks' candidates by the same order. The union
// of the chunks' top-K holds the row's, and it is in index order, so the
// draw over the kept candidates is the one-row kernel's.
constexpr int SK_SPREAD = 64;

// Chunk blockIdx.x of row blockIdx.y: its top-K candidates (z and token id,
// index order) to cz / ci [row][chunk][SK_SPREAD], their count to cn.
__global__ __launch_bounds__(SNT) void chunk_topk_kernel(const float *__restrict__ L, int V, float invT, int K,
                                                         SpreadWs ws) {
    __shared__ float s_redf[2 * SNW];
    __shared__ uint32_t s_redu[SNW];
    __shared__ uint32_t s_hist[256];
    __shared__ unsigned long long s_mass[256];
    __shared__ uint32_t s_sel[2];
    __shared__ unsigned long long s_selm[2];
    __shared__ uint32_t s_ck[SK_MAX];
    __shared__ float s_cz[SK_MAX];
    __shared__ int s_ncnt;
    const int c = blockIdx.x, row = blockIdx.y, t = threadIdx.x, nround = gridDim.x;
    const float2 *part = ws.part;
    float lm = -__builtin_huge_valf();
    for (int i = t; i < nround; i += SNT) lm = fmaxf(lm, part[(size_t)row * nround + i].x);
    const float zm = block_max(lm, s_redf);
    const float *Lc = L + (size_t)row * V + (size_t)c * SROUND;
    const int Vc = min(SROUND, V - c * SROUND);
    Select R;
    select_threshold<false>(Lc, Vc, 1, invT, zm, 1.f, (unsigned long long)K, s_hist, s_mass, s_sel, s_selm, s_ck,
                            s_cz, &s_ncnt, R);
    const uint32_t zb = R.zb, tau = R.tau;
    const int rem = (int)R.rem;
    float z[4];
    bool in;
    load_round(Lc, Vc, 0, invT, z, in);
    bool g[4], q[4];
    uint32_t ng = 0, nq = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const uint32_t b = zbin(z[e], zm);
        const uint32_t k = okey(z[e]);
        g[e] = in && (R.all || b < zb || (b == zb && k > tau));
        q[e] = in && !R.all && b == zb && k == tau;
        ng += g[e];
        nq += q[e];
    }
    uint32_t tot;
    const uint32_t ex = block_excl_scan_u(ng | (nq << 16), s_redu, tot);
    const int eq_before = (int)(ex >> 16);
    int pos = (int)(ex & 0xffffu) + min(max(rem, 0), eq_before);
    int er = eq_before;
    uint8_t *sl = ws.slot(row, c);
    float *cz = (float *)sl;
    int32_t *ci = (int32_t *)(sl + SK_SPREAD * 4);
#pragma unroll
    for (int e = 0; e < 4; e++) {
        if (g[e] || (q[e] && er < rem)) {
            if (pos < SK_SPREAD) {
                cz[pos] = z[e];
                ci[pos] = c * SROUND + 4 * t + e;
            }
            pos++;
        }
        if (q[e]) er++;
    }
    if (t == 0)
        *(int32_t *)(sl + SK_SPREAD * 8) = min((int)(tot & 0xffffu) + min(max(rem, 0), (int)(tot >> 16)), SK_SPREAD);
}

// select_threshold over the n slots of z in LDS whose id is >= 0 (MASS
// off): the bucket of pass A, its keys gathered into ck (n entries), then
// refine_threshold; R.all when fewer than target.
__device__ void select_lds(const float *z, const int *id, int n, float zmax, unsigned long long target,
                           uint32_t *hist, uint32_t *sel, unsigned long long *selm, uint32_t *ck, int *ncnt,
                           Select &R) {
    const int t = threadIdx.x;
    R.zb = 255u;
    R.tau = 0u;
    R.rem = target;
    R.cnt = 0;
    R.all = false;
    if (t < 256) hist[t] = 0;
    if (t == 0) *ncnt = 0;
    __syncthreads();
    for (int i = t; i < n; i += SNT)
        if (id[i] >= 0) atomicAdd(&hist[zbin(z[i], zmax)], 1u);
    __syncthreads();
    pick_bucket<false>(hist, nullptr, R.rem, sel, selm, false);
    __syncthreads();
    const uint32_t zb = sel[0];
    const unsigned long long aboveA = selm[0];
    __syncthreads();
    if (aboveA == ~0ull) {
        R.all = true;
        return;
    }
    R.rem -= aboveA;
    R.zb = zb;
    for (int i = t; i < n; i += SNT)
        if (id[i] >= 0 && zbin(z[i], zmax) == zb) ck[atomicAdd(ncnt, 1)] = okey(z[i]);
    __syncthreads();
    refine_threshold<false>(nullptr, 0, 0, 1.f, zmax, 1.f, true, *ncnt, hist, nullptr, sel, selm, ck, nullptr, R);
}

// Row blockIdx.x: the chunks' candidates gathered in index order, the row's
// top-K among them, then draw_candidates as draft_sample_kernel's top-k path.
__global__ __launch_bounds__(SNT) void topk_draw_kernel(int V, SampleArgs a, SpreadWs ws, const float *__restrict__ u,
                                                        int32_t *__restrict__ out) {
    __shared__ float s_redf[2 * SNW];
    __shared__ uint32_t s_redu[SNW];
    __shared__ int s_redi[SNW];
    __shared__ uint32_t s_hist[256];
    __shared__ uint32_t s_sel[2];
    __shared__ unsigned long long s_selm[2];
    __shared__ float s_gz[SK_MAX];
    __shared__ int s_gi[SK_MAX];
    __shared__ int s_cidx[SK_MAX];
    __shared__ float s_cp[SK_MAX];
    __shared__ int s_sort[SK_MAX];
    __shared__ int s_ncnt;
    const int row = blockIdx.x, t = threadIdx.x;
    const int nround = (V + SROUND - 1) / SROUND;
    const float ur = u[row];
    // chunk c's candidates at slots c * SK_SPREAD + j (j < its count; id -1
    // beyond): index order, loaded with the statistics, no offsets needed
    const int n = nround * SK_SPREAD;  // <= SK_MAX
    for (int i = t; i < n; i += SNT) {  // (count and slot loaded together: the slot is workspace either way)
        const int c = i / SK_SPREAD, j = i - c * SK_SPREAD;
        const uint8_t *sl = ws.slot(row, c);
        const int cnt = *(const int32_t *)(sl + SK_SPREAD * 8);
        const float zj = ((const float *)sl)[j];
        const int ij = ((const int32_t *)(sl + SK_SPREAD * 4))[j];
        const bool live = j < cnt;
        s_gz[i] = live ? zj : 0.f;
        s_gi[i] = live ? ij : -1;
    }
    float lm = -__builtin_huge_valf(), nan = 0.f;
    for (int i = t; i < nround; i += SNT) {
        const float2 p = ws.part[(size_t)row * nround + i];
        lm = fmaxf(lm, p.x);
        if (p.y != p.y) nan = 1.f;
    }
    const float zm = block_max(lm, s_redf);  // (its barriers also publish the slots)
    if (block_max(nan, s_redf) > 0.f || !(zm > -__builtin_huge_valf() && zm < __builtin_huge_valf()) || ur != ur) {
        if (t == 0) out[row] = V - 1;  // degenerate row (a NaN is kept by the reference's top-k): NaN probabilities
        return;
    }
    if (!(ur > 0.f)) {  // the reference's draw returns index 1 (here 0) when r <= 0
        if (t == 0) out[row] = 0;
        return;
    }
    Select R;
    select_lds(s_gz, s_gi, n, zm, (unsigned long long)a.top_k, s_hist, s_sel, s_selm, (uint32_t *)s_sort, &s_ncnt, R);
    const uint32_t zb = R.zb, tau = R.tau;
    const int rem = (int)R.rem;
    // the kept candidates in index order (slots 4 t .. 4 t + 3: n <= SK_MAX)
    bool g[4], q[4];
    uint32_t ng = 0, nq = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int j = 4 * t + e;
        const bool live = j < n && s_gi[j] >= 0;
        const float z = live ? s_gz[j] : 0.f;
        const uint32_t b = zbin(z, zm), k = okey(z);
        g[e] = live && (R.all || b < zb || (b == zb && k > tau));
        q[e] = live && !R.all && b == zb && k == tau;
        ng += g[e];
        nq += q[e];
    }
    uint32_t tot;
    const uint32_t ex = block_excl_scan_u(ng | (nq << 16), s_redu, tot);
    const int eq_before = (int)(ex >> 16);
    int pos = (int)(ex & 0xffffu) + min(max(rem, 0), eq_before);
    int er = eq_before;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int j = 4 * t + e;
        if (g[e] || (q[e] && er < rem)) {
            if (pos < SK_MAX) {
                s_cidx[pos] = s_gi[j];
                s_cp[pos] = s_gz[j];
            }
            pos++;
        }
        if (q[e]) er++;
    }
    __syncthreads();
    const int nk = min((int)(tot & 0xffffu) + min(max(rem, 0), (int)(tot >> 16)), SK_MAX);  // == K
    draw_candidates(nk, a, ur, V, s_cidx, s_cp, s_sort, s_redf, s_redi, out + row);
}

// Spread top-p and / or min-p (no top-k): the row's statistics from the chunk
// partials; for top-p the chunks' pass-A histograms (counts and 2^-40 masses
// of the buckets below the row maximum) merged per row to the threshold
// bucket, that bucket's elements gathered in index order, the key passes
// over them (or over the row when the bucket holds more than SK_MAX), the
// ties at the threshold kept lowest index first; then each chunk's sum of
// the kept probabilities and one workgroup per row drawing from those sums,
// as draft_sample_kernel's whole-row path does (the same threshold rules).
enum : int { SEL_SELECT = 0, SEL_ALL = 1, SEL_DEGEN = 2 };
struct RowSel {
    int mode;
    uint32_t zb, tau;
    int tie_lim;
    unsigned long long rem;
    int nzb;
    float zmax, S;
};

__global__ __launch_bounds__(SNT) void chunk_hist_kernel(const float *__restrict__ L, int V, float invT, bool count,
                                                         SpreadWs ws) {
    __shared__ float s_redf[2 * SNW];
    __shared__ uint32_t s_hist[256];
    __shared__ unsigned long long s_mass[256];
    const int c = blockIdx.x, row = blockIdx.y, t = threadIdx.x;
    float zmax, S;
    const bool ok = row_stats(ws.part + (size_t)row * ws.nround, ws.nround, s_redf, zmax, S, count);
    if (t < 256) {
        s_hist[t] = 0;
        s_mass[t] = 0;
    }
    __syncthreads();
    if (ok) {
        const float invS = 1.0f / S;
        float z[4];
        bool in;
        load_round(L + (size_t)row * V + (size_t)c * SROUND, min(SROUND, V - c * SROUND), 0, invT, z, in);
        if (in)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t b = zbin(z[e], zmax);
                atomicAdd(&s_hist[b], 1u);
                if (!count) atomicAdd(&s_mass[b], mass_fx(z[e], zmax, invS));
            }
    }
    __syncthreads();
    uint8_t *sl = ws.slot(row, c);
    if (t < 256) {
        ((uint32_t *)sl)[t] = s_hist[t];
        ((unsigned long long *)(sl + 1024))[t] = s_mass[t];
    }
}

// Row blockIdx.x: the merged histograms, the bucket holding the target mass
// (top_k > 0: the bucket holding the top_k-th element).
__global__ __launch_bounds__(SNT) void row_pick_kernel(float top_p, int top_k, SpreadWs ws) {
    __shared__ float s_redf[2 * SNW];
    __shared__ uint32_t s_hist[256];
    __shared__ unsigned long long s_mass[256];
    __shared__ uint32_t s_sel[2];
    __shared__ unsigned long long s_selm[2];
    const int row = blockIdx.x, t = threadIdx.x, nround = ws.nround;
    RowSel *rs = (RowSel *)ws.rowb(row);
    float zmax, S;
    if (!row_stats(ws.part + (size_t)row * nround, nround, s_redf, zmax, S, top_k > 0)) {
        if (t == 0) rs->mode = SEL_DEGEN;
        return;
    }
    if (t < 256) {
        s_hist[t] = 0;
        s_mass[t] = 0;
    }
    __syncthreads();
    {  // bucket t % 256 over every fourth chunk from t / 256 (integer sums: any order)
        const int b = t & 255;
        uint32_t h = 0;
        unsigned long long m = 0;
#pragma unroll 4
        for (int c = t >> 8; c < nround; c += SNT / 256) {
            const uint8_t *sl = ws.slot(row, c);
            h += ((const uint32_t *)sl)[b];
            if (top_k == 0) m += ((const unsigned long long *)(sl + 1024))[b];
        }
        atomicAdd(&s_hist[b], h);
        if (top_k == 0) atomicAdd(&s_mass[b], m);
    }
    __syncthreads();
    const float tp = fmaxf(top_p, 0.f) * 1099511627776.0f;
    const unsigned long long target =
        top_k > 0 ? (unsigned long long)top_k : tp < 1.0f ? 1ull : (unsigned long long)ceilf(tp);
    if (top_k > 0)
        pick_bucket<false>(s_hist, nullptr, target, s_sel, s_selm, false);
    else
        pick_bucket<true>(s_hist, s_mass, target, s_sel, s_selm, false);
    __syncthreads();
    if (t == 0) {
        const uint32_t zb = s_sel[0];
        const unsigned long long above = s_selm[0];
        rs->zmax = zmax;
        rs->S = S;
        if (above == ~0ull) {
            rs->mode = SEL_ALL;
        } else {
            rs->mode = SEL_SELECT;
            rs->zb = zb;
            rs->rem = target - above;
            rs->nzb = (int)s_hist[zb];
        }
    }
}

// Chunk blockIdx.x of row blockIdx.y: its elements of the threshold bucket
// (key, z, index) at their index-order place in the row's gather.
__global__ __launch_bounds__(SNT) void chunk_gather_kernel(const float *__restrict__ L, int V, float invT, SpreadWs ws) {
    __shared__ uint32_t s_redu[SNW];
    const int c = blockIdx.x, row = blockIdx.y, t = threadIdx.x;
    const RowSel *rs = (const RowSel *)ws.rowb(row);
    if (rs->mode != SEL_SELECT || rs->nzb > SK_MAX) return;
    const uint32_t zb = rs->zb;
    const float zmax = rs->zmax;
    uint32_t tot;
    const uint32_t before = t < c ? ((const uint32_t *)ws.slot(row, t))[zb] : 0u;  // (c < nround <= SNT)
    block_excl_scan_u(before, s_redu, tot);
    const uint32_t off = tot;
    float z[4];
    bool in;
    load_round(L + (size_t)row * V + (size_t)c * SROUND, min(SROUND, V - c * SROUND), 0, invT, z, in);
    bool q[4];
    uint32_t nq = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        q[e] = in && zbin(z[e], zmax) == zb;
        nq += q[e];
    }
    uint32_t tq;
    uint32_t pos = off + block_excl_scan_u(nq, s_redu, tq);
    uint8_t *g = ws.rowb(row) + ROW_GATHER;
#pragma unroll
    for (int e = 0; e < 4; e++)
        if (q[e] && pos < (uint32_t)SK_MAX) {  // (pos < nzb: the counts of chunk_hist_kernel)
            ((uint32_t *)g)[pos] = okey(z[e]);
            ((float *)(g + SK_MAX * 4))[pos] = z[e];
            ((int32_t *)(g + SK_MAX * 8))[pos] = c * SROUND + 4 * t + e;
            pos++;
        }
}

// Row blockIdx.x: the key passes inside the threshold bucket, then the ties
// kept at the threshold (the first n_eq in index order; count: top-k, n_eq
// the units left at tau).
__global__ __launch_bounds__(SNT) void row_select_kernel(const float *__restrict__ L, int V, float invT, bool count,
                                                         SpreadWs ws) {
    __shared__ uint32_t s_redu[SNW];
    __shared__ int s_redi[SNW];
    __shared__ uint32_t s_hist[256];
    __shared__ unsigned long long s_mass[256];
    __shared__ uint32_t s_sel[2];
    __shared__ unsigned long long s_selm[2];
    __shared__ uint32_t s_ck[SK_MAX];
    __shared__ float s_cz[SK_MAX];
    __shared__ int s_ci[SK_MAX];
    const int row = blockIdx.x, t = threadIdx.x, nround = ws.nround;
    RowSel *rs = (RowSel *)ws.rowb(row);
    if (rs->mode != SEL_SELECT) return;
    const float zmax = rs->zmax, S = rs->S;
    const int nzb = rs->nzb;
    const bool gathered = nzb <= SK_MAX;
    const float *Lr = L + (size_t)row * V;
    if (gathered) {
        const uint8_t *g = ws.rowb(row) + ROW_GATHER;
        for (int i = t; i < nzb; i += SNT) {
            s_ck[i] = ((const uint32_t *)g)[i];
            s_cz[i] = ((const float *)(g + SK_MAX * 4))[i];
            s_ci[i] = ((const int32_t *)(g + SK_MAX * 8))[i];
        }
    }
    __syncthreads();
    Select R;
    R.zb = rs->zb;
    R.tau = 0u;
    R.rem = rs->rem;
    R.cnt = 0;
    R.all = false;
    if (count)
        refine_threshold<false>(Lr, V, nround, invT, zmax, 1.f, gathered, nzb, s_hist, s_mass, s_sel, s_selm, s_ck,
                                s_cz, R);
    else
        refine_threshold<true>(Lr, V, nround, invT, zmax, S, gathered, nzb, s_hist, s_mass, s_sel, s_selm, s_ck,
                               s_cz, R);
    if (R.all) {
        if (t == 0) rs->mode = SEL_ALL;
        return;
    }
    const uint32_t zb = R.zb, tau = R.tau;
    // ties at tau share one probability: keep the first n_eq of them
    unsigned long long n_eq = R.rem;
    if (!count) {
        const float ptau = pexp(okey_inv(tau) - zmax) * (1.0f / S);
        const unsigned long long mt = (unsigned long long)(ptau * 1099511627776.0f);
        n_eq = mt ? (R.rem + mt - 1) / mt : (unsigned long long)R.cnt;
    }
    if (n_eq < 1) n_eq = 1;
    int tie_lim = V;
    if (n_eq < R.cnt) {
        if (gathered) {  // the gather is in index order: slots 4 t .. 4 t + 3
            bool q[4];
            uint32_t nq = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int j = 4 * t + e;
                q[e] = j < nzb && s_ck[j] == tau;
                nq += q[e];
            }
            uint32_t tot;
            int cnum = (int)block_excl_scan_u(nq, s_redu, tot);
            int cand = INT_MAX;
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (q[e]) {
                    cnum++;
                    if (cnum == (int)n_eq && cand == INT_MAX) cand = s_ci[4 * t + e] + 1;
                }
            tie_lim = block_min_i(cand, s_redi);
        } else {
            int run = 0, lim = V;
            for_rounds(Lr, V, nround, invT, [&](const float (&z)[4], bool in, int r) {
                bool q[4];
                uint32_t nq = 0;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    q[e] = in && zbin(z[e], zmax) == zb && okey(z[e]) == tau;
                    nq += q[e];
                }
                uint32_t tot;
                const uint32_t ex = block_excl_scan_u(nq, s_redu, tot);
                int cand = INT_MAX;
                int cc = run + (int)ex;
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (q[e]) {
                        cc++;
                        if (cc == (int)n_eq && cand == INT_MAX) cand = r * SROUND + 4 * t + e + 1;
                    }
                const int got = block_min_i(cand, s_redi);
                if (lim == V && got != INT_MAX) lim = got;
                run += (int)tot;
            });
            tie_lim = lim;
        }
    }
    if (t == 0) {
        rs->tau = tau;
        rs->tie_lim = tie_lim;
    }
}

// An entry's probability through the cuts: p = exp(z - zmax) / S, 0 when
// top-p (the row's selection) drops it; with min-p, renormalized by the
// nucleus mass (inv1 = 1 / its total; 1 without top-p) and 0 below
// thr = inv1 / S * min_p (the largest probability times min_p).
struct Keep {
    bool topp, minp, all;
    uint32_t zb, tau;
    int tie_lim;
    float zmax, invS, inv1, thr;
    __device__ float p1(float z, int j) const {
        if (topp && !(all || above_threshold(z, j, zmax, zb, tau, tie_lim))) return 0.f;
        float p = pexp(z - zmax) * invS;
        if (minp) {
            if (topp) p = p * inv1;
            if (p < thr) return 0.f;
        }
        return p;
    }
};

// 1 / the sum of the row's chunk values at byte `off` of their slots (a
// fixed order), or 1 when it is not positive.
__device__ float kept_inv(const SpreadWs &ws, int row, int off, float *s_redf) {
    float l = 0.f;
    for (int i = threadIdx.x; i < ws.nround; i += SNT) l += *(const float *)(ws.slot(row, i) + off);
    const float total = block_sum(l, s_redf);
    return total > 0.f ? 1.0f / total : 1.0f;
}

// false for a row without finite statistics (no draw); minp: the min-p
// stage (its inv1 from the top-p stage's kept sums).
__device__ bool load_keep(const SpreadWs &ws, int row, bool topp, bool minp, float min_p, float zmax, float S,
                          float *s_redf, Keep &k) {
    k.topp = topp;
    k.minp = minp;
    k.zmax = zmax;
    k.invS = 1.0f / S;
    k.all = false;
    k.zb = 256u;
    k.tau = 0u;
    k.tie_lim = 0;
    k.inv1 = 1.0f;
    if (topp) {
        const RowSel *rs = (const RowSel *)ws.rowb(row);
        if (rs->mode == SEL_DEGEN) return false;
        k.all = rs->mode == SEL_ALL;
        k.zb = rs->zb;
        k.tau = rs->tau;
        k.tie_lim = rs->tie_lim;
        if (minp) k.inv1 = kept_inv(ws, row, SLOT_CSUM, s_redf);
    }
    k.thr = k.invS * k.inv1 * min_p;
    return true;
}

// Chunk blockIdx.x of row blockIdx.y: the sum of its kept probabilities,
// stage 0 (top-p) at SLOT_CSUM, stage 1 (min-p, after top-p if topp) at
// SLOT_CSUM + 4.
__global__ __launch_bounds__(SNT) void chunk_keptsum_kernel(const float *__restrict__ L, int V, float invT, bool topp,
                                                            int stage, float min_p, SpreadWs ws) {
    __shared__ float s_redf[2 * SNW];
    const int c = blockIdx.x, row = blockIdx.y, t = threadIdx.x;
    float zmax, S;
    if (topp) {  // (the statistics row_pick_kernel stored: the same bits)
        const RowSel *rs = (const RowSel *)ws.rowb(row);
        if (rs->mode == SEL_DEGEN) return;
        zmax = rs->zmax;
        S = rs->S;
    } else if (!row_stats(ws.part + (size_t)row * ws.nround, ws.nround, s_redf, zmax, S)) {
        return;
    }
    Keep keep;
    if (!load_keep(ws, row, topp, stage == 1, min_p, zmax, S, s_redf, keep)) return;
    float z[4];
    bool in;
    load_round(L + (size_t)row * V + (size_t)c * SROUND, min(SROUND, V - c * SROUND), 0, invT, z, in);
    float sum = 0.f;
    if (in)
#pragma unroll
        for (int e = 0; e < 4; e++) sum += keep.p1(z[e], c * SROUND + 4 * t + e);
    sum = block_sum(sum, s_redf);
    if (t == 0) *(float *)(ws.slot(row, c) + SLOT_CSUM + 4 * stage) = sum;
}

// Row blockIdx.x: the kept mass of the last stage, each round's share of
// it, the round holding u, then the index inside it (as chunk_draw_kernel
// over the kept entries).
__global__ __launch_bounds__(SNT) void keep_draw_kernel(const float *__restrict__ L, int V, float invT, bool topp,
                                                        bool minp, float min_p, SpreadWs ws,
                                                        const float *__restrict__ u, int32_t *__restrict__ out) {
    __shared__ float s_redf[2 * SNW];
    __shared__ int s_redi[SNW];
    __shared__ float s_round[SMAX_ROUNDS];
    __shared__ float s_before;
    __shared__ int s_rr;
    const int row = blockIdx.x, t = threadIdx.x, nround = ws.nround;
    const float ur = u[row];
    float zmax, S;
    bool ok;
    if (topp) {  // (the statistics row_pick_kernel stored: the same bits)
        const RowSel *rs = (const RowSel *)ws.rowb(row);
        ok = rs->mode != SEL_DEGEN;
        zmax = rs->zmax;
        S = rs->S;
    } else {
        ok = row_stats(ws.part + (size_t)row * nround, nround, s_redf, zmax, S);
    }
    Keep keep;
    if (!ok || !load_keep(ws, row, topp, minp, min_p, zmax, S, s_redf, keep) || ur != ur) {
        if (t == 0) out[row] = V - 1;
        return;
    }
    if (!(ur > 0.f)) {  // the reference's draw returns index 1 (here 0) when r <= 0
        if (t == 0) out[row] = 0;
        return;
    }
    const int off = SLOT_CSUM + (minp ? 4 : 0);
    const float inv = kept_inv(ws, row, off, s_redf);
    for (int i = t; i < nround; i += SNT) s_round[i] = *(const float *)(ws.slot(row, i) + off) * inv;
    __syncthreads();
    if (t == 0) {
        float cum = 0.f;
        int rr = -1;
        for (int r = 0; r < nround; r++) {
            const float nc = cum + s_round[r];
            if (ur <= nc) {
                rr = r;
                break;
            }
            cum = nc;
        }
        s_rr = rr;
        s_before = cum;
    }
    __syncthreads();
    const int rr = s_rr;
    const float before = s_before;
    if (rr < 0) {
        if (t == 0) out[row] = V - 1;
        return;
    }
    float z[4], v[4];
    bool in;
    load_round(L + (size_t)row * V, V, rr, invT, z, in);
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = in ? keep.p1(z[e], rr * SROUND + 4 * t + e) * inv : 0.f;
    float tot;
    const int hit = first_cdf_hit(v, in ? 4 : 0, before, ur, s_redf, tot);
    const int local = block_min_i(hit, s_redi);
    int last = INT_MAX;
#pragma unroll
    for (int e = 0; e < 4; e++)
        if (v[e] > 0.f) last = INT_MAX - (4 * t + e);
    const int lastk = block_min_i(last, s_redi);
    if (t == 0) {
        const int tok =
            local != INT_MAX ? rr * SROUND + local : lastk != INT_MAX ? rr * SROUND + (INT_MAX - lastk) : V - 1;
        out[row] = min(tok, V - 1);
    }
}

// Spread top-k above SK_SPREAD (or over more than SPART_ROUNDS rounds), with
// any top-p / min-p after it: the k-th element's bucket and key by count
// (as top-p's threshold), then each chunk's kept entries counted, compacted
// in index order into the row's gather (k <= SK_MAX), and one workgroup per
// row runs draft_sample_kernel's candidate draw over them: its tokens.
__global__ __launch_bounds__(SNT) void chunk_keptcount_kernel(const float *__restrict__ L, int V, float invT,
                                                              SpreadWs ws) {
    __shared__ uint32_t s_redu[SNW];
    const int c = blockIdx.x, row = blockIdx.y, t = threadIdx.x;
    const RowSel *rs = (const RowSel *)ws.rowb(row);
    const int mode = rs->mode;
    if (mode == SEL_DEGEN) return;
    const uint32_t zb = rs->zb, tau = rs->tau;
    const int tie_lim = rs->tie_lim;
    const float zmax = rs->zmax;
    float z[4];
    bool in;
    load_round(L + (size_t)row * V + (size_t)c * SROUND, min(SROUND, V - c * SROUND), 0, invT, z, in);
    uint32_t n = 0;
    if (in)
#pragma unroll
        for (int e = 0; e < 4; e++)
            n += mode == SEL_ALL || above_threshold(z[e], c * SROUND + 4 * t + e, zmax, zb, tau, tie_lim);
    uint32_t tot;
    block_excl_scan_u(n, s_redu, tot);
    if (t == 0) *(uint32_t *)(ws.slot(row, c) + SLOT_CSUM) = tot;
}

__global__ __launch_bounds__(SNT) void chunk_compact_kernel(const float *__restrict__ L, int V, float invT,
                                                            SpreadWs ws) {
    __shared__ uint32_t s_redu[SNW];
    const int c = blockIdx.x, row = blockIdx.y, t = threadIdx.x;
    const RowSel *rs = (const RowSel *)ws.rowb(row);
    const int mode = rs->mode;
    if (mode == SEL_DEGEN) return;
    const uint32_t zb = rs->zb, tau = rs->tau;
    const int tie_lim = rs->tie_lim;
    const float zmax = rs->zmax;
    uint32_t tot;
    const uint32_t before = t < c ? *(const uint32_t *)(ws.slot(row, t) + SLOT_CSUM) : 0u;  // (c < nround <= SNT)
    block_excl_scan_u(before, s_redu, tot);
    const uint32_t off = tot;
    float z[4];
    bool in;
    load_round(L + (size_t)row * V + (size_t)c * SROUND, min(SROUND, V - c * SROUND), 0, invT, z, in);
    bool k[4];
    uint32_t n = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        k[e] = in && (mode == SEL_ALL || above_threshold(z[e], c * SROUND + 4 * t + e, zmax, zb, tau, tie_lim));
        n += k[e];
    }
    uint32_t tk;
    uint32_t pos = off + block_excl_scan_u(n, s_redu, tk);
    uint8_t *g = ws.rowb(row) + ROW_GATHER;
#pragma unroll
    for (int e = 0; e < 4; e++)
        if (k[e]) {
            if (pos < (uint32_t)SK_MAX) {
                ((float *)(g + SK_MAX * 4))[pos] = z[e];
                ((int32_t *)(g + SK_MAX * 8))[pos] = c * SROUND + 4 * t + e;
            }
            pos++;
        }
}

__global__ __launch_bounds__(SNT) void cand_draw_kernel(int V, SampleArgs a, SpreadWs ws, const float *__restrict__ u,
                                                        int32_t *__restrict__ out) {
    __shared__ float s_redf[2 * SNW];
    __shared__ int s_redi[SNW];
    __shared__ int s_cidx[SK_MAX];
    __shared__ float s_cp[SK_MAX];
    __shared__ int s_sort[SK_MAX];
    const int row = blockIdx.x, t = threadIdx.x, nround = ws.nround;
    const float ur = u[row];
    if (((const RowSel *)ws.rowb(row))->mode == SEL_DEGEN || ur != ur) {  // (as the one-row kernel)
        if (t == 0) out[row] = V - 1;
        return;
    }
    if (!(ur > 0.f)) {  // the reference's draw returns index 1 (here 0) when r <= 0
        if (t == 0) out[row] = 0;
        return;
    }
    float l = 0.f;
    for (int c = t; c < nround; c += SNT) l += (float)*(const uint32_t *)(ws.slot(row, c) + SLOT_CSUM);
    const int n = min((int)block_sum(l, s_redf), SK_MAX);  // (counts below 2^24: exact)
    const uint8_t *g = ws.rowb(row) + ROW_GATHER;
    for (int i = t; i < n; i += SNT) {
        s_cp[i] = ((const float *)(g + SK_MAX * 4))[i];
        s_cidx[i] = ((const int32_t *)(g + SK_MAX * 8))[i];
    }
    __syncthreads();
    draw_candidates(n, a, ur, V, s_cidx, s_cp, s_sort, s_redf, s_redi, out + row);
}

// In place on rows of logits: for every distinct id of the row's list in
// [0, V): x -= presence (if presence != 0), then x = x > 0 ? x / rep : x * rep
// (if rep != 1). A bitmap in LDS skips repeated ids; it covers a window of
// PEN_WINDOW ids, and a vocabulary past that is taken window by window
// (each reads the row's list once).
constexpr int PEN_NT = 256;
constexpr int PEN_WINDOW = 262144;
__global__ __launch_bounds__(PEN_NT) void penalty_kernel(float *__restrict__ L, int V, const int32_t *__restrict__ tok,
                                                          int n_tok, int64_t tok_stride, float presence,
                                                          float repetition) {
    __shared__ uint32_t seen[PEN_WINDOW / 32];
    const int row = blockIdx.x, t = threadIdx.x;
    const int32_t *ids = tok + (size_t)row * tok_stride;
    float *x = L + (size_t)row * V;
    for (int w0 = 0; w0 < V; w0 += PEN_WINDOW) {
        const int wn = min(PEN_WINDOW, V - w0);
        const int nw = (wn + 31) / 32;
        __syncthreads();  // (the previous window's bitmap is no longer read)
        for (int i = t; i < nw; i += PEN_NT) seen[i] = 0u;
        __syncthreads();
        for (int i = t; i < n_tok; i += PEN_NT) {
            const int id = ids[i] - w0;
            if (id < 0 || id >= wn) continue;
            const uint32_t bit = 1u << (id & 31);
            if (atomicOr(&seen[id >> 5], bit) & bit) continue;
            float v = x[w0 + id];
            if (presence != 0.f) v -= presence;
            if (repetition != 1.0f) v = v > 0.f ? v / repetition : v * repetition;
            x[w0 + id] = v;
        }
    }
}

}  // namespace

int sample_max_v() { return SMAX_ROUNDS * SROUND; }

hipError_t launch_sample(const float *L, int rows, int V, float T, int top_k, float top_p, float min_p, const float *u,
                         int32_t *out, hipStream_t st) {
    const SampleArgs a{T, top_k, top_p, min_p};
    draft_sample_kernel<<<rows, SNT, 0, st>>>(L, V, a, u, out);
    return hipGetLastError();
}

size_t sample_spread_ws(int rows, int V) {
    const size_t rc = (size_t)rows * ((V + SROUND - 1) / SROUND);
    return rc * (sizeof(float2) + SLOT_BYTES) + (size_t)rows * ROW_BYTES;
}

// Rows spread over workgroups of one round each (chunk statistics first):
// plain draws (T > 0, no top-k, top-p or min-p), then one workgroup per row
// merges them, picks the round and scans it (as draft_sample_kernel's draw);
// top-k from 1 to SK_SPREAD over at most SPART_ROUNDS rounds: each chunk's
// top-k, then one workgroup per row draws among the candidates; top-p
// and / or min-p without top-k (threshold histograms, pick, gather, key
// passes): the chunks' kept sums per stage, then the draw; a larger top-k
// (any top-p / min-p after it): its threshold as top-p's but by count, the
// kept entries compacted, then the candidate draw; T = 0: each chunk's
// argmax, then the row's. Rows over more than SMAX_ROUNDS rounds run draft_sample_kernel.
// ws: sample_spread_ws bytes (8-byte aligned).
hipError_t launch_sample_spread(const float *L, int rows, int V, float T, int top_k, float top_p, float min_p,
                                const float *u, int32_t *out, void *ws, hipStream_t st) {
    const int nround = (V + SROUND - 1) / SROUND;
    if (T == 0.f && nround <= SMAX_ROUNDS) {
        float2 *part = (float2 *)ws;
        chunk_argmax_kernel<<<dim3(nround, rows), SNT, 0, st>>>(L, V, part);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        argmax_draw_kernel<<<rows, SNT, 0, st>>>(V, part, out);
        return hipGetLastError();
    }
    const bool live = T > 0.f && nround <= SMAX_ROUNDS;
    const bool plain = live && top_k == 0 && top_p >= 1.0f && min_p <= 0.f;
    const bool topk = live && top_k >= 1 && top_k <= SK_SPREAD && nround <= SPART_ROUNDS;
    // top-k beyond the chunk-candidate path: the threshold as top-p's, by
    // count, its kept entries compacted (up to SK_MAX of them; a larger top-k
    // takes the one-workgroup kernel's threshold path)
    const bool bigk = live && top_k > 0 && top_k <= SK_MAX && !topk;
    const bool topp = live && ((top_k == 0 && top_p < 1.0f) || bigk);
    const bool minp = live && top_k == 0 && min_p > 0.f;
    if (!plain && !topk && !topp && !minp) return launch_sample(L, rows, V, T, top_k, top_p, min_p, u, out, st);
    if (top_k > SK_MAX) return launch_sample(L, rows, V, T, top_k, top_p, min_p, u, out, st);
    const float invT = 1.0f / T;
    const size_t rc = (size_t)rows * nround;
    uint8_t *w = (uint8_t *)ws;
    const SpreadWs W{(float2 *)w, w + rc * sizeof(float2), w + rc * (sizeof(float2) + SLOT_BYTES), nround};
    const dim3 chunks(nround, rows);
    chunk_stats_kernel<<<chunks, SNT, 0, st>>>(L, V, invT, W.part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (plain) {
        chunk_draw_kernel<<<rows, SNT, 0, st>>>(L, V, invT, W.part, u, out);
        return hipGetLastError();
    }
    if (topk) {
        chunk_topk_kernel<<<chunks, SNT, 0, st>>>(L, V, invT, top_k, W);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        const SampleArgs a{T, top_k, top_p, min_p};
        topk_draw_kernel<<<rows, SNT, 0, st>>>(V, a, W, u, out);
        return hipGetLastError();
    }
    if (topp) {
        chunk_hist_kernel<<<chunks, SNT, 0, st>>>(L, V, invT, bigk, W);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        row_pick_kernel<<<rows, SNT, 0, st>>>(top_p, bigk ? top_k : 0, W);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        chunk_gather_kernel<<<chunks, SNT, 0, st>>>(L, V, invT, W);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        row_select_kernel<<<rows, SNT, 0, st>>>(L, V, invT, bigk, W);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if (bigk) {
        chunk_keptcount_kernel<<<chunks, SNT, 0, st>>>(L, V, invT, W);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        chunk_compact_kernel<<<chunks, SNT, 0, st>>>(L, V, invT, W);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        const SampleArgs a{T, top_k, top_p, min_p};
        cand_draw_kernel<<<rows, SNT, 0, st>>>(V, a, W, u, out);
        return hipGetLastError();
    }
    for (int stage = topp ? 0 : 1; stage <= (minp ? 1 : 0); stage++) {
        chunk_keptsum_kernel<<<chunks, SNT, 0, st>>>(L, V, invT, topp, stage, min_p, W);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    keep_draw_kernel<<<rows, SNT, 0, st>>>(L, V, invT, topp, minp, min_p, W, u, out);
    return hipGetLastError();
}

hipError_t launch_penalties(float *L, int rows, int V, const int32_t *tok, int n_tok, int64_t tok_stride,
                            float presence, float repetition, hipStream_t st) {
    if (n_tok == 0 || (presence == 0.f && repetition == 1.0f)) return hipSuccess;
    penalty_kernel<<<rows, PEN_NT, 0, st>>>(L, V, tok, n_tok, tok_stride, presence, repetition);
    return hipGetLastError();
}
