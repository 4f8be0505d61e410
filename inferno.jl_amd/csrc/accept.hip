// LM-head softmax statistics and speculative acceptance on gfx950.
//
// Softmax statistics are two-level: a grid of (V-chunk, row) workgroups
// writes a partial (max, sum exp(z - max)) per chunk of 4096 entries (each
// thread holds its 16 entries in registers: one round of loads); consumers
// merge the partials in chunk order (deterministic). z = L / T as the
// reference computes logits ./ temperature (src/ModelCPU.jl:1130-1132).
//
// Probabilities, their sums and every prefix sum of the draws are fp64:
// exp((double)z - max) with the exponent's argument exact, sums and scans
// in double. A draw over 151936 entries of mass ~1e-5 each moves when the
// cumulative sum errs by a fraction of one entry's mass; fp32 sums err by
// ~1e-7 of the total, which moved ~0.4 % of residual draws against the
// exact prefix sums, fp64 ones by ~1e-15.
//
// Acceptance (src/SpeculativeDecoding.jl:75-104 with explicit uniforms) runs
// as four launches: statistics of every target and draft row; one wave per
// verify step for the ratio tests (lane i judges draft i); per (chunk, step)
// sums of the sampling weights (residual or bonus distribution); and one
// workgroup per step that locates u * S by a chunk prefix, then a round
// prefix, then a wave scan inside the chunk. Every partial sum is formed in
// one fixed order, and the running value C_j at the last entry of a round
// or chunk equals the prefix the next level starts from, so the search
// always lands inside the level it selected.
#include "common.h"

namespace {

constexpr int CHUNK = 4096;      // V elements per partial
constexpr int NT = 256;          // threads per workgroup

// exp(z - m) for an entry's probability: the difference rounded to fp32 plus
// its exact rounding error (two-sum), the accurate fp32 exp of the former
// times 1 + the latter (relative error ~1e-7, independent across entries;
// summed in double, such errors move a prefix sum by far less than one
// entry's mass). Non-finite differences give exp's own result.
__device__ __forceinline__ double dexp(float z, float m) {
    const float d = z - m;
    const float bz = d - z;
    const float err = (z - (d - bz)) + (-m - bz);
    const float e = expf(d);
    return (double)(e > 0.f && e < __builtin_huge_valf() ? fmaf(e, err, e) : e);
}
// exp(m2 - m) in double for rescaling a partial sum (a few per row).
__device__ __forceinline__ double rescale(float m2, float m) { return exp((double)m2 - (double)m); }

// Partial softmax statistics: max z and sum exp(z - max) (16 bytes).
struct __align__(16) MS {
    float m, pad;
    double s;
};
__device__ __forceinline__ MS make_ms(float m, double s) {
    MS r;
    r.m = m;
    r.pad = 0.f;
    r.s = s;
    return r;
}

// (m, s) merged with (m2, s2): the smaller maximum's sum rescaled. The same
// bits whichever argument comes first (a single exp, then a commutative
// add); a NaN or +Inf entry makes the sum NaN, as exp(Inf - Inf) does.
__device__ __forceinline__ void merge_ms(float &m, double &s, float m2, double s2) {
    if (m2 == -__builtin_huge_valf()) return;
    if (m == -__builtin_huge_valf()) { m = m2; s = s2; return; }
    if (m >= m2) {
        s = s + s2 * rescale(m2, m);
    } else {
        s = s * rescale(m, m2) + s2;
        m = m2;
    }
}

// Cross-lane moves on the VALU (DPP) and, across rows, one swizzle or
// bpermute: partner of lane l at butterfly level o (l ^ o for o = 1, 2, 16,
// 32; the mirror 7 - l within 8 for o = 4 and 15 - l within 16 for o = 8,
// which pair the same lanes' results once the lower levels have made every
// quad (octet) uniform).
template <int CTRL> __device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int O> __device__ __forceinline__ float partner(float v) {
    if constexpr (O == 1) return dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
    if constexpr (O == 2) return dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
    if constexpr (O == 4) return dpp_mov<0x141>(v);  // row_half_mirror
    if constexpr (O == 8) return dpp_mov<0x140>(v);  // row_mirror
    if constexpr (O == 16)                           // swizzle: xor 16 within 32
        return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
    return __shfl_xor(v, 32);
}
template <int O> __device__ __forceinline__ double partner_d(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = __builtin_bit_cast(uint32_t, partner<O>(__builtin_bit_cast(float, (uint32_t)b)));
    const uint32_t hi = __builtin_bit_cast(uint32_t, partner<O>(__builtin_bit_cast(float, (uint32_t)(b >> 32))));
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Butterfly merge of one (max, sum) pair per lane (levels 1, 2, 4, 8, 16,
// 32 as above); merge_ms is symmetric, so both partners compute the same
// bits and every lane ends with the same value.
template <int O> __device__ __forceinline__ void merge_level(float &m, double &s) {
    const float m2 = partner<O>(m);
    const double s2 = partner_d<O>(s);
    merge_ms(m, s, m2, s2);
}
__device__ __forceinline__ MS wave_merge_pairs(float m, double s) {
    merge_level<1>(m, s);
    merge_level<2>(m, s);
    merge_level<4>(m, s);
    merge_level<8>(m, s);
    merge_level<16>(m, s);
    merge_level<32>(m, s);
    return make_ms(m, s);
}

// Block-wide (max, sum) merge of per-thread pairs.
__device__ void block_merge_ms(float &m, double &s, MS *sh) {
    const MS wv = wave_merge_pairs(m, s);
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    if (l == 0) sh[w] = wv;
    __syncthreads();
    if (threadIdx.x == 0) {
        float M = sh[0].m;
        double S = sh[0].s;
        for (int i = 1; i < (int)(blockDim.x >> 6); i++) merge_ms(M, S, sh[i].m, sh[i].s);
        sh[0] = make_ms(M, S);
    }
    __syncthreads();
    m = sh[0].m;
    s = sh[0].s;
    __syncthreads();
}

// partial[row][chunk] = (max z, sum exp(z - max)). Rows [0, rows1) come from
// L1 at temperature T1, except every period-th row (r % period == period - 1,
// the bonus row of a verify step) at T_last; rows [rows1, ..) come from L2 at
// T2. Entry c * CHUNK + i * NT + t is thread t's i-th value.
constexpr int PER = CHUNK / NT;  // 16 entries per thread
__global__ __launch_bounds__(NT) void stats_partial_kernel(const float *__restrict__ L1, int rows1, float T1,
                                                           float T_last, int period, const float *__restrict__ L2,
                                                           float T2, int V, int nchunk, MS *__restrict__ part) {
    __shared__ MS sh[NT / 64];
    const int chunk = blockIdx.x, row = blockIdx.y;
    const bool first = row < rows1;
    const float Tr = first ? ((period > 0 && row % period == period - 1) ? T_last : T1) : T2;
    const float *src = first ? L1 + (size_t)row * V : L2 + (size_t)(row - rows1) * V;
    const int j0 = chunk * CHUNK;
    float z[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int j = j0 + i * NT + threadIdx.x;
        z[i] = j < V ? src[j] / Tr : -__builtin_huge_valf();
    }
    float m = -__builtin_huge_valf();
#pragma unroll
    for (int i = 0; i < PER; i++) m = fmaxf(m, z[i]);
    double s = 0.0;
    if (m > -__builtin_huge_valf()) {
#pragma unroll
        for (int i = 0; i < PER; i++) s += dexp(z[i], m);
    }
    block_merge_ms(m, s, sh);
    if (threadIdx.x == 0) part[(size_t)row * nchunk + chunk] = make_ms(m, s);
}

// Sequential merge of a row's chunk partials (chunk order), the loads issued
// eight at a time.
__device__ __forceinline__ MS merge_row(const MS *part, int nchunk) {
    float m = -__builtin_huge_valf();
    double s = 0.0;
    for (int c = 0; c < nchunk; c += 8) {
        MS v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = part[min(c + j, nchunk - 1)];
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (c + j < nchunk) merge_ms(m, s, v[j].m, v[j].s);
    }
    return make_ms(m, s);
}

// Merge of a row's chunk partials by one wave: lane l folds chunks l, l+64,
// ... in order, then the butterfly.
__device__ __forceinline__ MS wave_merge_row(const MS *part, int nchunk) {
    const int lane = threadIdx.x & 63;
    float m = -__builtin_huge_valf();
    double s = 0.0;
    for (int c = lane; c < nchunk; c += 64) {
        const MS p = part[c];
        merge_ms(m, s, p.m, p.s);
    }
    return wave_merge_pairs(m, s);
}

__global__ void stats_merge_kernel(const MS *__restrict__ part, int rows, int nchunk, float *__restrict__ zmax,
                                   float *__restrict__ zsum) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const MS ms = merge_row(part + (size_t)r * nchunk, nchunk);
    zmax[r] = ms.m;
    zsum[r] = (float)ms.s;
}

// Sampling distribution of one draw of a verify step, set by the ratio
// tests:
//   kind 0: p_j (target row, temperature Tp)       bonus draw
//   kind 1: max(0, p_j - q_j)  (q: draft row)      standard residual
//   kind 2: max(0, p_j - qs)   (qs: scalar q_i)    reference residual
//   kind 3: the bonus token drawn beforehand by the filtered sampler
//           (top-k / top-p / min-p on target row k at T with u_bonus)
//   kind -1: invalid draft id (out_n = -1, nothing drawn)
//   kind -2: no draw in this slot
// fallback when the weights sum to 0: 1 = draw from p (standard mode),
// 2 = return V - 1 (the reference's all-NaN residual, length(probs)).
// pos: the index of the drawn token in the step's out_tok row. A step has
// one draw slot in the standard mode and two in the reference mode, whose
// second slot holds the bonus the reference appends after a rejection of
// the last draft (src/SpeculativeDecoding.jl:100: length(accepted) == gamma).
struct Decision {
    int kind, n, prow, qrow, fallback, pos;
    float Tp, mp, Tq, mq, u, pad;
    double isp, isq, qs;  // 1 / (sum of exp) of the p and q rows
};
__host__ __device__ constexpr int draw_slots(int mode) { return mode == 1 ? 2 : 1; }

// Inclusive scan over the 64 lanes of a wave (fixed association): a
// Hillis-Steele scan inside each row of 16 (DPP row shifts by 1, 2, 4, 8;
// lanes shifted in from outside the row read 0), then row r + 1 adds the
// total of row r (row broadcast of lane 15 into rows 1 and 3) and rows 2, 3
// add the total of rows 0, 1 (row broadcast of lane 31).
// A double moves as its two halves.
template <int CTRL, int ROWS> __device__ __forceinline__ double dpp_row(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, ROWS, 0xF, true);
    const uint32_t hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, ROWS, 0xF, true);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ double wave_scan(double v) {
    v += dpp_row<0x111, 0xF>(v);  // row_shr:1
    v += dpp_row<0x112, 0xF>(v);  // row_shr:2
    v += dpp_row<0x114, 0xF>(v);  // row_shr:4
    v += dpp_row<0x118, 0xF>(v);  // row_shr:8
    v += dpp_row<0x142, 0xA>(v);  // row_bcast:15 into rows 1, 3
    v += dpp_row<0x143, 0xC>(v);  // row_bcast:31 into rows 2, 3
    return v;
}

// Ratio tests of one verify step by a whole workgroup: the statistics of the
// step's 2k + 1 rows are merged first (row r by wave r % 4: the loads of
// all its rows in flight before any merge; kept in LDS), then lane i of wave
// 0 judges draft i (groups of 64 lanes for k > 64). The result is the
// decision of each draw slot (s_dec[0], s_dec[1]); with publish, the
// accepted drafts, out_n and the decisions are also written out. Every
// workgroup that calls it for the same step computes the same decision.
constexpr int DECIDE_MAX_ROWS = 255;  // 2k + 1, k <= 127
constexpr int DECIDE_WAVES = NT / 64;
__device__ void decide_block(const float *__restrict__ tgt, const float *__restrict__ drf,
                             const int32_t *__restrict__ draft_tok, int k, int V, float T,
                             const float *__restrict__ u_acc, const float *__restrict__ u_res,
                             const float *__restrict__ u_bonus, int mode, const MS *__restrict__ part,
                             int nchunk, int step, int steps, bool publish, const int32_t *__restrict__ bonus_pre,
                             int32_t *__restrict__ out_tok, int32_t *__restrict__ out_n,
                             Decision *__restrict__ dec, MS *ms, Decision *s_dec) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const float *Lt = tgt + (size_t)step * (k + 1) * V;
    const float *Ld = drf + (size_t)step * k * V;
    const int32_t *dt = draft_tok + (size_t)step * k;
    const MS *Pt = part + (size_t)step * (k + 1) * nchunk;
    const MS *Pd = part + ((size_t)steps * (k + 1) + (size_t)step * k) * nchunk;
    const float Tr = mode == 0 ? T : 1.0f;
    // wave 0: the first 64 drafts' ids and uniforms, then (once the ids are
    // in) their two logits, issued before the merges
    const bool has0 = wave == 0 && lane < k;
    const int x0 = has0 ? dt[lane] : 0;
    const float ua0 = has0 ? u_acc[(size_t)step * k + lane] : 0.f;
    const int nrows = 2 * k + 1;
    float lx0 = 0.f, dx0 = 0.f;
    // rows wave, wave + W, ..: in batches of 8 per wave
    for (int r0 = wave; r0 < nrows; r0 += 8 * DECIDE_WAVES) {
        MS pv[8][2];
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const int r = min(r0 + b * DECIDE_WAVES, nrows - 1);
            const MS *row = r <= k ? Pt + (size_t)r * nchunk : Pd + (size_t)(r - k - 1) * nchunk;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int c = lane + 64 * h;
                pv[b][h] = c < nchunk ? row[c] : make_ms(-__builtin_huge_valf(), 0.0);
            }
        }
        if (r0 == 0 && has0 && x0 >= 0 && x0 < V) {
            lx0 = Lt[(size_t)lane * V + x0];
            dx0 = Ld[(size_t)lane * V + x0];
        }
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const int r = r0 + b * DECIDE_WAVES;
            if (r >= nrows) break;
            MS v;
            if (nchunk <= 128) {
                float m = -__builtin_huge_valf();
                double sm = 0.0;
                merge_ms(m, sm, pv[b][0].m, pv[b][0].s);
                merge_ms(m, sm, pv[b][1].m, pv[b][1].s);
                v = wave_merge_pairs(m, sm);
            } else {
                v = wave_merge_row(r <= k ? Pt + (size_t)r * nchunk : Pd + (size_t)(r - k - 1) * nchunk, nchunk);
            }
            if (lane == 0) ms[r] = v;
        }
    }
    __syncthreads();
    if (wave == 0) {
        int first = k;  // first draft that is invalid or rejected
        bool invalid = false;
        double f_q = 0.0;
        for (int base = 0; base < k && first == k; base += 64) {
            const int i = base + lane;
            bool bad = false, inv = false;
            double q = 0.0;
            if (i < k) {
                const bool pre = base == 0;  // the first 64 were fetched up front
                const int x = pre ? x0 : dt[i];
                if (x < 0 || x >= V) {
                    bad = inv = true;
                } else {
                    const MS pt = ms[i], pd = ms[k + 1 + i];
                    const double p = dexp((pre ? lx0 : Lt[(size_t)i * V + x]) / Tr, pt.m) / pt.s;
                    q = dexp((pre ? dx0 : Ld[(size_t)i * V + x]) / Tr, pd.m) / pd.s;
                    const double ratio = q > 0.0 ? fmin(1.0, p / q) : 1.0;
                    bad = !((double)(pre ? ua0 : u_acc[(size_t)step * k + i]) < ratio);
                }
            }
            const uint64_t m = __ballot(bad);
            if (m) {
                const int f = __ffsll((unsigned long long)m) - 1;
                first = base + f;
                invalid = __shfl(inv ? 1 : 0, f) != 0;
                f_q = __shfl(q, f);
            }
        }
        // accepted drafts
        if (publish)
            for (int i = lane; i < first; i += 64) out_tok[(size_t)step * (k + 1) + i] = dt[i];
        if (lane == 0) {
            const int nd = draw_slots(mode);
            Decision D{}, D2{};
            D2.kind = -2;
            if (invalid) {
                D.kind = -1;
                D.n = -1;
            } else {
                D.n = first;
                D.pos = first;
                if (first < k) {
                    const MS pt = ms[first], pd = ms[k + 1 + first];
                    D.kind = mode == 0 ? 1 : 2;
                    D.prow = first;
                    D.qrow = first;
                    D.Tp = Tr; D.mp = pt.m; D.isp = 1.0 / pt.s;
                    D.Tq = Tr; D.mq = pd.m; D.isq = 1.0 / pd.s;
                    D.qs = f_q;
                    D.u = u_res[step];
                    D.fallback = mode == 0 ? 1 : 2;
                    if (mode == 1 && first == k - 1) {  // the reference's bonus after the residual
                        const MS pk = ms[k];
                        D2.kind = bonus_pre ? 3 : 0;
                        D2.n = first;
                        D2.pos = first + 1;
                        D2.prow = k;
                        D2.Tp = T; D2.mp = pk.m; D2.isp = 1.0 / pk.s;
                        D2.Tq = T; D2.mq = 0.f; D2.isq = 1.0;
                        D2.u = u_bonus[step];
                        D2.fallback = 2;
                    }
                } else {
                    const MS pt = ms[k];
                    D.kind = bonus_pre ? 3 : 0;
                    D.prow = k;
                    D.qrow = 0;
                    D.Tp = T; D.mp = pt.m; D.isp = 1.0 / pt.s;
                    D.Tq = T; D.mq = 0.f; D.isq = 1.0; D.qs = 0.0;
                    D.u = u_bonus[step];
                    D.fallback = 2;
                }
            }
            s_dec[0] = D;
            s_dec[1] = D2;
            if (publish) {
                out_n[step] = D.n;
                dec[(size_t)step * nd] = D;
                if (nd > 1) dec[(size_t)step * nd + 1] = D2;
            }
        }
    }
    __syncthreads();
}

// Sampling weights of the PER x NT entries of chunk c: thread t holds entries
// c * CHUNK + r * NT + t (r < PER) of w and, for the standard residual, of p.
// Per round r: wave inclusive scans, round total R_r = ((T0 + T1) + T2) + T3
// of the four wave totals.
struct ChunkScan {
    double cw[PER];  // wave-inclusive scans of the weights
    double R[PER];   // round totals (uniform)
};

__device__ void chunk_scan(const Decision &D, const float *lt, const float *ld, int V, int c, bool use_p,
                           ChunkScan &cs, double *sh /* [PER][4] */) {
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    // every load of the chunk in flight before any arithmetic
    float lv[PER], dv[PER];
    const bool need_q = !use_p && D.kind == 1;
#pragma unroll
    for (int r = 0; r < PER; r++) {
        const int j = min(c * CHUNK + r * NT + t, V - 1);
        lv[r] = lt[j];
        dv[r] = need_q ? ld[j] : 0.f;
    }
#pragma unroll
    for (int r = 0; r < PER; r++) {
        const int j = c * CHUNK + r * NT + t;
        double w = 0.0;
        if (j < V) {
            const double p = dexp(lv[r] / D.Tp, D.mp) * D.isp;
            if (use_p || D.kind == 0) w = p;
            else w = fmax(p - (D.kind == 1 ? dexp(dv[r] / D.Tq, D.mq) * D.isq : D.qs), 0.0);
        }
        cs.cw[r] = wave_scan(w);
        if (lane == 63) sh[r * 4 + wave] = cs.cw[r];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < PER; r++) cs.R[r] = ((sh[r * 4] + sh[r * 4 + 1]) + sh[r * 4 + 2]) + sh[r * 4 + 3];
    __syncthreads();
}

// The decision of verify step `step` (decide_block, computed by every
// workgroup; the first one publishes it), then csum[step][slot][c] = the
// sum of w over chunk c: the sequential sum of its round totals (grid: x
// chunk, y step, z draw slot).
__global__ __launch_bounds__(NT) void decide_sum_kernel(const float *__restrict__ tgt, const float *__restrict__ drf,
                                                        const int32_t *__restrict__ draft_tok, int k, int V, float T,
                                                        const float *__restrict__ u_acc,
                                                        const float *__restrict__ u_res,
                                                        const float *__restrict__ u_bonus, int mode,
                                                        const MS *__restrict__ part, int nchunk,
                                                        const int32_t *__restrict__ bonus_pre,
                                                        int32_t *__restrict__ out_tok, int32_t *__restrict__ out_n,
                                                        Decision *__restrict__ dec, double *__restrict__ csum) {
    __shared__ double sh[PER * 4];
    __shared__ MS ms[DECIDE_MAX_ROWS];
    __shared__ Decision s_dec[2];
    const int c = blockIdx.x, step = blockIdx.y;
    decide_block(tgt, drf, draft_tok, k, V, T, u_acc, u_res, u_bonus, mode, part, nchunk, step, gridDim.y,
                 c == 0 && blockIdx.z == 0, bonus_pre, out_tok, out_n, dec, ms, s_dec);
    const size_t slot = (size_t)step * gridDim.z + blockIdx.z;
    const Decision D = s_dec[blockIdx.z];
    if (D.kind < 0 || D.kind == 3) return;
    const float *lt = tgt + ((size_t)step * (k + 1) + D.prow) * V;
    const float *ld = D.kind == 1 ? drf + ((size_t)step * k + D.qrow) * V : nullptr;
    ChunkScan cs;
    chunk_scan(D, lt, ld, V, c, false, cs, sh);
    double sw = 0.0;
#pragma unroll
    for (int r = 0; r < PER; r++) sw += cs.R[r];
    if (threadIdx.x == 0) csum[slot * nchunk + c] = sw;
}

// First j with u * S <= C_j, where C_j = before(chunk) + (P_r + (off_w +
// scan)): chunk prefix, then round prefix, then lane. When the weights sum
// to zero the standard mode draws from p (its chunk sums are formed here, in
// the same order), the reference mode returns V - 1.
constexpr int MAX_CHUNKS = 1024;
__global__ __launch_bounds__(NT) void sample_kernel(const float *__restrict__ tgt, const float *__restrict__ drf,
                                                    int k, int V, const Decision *__restrict__ dec, int nchunk,
                                                    const double *__restrict__ csum,
                                                    const int32_t *__restrict__ bonus_pre,
                                                    int32_t *__restrict__ out_tok) {
    __shared__ double sh[PER * 4];
    __shared__ double s_psum[MAX_CHUNKS];
    __shared__ double s_csum[MAX_CHUNKS];
    __shared__ double s_before, s_target;
    __shared__ int s_chunk, s_usep, s_tok;
    __shared__ int s_first[NT / 64];
    const int step = blockIdx.x, t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const size_t slot = (size_t)step * gridDim.y + blockIdx.y;
    const Decision D = dec[slot];
    if (D.kind < 0) return;
    if (D.kind == 3) {
        if (t == 0) out_tok[(size_t)step * (k + 1) + D.pos] = bonus_pre[step];
        return;
    }
    const double *cw = csum + slot * nchunk;
    const float *lt = tgt + ((size_t)step * (k + 1) + D.prow) * V;
    const float *ld = D.kind == 1 ? drf + ((size_t)step * k + D.qrow) * V : nullptr;
    for (int c = t; c < nchunk; c += NT) s_csum[c] = cw[c];
    __syncthreads();
    if (t == 0) {
        double S = 0.0;
        for (int c = 0; c < nchunk; c++) S += s_csum[c];
        s_usep = 0;
        s_tok = -1;
        if (!(S > 0.0)) {
            if (D.fallback == 1) s_usep = 1;
            else s_tok = V - 1;
        }
    }
    __syncthreads();
    if (s_tok >= 0) {
        if (t == 0) out_tok[(size_t)step * (k + 1) + D.pos] = s_tok;
        return;
    }
    const bool usep = s_usep != 0;
    ChunkScan cs;
    if (usep) {
        for (int c = 0; c < nchunk; c++) {
            chunk_scan(D, lt, ld, V, c, true, cs, sh);
            if (t == 0) {
                double sp = 0.0;
#pragma unroll
                for (int r = 0; r < PER; r++) sp += cs.R[r];
                s_psum[c] = sp;
            }
        }
        __syncthreads();
    }
    if (t == 0) {
        double S = 0.0;
        for (int c = 0; c < nchunk; c++) S += usep ? s_psum[c] : s_csum[c];
        const double target = (double)D.u * S;
        double before = 0.0;
        int chunk = nchunk - 1;
        for (int c = 0; c < nchunk; c++) {
            const double nb = before + (usep ? s_psum[c] : s_csum[c]);
            if (target <= nb) { chunk = c; break; }
            before = nb;
        }
        s_before = before;
        s_target = target;
        s_chunk = chunk;
    }
    __syncthreads();
    const int c = s_chunk;
    const double before = s_before, target = s_target;
    chunk_scan(D, lt, ld, V, c, usep, cs, sh);
    // round: first r with target <= before + P_{r+1}
    double P = 0.0, Pr = 0.0;
    int rr = -1;
#pragma unroll
    for (int r = 0; r < PER; r++) {
        const double Pn = P + cs.R[r];
        if (rr < 0 && target <= before + Pn) { rr = r; Pr = P; }
        P = Pn;
    }
    if (rr < 0) {  // unreachable: the chunk total bounds the target
        rr = PER - 1;
        Pr = P - cs.R[PER - 1];
    }
    double cw_rr = 0.0;
#pragma unroll
    for (int r = 0; r < PER; r++)
        if (r == rr) cw_rr = cs.cw[r];
    if (lane == 63) sh[wave] = cw_rr;
    __syncthreads();
    double off = 0.0;
    for (int w = 0; w < wave; w++) off += sh[w];
    const double C = before + (Pr + (off + cw_rr));
    const int j = c * CHUNK + rr * NT + t;
    const bool hit = j < V && target <= C;
    const uint64_t m = __ballot(hit);
    if (lane == 0) s_first[wave] = m ? (wave * 64 + __ffsll((unsigned long long)m) - 1) : NT;
    __syncthreads();
    if (t == 0) {
        int f = NT;
        for (int w = 0; w < NT / 64; w++) f = min(f, s_first[w]);
        const int tok = min(c * CHUNK + rr * NT + (f < NT ? f : NT - 1), V - 1);
        out_tok[(size_t)step * (k + 1) + D.pos] = tok;
    }
}

// Julia's findmax order (the argmax of mtp_verify_step!): isless, the total
// order -Inf < ... < -0.0 < +0.0 < ... < +Inf < NaN; among equals (and among
// NaNs) the first index wins. `beats` is the strict order, `first_of` picks
// (value, index) pairs under it.
__device__ __forceinline__ bool beats(float a, float b) {
    if (isnan(a) || isnan(b)) return isnan(a) && !isnan(b);
    return a > b || (a == b && signbit(b) && !signbit(a));
}
__device__ __forceinline__ bool first_of(float v2, int i2, float bv, int bi) {
    return beats(v2, bv) || (!beats(bv, v2) && i2 < bi);
}

// Partial first-index argmax per (chunk, row). Every thread of a non-empty
// chunk holds a real index (a row of -Inf gives its first index).
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
        if (first_of(v, j, bv, bi)) { bv = v; bi = j; }
    }
    for (int o = 32; o > 0; o >>= 1) {
        const float v2 = __shfl_xor(bv, o);
        const int i2 = __shfl_xor(bi, o);
        if (first_of(v2, i2, bv, bi)) { bv = v2; bi = i2; }
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { sv[w] = bv; si[w] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < NT / 64; i++)
            if (first_of(sv[i], si[i], bv, bi)) { bv = sv[i]; bi = si[i]; }
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
        for (int c = 1; c < nchunk; c++)  // chunks ascend: the strict order keeps the first
            if (beats(p[c].x, bv)) { bv = p[c].x; bi = __float_as_int(p[c].y); }
        if (out_argmax) out_argmax[(size_t)step * (k + 1) + i] = bi;
        if (i < k && go) {
            if (bi == draft_tok[(size_t)step * k + i]) n++;
            else go = false;
        }
    }
    out_n[step] = n;
}

// Tree walk: the workgroup first merges the statistics of every row (target
// rows then draft rows) into ms, then tests every node in parallel (the test
// of node i reads only its parent's rows and its own token: pass = u_i <
// min(1, p/q)), then one thread walks the nodes in index order (parent[i] <
// i) with integers only: st[i] = depth of i if i and all its ancestors
// passed, else -1; the deepest accepted node, smallest index on ties, ends
// the path. Node state lives in LDS up to TREE_LDS nodes (in the workspace
// beyond that).
constexpr int TREE_LDS = 4096;
__global__ __launch_bounds__(NT) void tree_kernel(const float *__restrict__ tgt, const float *__restrict__ drf,
                                                  const int32_t *__restrict__ tok, const int32_t *__restrict__ parent,
                                                  int n, int V, float T, const float *__restrict__ u,
                                                  const MS *__restrict__ part, int nchunk, MS *__restrict__ ms,
                                                  int32_t *__restrict__ out_path, int32_t *__restrict__ out_len,
                                                  int32_t *__restrict__ wsi) {
    __shared__ int32_t s_par[TREE_LDS], s_st[TREE_LDS];
    __shared__ int8_t s_pass[TREE_LDS];
    const bool in_lds = n <= TREE_LDS;
    int32_t *par = in_lds ? s_par : wsi;
    int32_t *st = in_lds ? s_st : wsi + n;
    int8_t *pass = in_lds ? s_pass : (int8_t *)(wsi + 2 * n);
    for (int r = threadIdx.x; r < 2 * n; r += blockDim.x) ms[r] = merge_row(part + (size_t)r * nchunk, nchunk);
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int p = parent[i];
        const int x = tok[i];
        par[i] = p;
        int8_t r = 1;  // (the root is accepted)
        if (i > 0) {
            if (p < 0 || p >= i || x < 0 || x >= V) {
                r = -1;  // malformed node: reported as out_len = -1
            } else {
                const MS pt = ms[p];
                const MS pd = ms[n + p];
                const double pp = dexp(tgt[(size_t)p * V + x] / T, pt.m) / pt.s;
                const double qq = dexp(drf[(size_t)p * V + x] / T, pd.m) / pd.s;
                const double ratio = qq > 0.0 ? fmin(1.0, pp / qq) : 1.0;
                r = (double)u[i] < ratio ? 1 : 0;
            }
        }
        pass[i] = r;
    }
    __syncthreads();
    if (threadIdx.x != 0) return;
    st[0] = 0;
    int best = 0;
    for (int i = 1; i < n; i++) {
        const int r = pass[i];
        if (r < 0) {
            *out_len = -1;
            return;
        }
        const int sp = st[par[i]];
        const int d = (sp >= 0 && r) ? sp + 1 : -1;
        st[i] = d;
        if (d > st[best]) best = i;
    }
    const int len = st[best] + 1;
    int v = best;
    for (int d = len - 1; d >= 0; d--) {
        out_path[d] = v;
        v = d > 0 ? par[v] : 0;
    }
    *out_len = len;
}

}  // namespace

int accept_nchunk(int V) { return (V + CHUNK - 1) / CHUNK; }

// Bytes of one softmax partial (MS) of a (row, chunk); a first-argmax
// partial (float2) fits in the same slot.
size_t accept_part_bytes() { return sizeof(MS); }

hipError_t launch_stats(const float *L, int rows, int V, float T, float T_last, int period, void *part,
                        hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    const int nc = accept_nchunk(V);
    stats_partial_kernel<<<dim3(nc, rows), NT, 0, st>>>(L, rows, T, T_last, period, L, T, V, nc, (MS *)part);
    return hipGetLastError();
}

hipError_t launch_stats_merge(const void *part, int rows, int V, float *zmax, float *zsum, hipStream_t st) {
    const int nc = accept_nchunk(V);
    stats_merge_kernel<<<(rows + 63) / 64, 64, 0, st>>>((const MS *)part, rows, nc, zmax, zsum);
    return hipGetLastError();
}

size_t spec_accept_ws(int steps, int k, int V) {
    const size_t nc = accept_nchunk(V);
    return (size_t)steps * (2 * k + 1) * nc * sizeof(MS) + (size_t)steps * 2 * sizeof(Decision) +
           (size_t)steps * 2 * nc * sizeof(double) + 256;
}

// ws: MS part[steps*(k+1) + steps*k][nchunk], Decision dec[steps][slots],
// double csum[steps][slots][nchunk] (slots = draw_slots(mode)). bonus_pre
// (nullptr: none): each step's bonus token, drawn beforehand from target row
// k by the filtered sampler; bonus draws then copy it.
hipError_t launch_spec_accept(const float *tgt, const float *drf, const int32_t *draft_tok, int steps, int k,
                              int V, float T, const float *u_acc, const float *u_res, const float *u_bonus,
                              int mode, const int32_t *bonus_pre, int32_t *out_tok, int32_t *out_n, void *ws,
                              hipStream_t st) {
    const int nc = accept_nchunk(V);
    const float Tr = mode == 0 ? T : 1.0f;
    const int nd = draw_slots(mode);
    MS *part = (MS *)ws;
    Decision *dec = (Decision *)(part + (size_t)steps * (2 * k + 1) * nc);
    double *csum = (double *)(dec + (size_t)steps * nd);
    stats_partial_kernel<<<dim3(nc, steps * (2 * k + 1)), NT, 0, st>>>(tgt, steps * (k + 1), Tr, T, k + 1,
                                                                      drf, Tr, V, nc, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    decide_sum_kernel<<<dim3(nc, steps, nd), NT, 0, st>>>(tgt, drf, draft_tok, k, V, T, u_acc, u_res, u_bonus,
                                                          mode, part, nc, bonus_pre, out_tok, out_n, dec, csum);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    sample_kernel<<<dim3(steps, nd), NT, 0, st>>>(tgt, drf, k, V, dec, nc, csum, bonus_pre, out_tok);
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

// ws: MS part[2n][nchunk] (target rows then draft rows), MS ms[2n] (their
// merged statistics), then (above TREE_LDS nodes) int32 [2n] and int8 [n].
size_t tree_ws(int n, int V) {
    return ((size_t)2 * n * accept_nchunk(V) + 2 * (size_t)n) * sizeof(MS) + (size_t)n * 9 + 256;
}

hipError_t launch_tree(const float *tgt, const float *drf, const int32_t *tok, const int32_t *parent, int n, int V,
                       float T, const float *u, void *ws, int32_t *out_path, int32_t *out_len, hipStream_t st) {
    const int nc = accept_nchunk(V);
    MS *part = (MS *)ws;
    MS *ms = part + (size_t)2 * n * nc;
    int32_t *wsi = (int32_t *)(ms + 2 * n);
    stats_partial_kernel<<<dim3(nc, 2 * n), NT, 0, st>>>(tgt, n, T, T, 0, drf, T, V, nc, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    tree_kernel<<<1, NT, 0, st>>>(tgt, drf, tok, parent, n, V, T, u, part, nc, ms, out_path, out_len, wsi);
    return hipGetLastError();
}
