// Applying a verify step's outcome on the device. The reference has no
// rollback (src/SpeculativeDecoding.jl:69-70 re-feeds the target without
// restoring its caches; KV writes at src/ModelCPU.jl:245-258, SSM state at
// :476-530). The accept kernels leave n = out_n[s] (drafts accepted, -1 for
// an invalid draft id) in device memory; these kernels read it there, so a
// captured verify step needs no host round trip:
//  * commit_state: state[s] = snapshot n of step s - a recurrent state as it
//    stood after the verify forward consumed x_0, d_1 .. d_n (the forward
//    keeps a snapshot after each of its k + 1 positions);
//  * advance_len: len[s] += n + 1 - a KV cache keeps the entries of the
//    n + 1 positions that stand; the rest are overwritten by the next step.
// n = -1 (or n > k) leaves the state and the length as they are.
#include "common.h"

namespace {

__global__ __launch_bounds__(256) void commit_state_kernel(uint32_t *__restrict__ state,
                                                           const uint32_t *__restrict__ snap, int64_t words,
                                                           int64_t snap_stride, int k,
                                                           const int32_t *__restrict__ n_acc,
                                                           int64_t state_step, int64_t snap_step) {
    const int s = blockIdx.y;
    const int n = n_acc[s];
    if (n < 0 || n > k) return;
    uint32_t *dst = state + (size_t)s * state_step;
    const uint32_t *src = snap + (size_t)s * snap_step + (size_t)n * snap_stride;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < words; i += (int64_t)gridDim.x * 256) dst[i] = src[i];
}

__global__ void advance_len_kernel(int32_t *__restrict__ len, const int32_t *__restrict__ n_acc, int steps) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s < steps && n_acc[s] >= 0) len[s] += n_acc[s] + 1;
}

}  // namespace

// (strides and sizes in 4-byte words)
hipError_t launch_commit_state(void *state, const void *snap, int64_t words, int64_t snap_stride, int k,
                               const int32_t *n_acc, int steps, int64_t state_step, int64_t snap_step,
                               hipStream_t st) {
    const int64_t blocks = (words + 255) / 256;
    const dim3 grid((unsigned)(blocks < 1024 ? (blocks > 0 ? blocks : 1) : 1024), (unsigned)steps);
    commit_state_kernel<<<grid, 256, 0, st>>>((uint32_t *)state, (const uint32_t *)snap, words, snap_stride, k,
                                              n_acc, state_step, snap_step);
    return hipGetLastError();
}

hipError_t launch_advance_len(int32_t *len, const int32_t *n_acc, int steps, hipStream_t st) {
    advance_len_kernel<<<(steps + 255) / 256, 256, 0, st>>>(len, n_acc, steps);
    return hipGetLastError();
}
