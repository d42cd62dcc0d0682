// Router and combine around the expert path (the reference runs them as precompiled Triton kernels `topk` and
// `combine`, glm-flash-rs src/moe.rs:89-100,171-181, whose source is not in its repository). Semantics here are the
// benchmark's: softmax over the routed experts' logits, top-k by logit (ties: lower id), weights renormalised over
// the k picks, the shared expert appended as the last slot with weight 1; combine = the slot-ordered weighted sum.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gfr {

// One wave a row; E <= 64 * 16 logits.
__global__ void __launch_bounds__(64) route_kernel(const float* __restrict__ logits, int E, int topk, int shared_id,
                                                   int* __restrict__ picks, float* __restrict__ weights) {
    constexpr int PER = 16;
    const int r = blockIdx.x, lane = threadIdx.x, slots = topk + 1;
    const float* l = logits + (size_t)r * E;
    float v[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = j * 64 + lane;
        v[j] = e < E ? l[e] : -__builtin_inff();
    }
    uint32_t taken = 0;                        // bit j: expert j * 64 + lane is picked
    int* pk = picks + (size_t)r * slots;
    float* wt = weights + (size_t)r * slots;
    for (int s = 0; s < topk; ++s) {
        float bv = -__builtin_inff();
        int be = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int e = j * 64 + lane;
            if (e < E && !((taken >> j) & 1u) && (v[j] > bv || be == 0x7fffffff)) {
                bv = v[j];
                be = e;
            }
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const float ov = __shfl_xor(bv, m, 64);
            const int oe = __shfl_xor(be, m, 64);
            if (ov > bv || (ov == bv && oe < be)) {
                bv = ov;
                be = oe;
            }
        }
        if ((be & 63) == lane) taken |= 1u << (be >> 6);
        if (lane == 0) {
            pk[s] = be;
            wt[s] = bv;                           // the logit, until the weights below
        }
    }
    if (lane == 0) {
        const float m = wt[0];
        float sum = 0.f;
        for (int s = 0; s < topk; ++s) {
            const float ex = expf(wt[s] - m);
            wt[s] = ex;
            sum += ex;
        }
        for (int s = 0; s < topk; ++s) wt[s] = wt[s] / sum;
        pk[topk] = shared_id;
        wt[topk] = 1.f;
    }
}

// out[r][n] = sum over slots s (in order) of weights[r][s] * y[r * slots + s][n]
__global__ void __launch_bounds__(256) combine_kernel(const float* __restrict__ y, const float* __restrict__ weights,
                                                      int slots, int D, float* __restrict__ out) {
    const int r = blockIdx.y, n = blockIdx.x * 256 + threadIdx.x;
    if (n >= D) return;
    float acc = 0.f;
    for (int s = 0; s < slots; ++s) acc += weights[r * slots + s] * y[((size_t)r * slots + s) * D + n];
    out[(size_t)r * D + n] = acc;
}

}  // namespace gfr

#include "launch.hpp"

namespace gfr {

hipError_t launch_route(hipStream_t s, const float* logits, int rows, int E, int topk, int shared_id, int* picks,
                        float* weights) {
    route_kernel<<<rows, 64, 0, s>>>(logits, E, topk, shared_id, picks, weights);
    return hipGetLastError();
}

hipError_t launch_combine(hipStream_t s, const float* y, const float* weights, int rows, int slots, int D,
                          float* out) {
    combine_kernel<<<dim3((D + 255) / 256, rows), 256, 0, s>>>(y, weights, slots, D, out);
    return hipGetLastError();
}

}  // namespace gfr
