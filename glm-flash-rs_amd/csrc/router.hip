// Router and combine around the expert path (the reference runs them as precompiled Triton kernels `topk` and
// `combine`, glm-flash-rs src/moe.rs:89-100,171-181, whose source is not in its repository). Semantics here are the
// benchmark's: softmax over the routed experts' logits, top-k by logit (ties: lower id), weights renormalised over
// the k picks, the shared expert appended as the last slot with weight 1; combine = the slot-ordered weighted sum.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "route.hpp"

namespace gfr {

__global__ void __launch_bounds__(64) route_kernel(const float* __restrict__ logits, int E, int topk, int shared_id,
                                                   int* __restrict__ picks, float* __restrict__ weights) {
    const int r = blockIdx.x, slots = topk + 1;
    route_token(logits + (size_t)r * E, E, topk, shared_id, picks + (size_t)r * slots, weights + (size_t)r * slots);
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
