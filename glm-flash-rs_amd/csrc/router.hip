// Router and combine around the expert path (the reference runs them as precompiled Triton kernels `topk` and
// `combine`, glm-flash-rs src/moe.rs:89-100,171-181, whose source is not in its repository). Two gates (route.hpp):
// the benchmark's softmax (top-k by logit, ties: lower id, weights renormalised over the k picks) and GLM's
// sigmoid + bias selection with scaled renormalised weights; the shared expert is appended as the last slot with
// weight 1; combine = the slot-ordered weighted sum.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "route.hpp"

namespace gfr {

__global__ void __launch_bounds__(64) route_kernel(const float* __restrict__ logits, int E, int topk, int shared_id,
                                                   int* __restrict__ picks, float* __restrict__ weights, RouteGate g) {
    const int r = blockIdx.x, slots = topk + 1;
    route_token(logits + (size_t)r * E, E, topk, shared_id, picks + (size_t)r * slots, weights + (size_t)r * slots,
                g);
}

// out[r][n] = sum over slots s (in order) of weights[r][s] * y[r * slots + s][n]; four columns a thread (16-byte
// loads and stores), every slot's row in flight at once. D a multiple of 4.
__global__ void __launch_bounds__(256) combine_kernel(const float* __restrict__ y, const float* __restrict__ weights,
                                                      int slots, int D, float* __restrict__ out) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    constexpr int MAXS = 32;
    const int r = blockIdx.y, n = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (n >= D) return;
    f4v v[MAXS];
#pragma unroll
    for (int s = 0; s < MAXS; ++s)
        if (s < slots) v[s] = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(y + ((size_t)r * slots + s) * D + n));
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int s = 0; s < MAXS; ++s)
        if (s < slots) {
            const float w = weights[r * slots + s];
            acc.x += w * v[s].x;
            acc.y += w * v[s].y;
            acc.z += w * v[s].z;
            acc.w += w * v[s].w;
        }
    *reinterpret_cast<float4*>(out + (size_t)r * D + n) = acc;
}

}  // namespace gfr

#include "launch.hpp"

namespace gfr {

hipError_t launch_route(hipStream_t s, const float* logits, int rows, int E, int topk, int shared_id, int* picks,
                        float* weights, const float* bias, float scale) {
    route_kernel<<<rows, 64, 0, s>>>(logits, E, topk, shared_id, picks, weights, RouteGate{bias, scale});
    return hipGetLastError();
}

hipError_t launch_combine(hipStream_t s, const float* y, const float* weights, int rows, int slots, int D,
                          float* out) {
    combine_kernel<<<dim3((D / 4 + 255) / 256, rows), 256, 0, s>>>(y, weights, slots, D, out);
    return hipGetLastError();
}

}  // namespace gfr
