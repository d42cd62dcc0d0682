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

// out[r][n] = sum over slots s (in order) of weights[r][s] * (y[r * slots + s][n] for the EXL3 slots s < exl3_slots,
// shared[r * shared_stride + n] for the others when the caller gives the shared expert's output, else nothing) --
// the reference's combine(y, shared, weights, out), moe.rs:171-181. Four columns a thread (16-byte loads and
// stores); the slots in groups of 8, each group's rows in flight at once and added in slot order (a group's 8
// registers, not one per possible slot, keep the kernel at a few dozen VGPRs and many resident waves). D a multiple
// of 4.
__global__ void __launch_bounds__(256) combine_kernel(const float* __restrict__ y, const float* __restrict__ weights,
                                                      int slots, int exl3_slots, int D,
                                                      const float* __restrict__ shared, int shared_stride,
                                                      float* __restrict__ out) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    constexpr int G = 8;
    const int r = blockIdx.y, n = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (n >= D) return;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = 0; s0 < slots; s0 += G) {
        f4v v[G];
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const int s = s0 + j;
            if (s < slots) {
                if (s < exl3_slots)
                    v[j] = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(y + ((size_t)r * slots + s) * D + n));
                else
                    v[j] = shared ? *reinterpret_cast<const f4v*>(shared + (size_t)r * shared_stride + n)
                                  : (f4v){0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const int s = s0 + j;
            if (s < slots && (s < exl3_slots || shared)) {
                const float w = weights[r * slots + s];
                acc.x += w * v[j].x;
                acc.y += w * v[j].y;
                acc.z += w * v[j].z;
                acc.w += w * v[j].w;
            }
        }
    }
    *reinterpret_cast<float4*>(out + (size_t)r * D + n) = acc;
}

// Router logits (the reference's router_part + router_sum, moe.rs:77-87; Triton, source absent): logits[r][e] =
// sum over k of x[r][k] * W[e][k], bf16 inputs, fp32 products and sums in a fixed order (v_dot2_f32_bf16 pairs in
// k order within a lane, then the 64 lanes in a fixed tree). Program (8 experts, up to RTMAX rows); wave w owns
// experts 8 b + w and 8 b + w + 4 and holds their weight chunks in registers while the program's rows stream past
// them (hidden sizes above 4096 reload the chunks a pass of 4096 a row).
typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
constexpr int ROUTER_RTMAX = 8;   // rows a program (the weight chunks are loaded once for them)
__global__ void __launch_bounds__(256) router_logits_kernel(const uint16_t* __restrict__ x, int x_stride,
                                                            const uint16_t* __restrict__ W, int D, int E, int rows,
                                                            int RT, float* __restrict__ logits) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    constexpr int CH = 8;                            // 16-byte chunks a lane a pass (4096 values a pass)
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r0 = blockIdx.y * RT, r1 = r0 + RT < rows ? r0 + RT : rows;
    const int ex[2] = {(int)blockIdx.x * 8 + wave, (int)blockIdx.x * 8 + wave + 4};
    u32x4 w[2][CH];                                  // lane l: 8 weights at k = k0 + (c * 64 + l) * 8
    auto load_w = [&](int k0) {
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int e = ex[q] < E ? ex[q] : E - 1;
                const int k = k0 + (c * 64 + lane) * 8;
                w[q][c] = k < D ? *reinterpret_cast<const u32x4*>(W + (size_t)e * D + k) : (u32x4){0, 0, 0, 0};
            }
    };
    const bool one_pass = D <= CH * 512;
    if (one_pass) load_w(0);
    for (int r = r0; r < r1; ++r) {
        float acc[2] = {0.f, 0.f};
        for (int k0 = 0; k0 < D; k0 += CH * 512) {
            if (!one_pass) load_w(k0);
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int k = k0 + (c * 64 + lane) * 8;
                const u32x4 xv = k < D ? *reinterpret_cast<const u32x4*>(x + (size_t)r * x_stride + k) : (u32x4){0, 0, 0, 0};
                const uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const uint32_t ws[4] = {w[q][c].x, w[q][c].y, w[q][c].z, w[q][c].w};
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[q] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2_t, ws[j]),
                                                                __builtin_bit_cast(bf2_t, xs[j]), acc[q], false);
                }
            }
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            float v = acc[q];
            v += lane_xor_f<1>(v);
            v += lane_xor_f<2>(v);
            v += lane_xor_f<4>(v);
            v += lane_xor_f<8>(v);
            v += lane_xor_f<16>(v);
            v += lane_xor_f<32>(v);
            if (lane == 0 && ex[q] < E) logits[(size_t)r * E + ex[q]] = v;
        }
    }
}

}  // namespace gfr

#include "launch.hpp"

namespace gfr {

hipError_t launch_route(hipStream_t s, const float* logits, int rows, int E, int topk, int shared_id, int* picks,
                        float* weights, const float* bias, float scale) {
    route_kernel<<<rows, 64, 0, s>>>(logits, E, topk, shared_id, picks, weights, RouteGate{bias, scale});
    return hipGetLastError();
}

hipError_t launch_combine(hipStream_t s, const float* y, const float* weights, int rows, int slots, int exl3_slots,
                          int D, const float* shared, int shared_stride, float* out) {
    combine_kernel<<<dim3((D / 4 + 255) / 256, rows), 256, 0, s>>>(y, weights, slots, exl3_slots, D, shared,
                                                                   shared_stride, out);
    return hipGetLastError();
}

int router_logits_max_hidden() { return 1 << 16; }

hipError_t launch_router_logits(hipStream_t s, const uint16_t* x, int x_stride, const uint16_t* W, int D, int E,
                                int rows, float* logits) {
    const int RT = rows >= 64 ? ROUTER_RTMAX : rows >= 8 ? 4 : 1;
    router_logits_kernel<<<dim3((E + 7) / 8, (rows + RT - 1) / RT), 256, 0, s>>>(x, x_stride, W, D, E, rows, RT,
                                                                                  logits);
    return hipGetLastError();
}

}  // namespace gfr
