// The FP8 shared expert of the reference's MoE layer on gfx950 (glm-flash-rs src/moe.rs:132-167: shared_gu ->
// reduce8_bf16 -> shared_swiglu -> shared_down, four launches of precompiled kernels there), in two launches, or
// inside the bs = 1 layer's two EXL3 GEMV launches (exl3_decode.hip):
//   gate/up  gu[r][n] = bf16(sum over the 8 K slices s, in order, of scale[n] * (sum over k in s of x[r][k] * W[n][k]))
//            act[r][i] = bf16(bf16(silu(min(g, 10))) * clamp(u, -10, 10)), g = gu[r][i], u = gu[r][inter + i]
//   down     out[r][n] = scale_d[n] * sum over k of act[r][k] * Wd[n][k]                                       (fp32)
// the arithmetic of the reference's scalar oracle (src/front.rs:190-217 reference_mm_at: fixed split-K slices, each
// an fp32 sum scaled by the row's bf16 scale, the slices added in order; front.rs:669-675 the limited SwiGLU), with
// W [2 inter][hidden] and Wd [hidden][inter] float8_e4m3fn (OCP), the scales bf16, x bf16.
//
// MI355X design: v_mfma_f32_16x16x32_bf16 with the weights as the A operand (16 weight rows x 32 k), the token rows
// as B (16 rows of a row block; a one-token call uses one column). v_cvt_scalef32_pk_bf16_fp8 turns two fp8 bytes into
// two bf16 (exact: e4m3 values are bf16 values). A lane (row a = lane % 16, chunk q = lane / 16) loads 16 weight bytes
// of its row and the 16 matching activations of its token row per 64 k; the k order inside an MFMA is the same for A
// and B, so no data is rearranged.
//   * gate/up: a workgroup = IDX (2 or 8) intermediate indices x one row block; its A tile holds the gate rows and
//     the up rows of those indices, so the SwiGLU runs in the workgroup; wave s (8 waves) owns K slice s. The scaled
//     slice sums meet in LDS and are added in slice order.
//   * down: one wave a 16-column tile of the hidden size, K = inter in one chain (the reference's sk = 1).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "launch.hpp"
#include "shared_fp8.hpp"

namespace gfr {

namespace {
// Program (IDX-index block j of the intermediate size, 16-row block rb); wave s = K slice s. IDX < 8: fewer weight
// bytes a workgroup and more workgroups, for windows of a few rows, whose weight reads are spread over more CUs.
template <int IDX>
__global__ void __launch_bounds__(64 * FP8_SLICES) shared_gu_kernel(
    const uint8_t* __restrict__ w, const uint16_t* __restrict__ scale, const uint16_t* __restrict__ x, int x_stride,
    int rows, int hidden, int inter, uint16_t* __restrict__ gu, uint16_t* __restrict__ act) {
    __shared__ Fp8Part part;
    fp8_gu_program<IDX, FP8_SLICES, 8>(w, scale, x, x_stride, rows, blockIdx.y, hidden, inter, blockIdx.x,
                                       threadIdx.x >> 6, threadIdx.x & 63, part, gu, act);
}

// Program (16-column tile nt of the hidden size, 16-row block rb), one wave.
__global__ void __launch_bounds__(64) shared_down_kernel(const uint8_t* __restrict__ w,
                                                        const uint16_t* __restrict__ scale,
                                                        const uint16_t* __restrict__ act, int rows, int hidden,
                                                        int inter, float* __restrict__ out, int out_stride) {
    fp8_down_program<8>(w, scale, act, rows, blockIdx.y, inter, blockIdx.x, threadIdx.x, out, out_stride);
}
}  // namespace

hipError_t launch_shared_fp8(hipStream_t s, const uint8_t* wgu, const uint16_t* sgu, const uint8_t* wd,
                             const uint16_t* sd, const uint16_t* x, int x_stride, int rows, int hidden, int inter,
                             uint16_t* gu, uint16_t* act, float* out, int out_stride) {
    const int rblocks = (rows + 15) / 16;
    // a few rows: two intermediate indices a workgroup (the weights over 4x the CUs); more: eight (the token rows
    // are read by 4x fewer workgroups)
    if (rows <= 4)
        shared_gu_kernel<2><<<dim3(inter / 2, rblocks), 64 * FP8_SLICES, 0, s>>>(wgu, sgu, x, x_stride, rows, hidden,
                                                                               inter, gu, act);
    else
        shared_gu_kernel<8><<<dim3(inter / 8, rblocks), 64 * FP8_SLICES, 0, s>>>(wgu, sgu, x, x_stride, rows, hidden,
                                                                               inter, gu, act);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    shared_down_kernel<<<dim3(hidden / 16, rblocks), 64, 0, s>>>(wd, sd, act, rows, hidden, inter, out, out_stride);
    return hipGetLastError();
}

}  // namespace gfr
