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
#include <rocblas/rocblas.h>
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

// The prefill form's weight preparation (the reference's f8_b16_copy, prefill.cu:7-17): out[n][k] =
// bf16_rn(fp8(w[n][k]) * scale[n]), sixteen weights a thread (k a multiple of 16, so they share a row). The e4m3
// conversion is exact (0x7f / 0xff are NaN, as the reference makes them); the product of a 4-bit and an 8-bit
// significand is exact in fp32, so the only rounding is the bf16 one.
__global__ void __launch_bounds__(256) fp8_b16_copy_kernel(const uint8_t* __restrict__ w,
                                                           const uint16_t* __restrict__ scale,
                                                           uint16_t* __restrict__ out, long long count, int k) {
    const long long i = ((long long)blockIdx.x * 256 + threadIdx.x) * 16;
    if (i >= count) return;
    const uint4 v = *reinterpret_cast<const uint4*>(w + i);
    const float sc = bf16_to_f32(scale[i / k]);
    const uint32_t words[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(words[q], false);
        const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(words[q], true);
        o[2 * q] = (__builtin_bit_cast(uint32_t, bf16r(lo[0] * sc)) >> 16) |
                   (__builtin_bit_cast(uint32_t, bf16r(lo[1] * sc)) & 0xffff0000u);
        o[2 * q + 1] = (__builtin_bit_cast(uint32_t, bf16r(hi[0] * sc)) >> 16) |
                       (__builtin_bit_cast(uint32_t, bf16r(hi[1] * sc)) & 0xffff0000u);
    }
    uint4* dst = reinterpret_cast<uint4*>(out + i);
    dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
    dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
}

// shared_swiglu over a window's bf16 gu rows (the prefill form): act[r][i] = bf16(bf16(silu(min(g, 10))) *
// clamp(u, -10, 10)), g = gu[r][i], u = gu[r][inter + i].
__global__ void __launch_bounds__(256) fp8_swiglu_kernel(const uint16_t* __restrict__ gu, uint16_t* __restrict__ act,
                                                         int rows, int inter) {
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (long long)rows * inter) return;
    const int r = (int)(idx / inter), i = (int)(idx % inter);
    const float gg = fminf(bf16_to_f32(gu[(size_t)r * 2 * inter + i]), SHARED_LIMIT);
    const float uu = __builtin_amdgcn_fmed3f(bf16_to_f32(gu[(size_t)r * 2 * inter + inter + i]), -SHARED_LIMIT,
                                             SHARED_LIMIT);
    const float v = bf16r(bf16r(gg / (1.f + expf(-gg))) * uu);
    act[(size_t)r * inter + i] = (uint16_t)(__builtin_bit_cast(uint32_t, v) >> 16);
}
}  // namespace

hipError_t launch_fp8_b16_copy(hipStream_t s, const uint8_t* w, const uint16_t* scale, uint16_t* out, int n, int k) {
    const long long count = (long long)n * k;
    fp8_b16_copy_kernel<<<(unsigned)((count / 16 + 255) / 256), 256, 0, s>>>(w, scale, out, count, k);
    return hipGetLastError();
}

// The prefill form (the reference's prefill.rs Matrix::run with its prepared bf16 weights, batch.rs:1183-1195): gu =
// x W_gu^T (bf16 out), shared_swiglu, out = act W_d^T (fp32 out); both GEMMs are rocBLAS gemm_ex (bf16 operands, fp32
// accumulation), row-major operands as the transposed column-major products.
hipError_t launch_shared_fp8_prefill(void* blas, hipStream_t s, const uint16_t* wgu16, const uint16_t* wd16,
                                     const uint16_t* x, int x_stride, int rows, int hidden, int inter, uint16_t* gu,
                                     uint16_t* act, float* out, int out_stride) {
    rocblas_handle h = static_cast<rocblas_handle>(blas);
    if (rocblas_set_stream(h, s) != rocblas_status_success) return hipErrorInvalidValue;
    const float one = 1.f, zero = 0.f;
    // gu^T [2 inter][rows] = W_gu [2 inter][hidden] (col-major hidden x 2 inter, transposed) x x^T (hidden x rows)
    if (rocblas_gemm_ex(h, rocblas_operation_transpose, rocblas_operation_none, 2 * inter, rows, hidden, &one, wgu16,
                        rocblas_datatype_bf16_r, hidden, x, rocblas_datatype_bf16_r, x_stride, &zero, gu,
                        rocblas_datatype_bf16_r, 2 * inter, gu, rocblas_datatype_bf16_r, 2 * inter,
                        rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, rocblas_gemm_flags_none) !=
        rocblas_status_success)
        return hipErrorLaunchFailure;
    const long long n = (long long)rows * inter;
    fp8_swiglu_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(gu, act, rows, inter);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (rocblas_gemm_ex(h, rocblas_operation_transpose, rocblas_operation_none, hidden, rows, inter, &one, wd16,
                        rocblas_datatype_bf16_r, inter, act, rocblas_datatype_bf16_r, inter, &zero, out,
                        rocblas_datatype_f32_r, out_stride, out, rocblas_datatype_f32_r, out_stride,
                        rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, rocblas_gemm_flags_none) !=
        rocblas_status_success)
        return hipErrorLaunchFailure;
    return hipSuccess;
}

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
