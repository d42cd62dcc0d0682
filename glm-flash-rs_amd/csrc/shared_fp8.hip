// The FP8 shared expert of the reference's MoE layer on gfx950 (glm-flash-rs src/moe.rs:132-167: shared_gu ->
// reduce8_bf16 -> shared_swiglu -> shared_down, four launches of precompiled kernels there), in two launches:
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
//   * gate/up: a workgroup = 8 intermediate indices x one row block; its A tile holds the 8 gate rows and the 8 up
//     rows of those indices, so the SwiGLU runs in the workgroup; wave s (8 waves) owns K slice s. The scaled slice
//     sums meet in LDS and are added in slice order.
//   * down: one wave a 16-column tile of the hidden size, K = inter in one chain (the reference's sk = 1).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "exl3_format.hpp"
#include "launch.hpp"

namespace gfr {

namespace {
typedef __bf16 bf8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int FP8_SLICES = 8;          // moe.rs:133-143: shared_gu runs with 8 K slices, reduce8_bf16 adds them
constexpr float SHARED_LIMIT = 10.f;   // moe.rs:148-153: shared_swiglu's limit

// Sixteen fp8 weights (16 consecutive k) -> the two A fragments of consecutive MFMAs (k 0..7, k 8..15).
__device__ __forceinline__ void fp8_fragments(const uint4 w, bf8_t& f0, bf8_t& f1) {
    const auto c0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.x, 1.f, false);
    const auto c1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.x, 1.f, true);
    const auto c2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.y, 1.f, false);
    const auto c3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.y, 1.f, true);
    const auto c4 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.z, 1.f, false);
    const auto c5 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.z, 1.f, true);
    const auto c6 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.w, 1.f, false);
    const auto c7 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.w, 1.f, true);
    f0 = (bf8_t){c0[0], c0[1], c1[0], c1[1], c2[0], c2[1], c3[0], c3[1]};
    f1 = (bf8_t){c4[0], c4[1], c5[0], c5[1], c6[0], c6[1], c7[0], c7[1]};
}

// One lane's share of an fp8 row segment times a bf16 token row: chunks c = 0 .. nch - 1 of 64 k, the lane's
// 16 k at 64 c + 16 q of each; w and x point at the lane's first k. Eight chunks' loads are issued before their
// MFMAs.
// wok / xok: the lane's weight row / token row exists (a missing one feeds zeros and loads nothing).
__device__ __forceinline__ f4_t fp8_chain(const uint8_t* __restrict__ w, const uint16_t* __restrict__ x, int nch,
                                          bool wok, bool xok) {
    constexpr int G = 8;
    f4_t acc = {0.f, 0.f, 0.f, 0.f};
    for (int c0 = 0; c0 < nch; c0 += G) {
        uint4 wv[G], x0[G], x1[G];
#pragma unroll
        for (int k = 0; k < G; ++k)
            if (c0 + k < nch) {
                wv[k] = x0[k] = x1[k] = make_uint4(0u, 0u, 0u, 0u);
                if (wok) wv[k] = *reinterpret_cast<const uint4*>(w + 64 * (c0 + k));
                if (xok) {
                    x0[k] = *reinterpret_cast<const uint4*>(x + 64 * (c0 + k));
                    x1[k] = *reinterpret_cast<const uint4*>(x + 64 * (c0 + k) + 8);
                }
            }
#pragma unroll
        for (int k = 0; k < G; ++k)
            if (c0 + k < nch) {
                bf8_t a0, a1;
                fp8_fragments(wv[k], a0, a1);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, __builtin_bit_cast(bf8_t, x0[k]), acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, __builtin_bit_cast(bf8_t, x1[k]), acc, 0, 0, 0);
            }
    }
    return acc;
}

// Program (IDX-index block j of the intermediate size, 16-row block rb); wave s = K slice s. The A tile's rows 0..7
// are gate rows, 8..15 up rows, of which the first IDX are the block's (IDX < 8: fewer weight bytes a workgroup and
// more workgroups, for windows of a few rows, whose weight reads are spread over more CUs).
template <int IDX>
__global__ void __launch_bounds__(64 * FP8_SLICES) shared_gu_kernel(
    const uint8_t* __restrict__ w, const uint16_t* __restrict__ scale, const uint16_t* __restrict__ x, int x_stride,
    int rows, int hidden, int inter, uint16_t* __restrict__ gu, uint16_t* __restrict__ act) {
    static_assert(IDX == 2 || IDX == 4 || IDX == 8, "indices a workgroup");
    __shared__ float part[FP8_SLICES][16][17];
    const int j = blockIdx.x, rb = blockIdx.y;
    const int s = threadIdx.x >> 6, lane = threadIdx.x & 63, a = lane & 15, q = lane >> 4;
    const int L = hidden / FP8_SLICES;                       // a slice's k
    const int ia = a & 7;
    const int wrow = (a < 8 ? 0 : inter) + IDX * j + ia;
    const int row = rb * 16 + a, rowc = row < rows ? row : rows - 1;
    // D holds weight rows 4 q + e of the tile: their scales, loaded with the operands
    float sc[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int it = 4 * (q & 1) + e;
        sc[e] = it < IDX ? bf16_to_f32(scale[(q < 2 ? 0 : inter) + IDX * j + it]) : 0.f;
    }
    const f4_t acc = fp8_chain(w + (size_t)(ia < IDX ? wrow : 0) * hidden + s * L + 16 * q,
                               x + (size_t)rowc * x_stride + s * L + 16 * q, L / 64, ia < IDX, row < rows);
    // D: weight row 4 q + e of the tile, token row a of the block; the slice's sum times the row's scale
#pragma unroll
    for (int e = 0; e < 4; ++e) part[s][4 * q + e][a] = acc[e] * sc[e];
    __syncthreads();
    if (threadIdx.x < 16 * IDX) {
        const int i = threadIdx.x % IDX, r = threadIdx.x / IDX, orow = rb * 16 + r;
        float g = part[0][i][r], u = part[0][8 + i][r];
#pragma unroll
        for (int p = 1; p < FP8_SLICES; ++p) {
            g += part[p][i][r];
            u += part[p][8 + i][r];
        }
        if (orow < rows) {
            const float gb = bf16r(g), ub = bf16r(u);
            gu[(size_t)orow * 2 * inter + IDX * j + i] = (uint16_t)(__builtin_bit_cast(uint32_t, gb) >> 16);
            gu[(size_t)orow * 2 * inter + inter + IDX * j + i] = (uint16_t)(__builtin_bit_cast(uint32_t, ub) >> 16);
            const float gg = fminf(gb, SHARED_LIMIT);
            const float uu = __builtin_amdgcn_fmed3f(ub, -SHARED_LIMIT, SHARED_LIMIT);
            const float v = bf16r(bf16r(gg / (1.f + expf(-gg))) * uu);
            act[(size_t)orow * inter + IDX * j + i] = (uint16_t)(__builtin_bit_cast(uint32_t, v) >> 16);
        }
    }
}

// Program (16-column tile nt of the hidden size, 16-row block rb), one wave.
__global__ void __launch_bounds__(64) shared_down_kernel(const uint8_t* __restrict__ w,
                                                        const uint16_t* __restrict__ scale,
                                                        const uint16_t* __restrict__ act, int rows, int hidden,
                                                        int inter, float* __restrict__ out, int out_stride) {
    const int nt = blockIdx.x, rb = blockIdx.y, lane = threadIdx.x, a = lane & 15, q = lane >> 4;
    const int row = rb * 16 + a, rowc = row < rows ? row : rows - 1;
    const int n = 16 * nt + 4 * q;
    const uint2 sc = *reinterpret_cast<const uint2*>(scale + n);
    const f4_t acc = fp8_chain(w + (size_t)(16 * nt + a) * inter + 16 * q, act + (size_t)rowc * inter + 16 * q,
                               inter / 64, true, row < rows);
    if (row < rows) {
        const float4 v = make_float4(acc[0] * bf16_to_f32((uint16_t)sc.x), acc[1] * bf16_to_f32((uint16_t)(sc.x >> 16)),
                                     acc[2] * bf16_to_f32((uint16_t)sc.y), acc[3] * bf16_to_f32((uint16_t)(sc.y >> 16)));
        *reinterpret_cast<float4*>(out + (size_t)row * out_stride + n) = v;
    }
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
