// The FP8 shared expert's device programs (glm-flash-rs src/moe.rs:132-167), shared by its own kernels
// (shared_fp8.hip) and by the bs = 1 layer's EXL3 launches (exl3_decode.hip), whose idle shared-slot workgroups run
// them when the layer's shared expert is FP8. Arithmetic and layout: shared_fp8.hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "exl3_format.hpp"

namespace gfr {

typedef __bf16 fp8_bf8_t __attribute__((ext_vector_type(8)));
typedef float fp8_f4_t __attribute__((ext_vector_type(4)));

constexpr int FP8_SLICES = 8;          // moe.rs:133-143: shared_gu runs with 8 K slices, reduce8_bf16 adds them
constexpr float SHARED_LIMIT = 10.f;   // moe.rs:148-153: shared_swiglu's limit

// Sixteen fp8 weights (16 consecutive k) -> the two A fragments of consecutive MFMAs (k 0..7, k 8..15).
__device__ __forceinline__ void fp8_fragments(const uint4 w, fp8_bf8_t& f0, fp8_bf8_t& f1) {
    const auto c0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.x, 1.f, false);
    const auto c1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.x, 1.f, true);
    const auto c2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.y, 1.f, false);
    const auto c3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.y, 1.f, true);
    const auto c4 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.z, 1.f, false);
    const auto c5 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.z, 1.f, true);
    const auto c6 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.w, 1.f, false);
    const auto c7 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.w, 1.f, true);
    f0 = (fp8_bf8_t){c0[0], c0[1], c1[0], c1[1], c2[0], c2[1], c3[0], c3[1]};
    f1 = (fp8_bf8_t){c4[0], c4[1], c5[0], c5[1], c6[0], c6[1], c7[0], c7[1]};
}

// One lane's share of an fp8 row segment times a bf16 token row: chunks c = 0 .. nch - 1 of 64 k, the lane's
// 16 k at 64 c + 16 q of each; w and x point at the lane's first k. G chunks' loads are issued before their MFMAs.
// wok / xok: the lane's weight row / token row exists (a missing one feeds zeros and loads nothing).
template <int G>
__device__ __forceinline__ fp8_f4_t fp8_chain(const uint8_t* __restrict__ w, const uint16_t* __restrict__ x, int nch,
                                              bool wok, bool xok) {
    fp8_f4_t acc = {0.f, 0.f, 0.f, 0.f};
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
                fp8_bf8_t a0, a1;
                fp8_fragments(wv[k], a0, a1);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, __builtin_bit_cast(fp8_bf8_t, x0[k]), acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, __builtin_bit_cast(fp8_bf8_t, x1[k]), acc, 0, 0, 0);
            }
    }
    return acc;
}

// The shared expert's operands when it rides on the bs = 1 layer's EXL3 launches (a second kernel argument of their
// FP8 forms): gate/up launch w / s = gate/up weights and scales, x = the token row, outputs gu / act; down launch
// w / s = down weights and scales, x = act, output out.
struct Fp8Args {
    const uint8_t* w;
    const uint16_t* s;
    const uint16_t* x;
    uint16_t* gu;
    uint16_t* act;
    float* out;
    int hidden, inter;
};

// The scaled slice sums of one workgroup's gate/up program meet here.
typedef float Fp8Part[FP8_SLICES][16][17];

// Gate/up program of IDX intermediate indices j IDX .. (the A tile's rows 0..7: gate rows, 8..15: up rows, of which the
// first IDX are the program's) for the 16-row block rb, run by NWV waves of a workgroup: wave v takes K slices
// v, v + NWV, ..; the slices' scaled sums are added in slice order, rounded to bf16 (gu) and through the limited
// SwiGLU (act) by the workgroup's first 16 IDX threads. Every thread of the workgroup calls it (one barrier inside).
template <int IDX, int NWV, int G>
__device__ __forceinline__ void fp8_gu_program(const uint8_t* __restrict__ w, const uint16_t* __restrict__ scale,
                                               const uint16_t* __restrict__ x, int x_stride, int rows, int rb,
                                               int hidden, int inter, int j, int wave, int lane, Fp8Part& part,
                                               uint16_t* __restrict__ gu, uint16_t* __restrict__ act) {
    static_assert(IDX == 2 || IDX == 4 || IDX == 8, "indices a program");
    const int a = lane & 15, q = lane >> 4, ia = a & 7;
    const int L = hidden / FP8_SLICES;                       // a slice's k
    const int wrow = (a < 8 ? 0 : inter) + IDX * j + ia;
    const int row = rb * 16 + a, rowc = row < rows ? row : rows - 1;
    // D holds weight rows 4 q + e of the tile: their scales, loaded with the operands
    float sc[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int it = 4 * (q & 1) + e;
        sc[e] = it < IDX ? bf16_to_f32(scale[(q < 2 ? 0 : inter) + IDX * j + it]) : 0.f;
    }
#pragma unroll
    for (int s = wave; s < FP8_SLICES; s += NWV) {
        const fp8_f4_t acc = fp8_chain<G>(w + (size_t)(ia < IDX ? wrow : 0) * hidden + s * L + 16 * q,
                                          x + (size_t)rowc * x_stride + s * L + 16 * q, L / 64, ia < IDX, row < rows);
        // D: weight row 4 q + e of the tile, token row a of the block; the slice's sum times the row's scale
#pragma unroll
        for (int e = 0; e < 4; ++e) part[s][4 * q + e][a] = acc[e] * sc[e];
    }
    __syncthreads();
    const int tid = wave * 64 + lane;
    if (tid < 16 * IDX) {
        const int i = tid % IDX, r = tid / IDX, orow = rb * 16 + r;
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

// Down program of one wave: the 16 hidden columns of tile nt for the 16-row block rb, K = inter in one chain (the
// reference's sk = 1), times the columns' scales -> out (fp32).
template <int G>
__device__ __forceinline__ void fp8_down_program(const uint8_t* __restrict__ w, const uint16_t* __restrict__ scale,
                                                 const uint16_t* __restrict__ act, int rows, int rb, int inter, int nt,
                                                 int lane, float* __restrict__ out, int out_stride) {
    const int a = lane & 15, q = lane >> 4;
    const int row = rb * 16 + a, rowc = row < rows ? row : rows - 1;
    const int n = 16 * nt + 4 * q;
    const uint2 sc = *reinterpret_cast<const uint2*>(scale + n);
    const fp8_f4_t acc = fp8_chain<G>(w + (size_t)(16 * nt + a) * inter + 16 * q,
                                      act + (size_t)rowc * inter + 16 * q, inter / 64, true, row < rows);
    if (row < rows) {
        const float4 v = make_float4(acc[0] * bf16_to_f32((uint16_t)sc.x), acc[1] * bf16_to_f32((uint16_t)(sc.x >> 16)),
                                     acc[2] * bf16_to_f32((uint16_t)sc.y), acc[3] * bf16_to_f32((uint16_t)(sc.y >> 16)));
        *reinterpret_cast<float4*>(out + (size_t)row * out_stride + n) = v;
    }
}

}  // namespace gfr
