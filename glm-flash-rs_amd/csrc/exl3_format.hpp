// EXL3 trellis format on gfx950: the codebook, the 16-bit states of a tile and the 128-point Hadamard transform,
// written for 64-wide wavefronts.
//
// Format (glm-flash-rs src/experts.rs:43-74, native/exl3.cu:21-40, after ExLlamaV3): a 16x16 tile of K-bit weights
// is 8K little-endian 32-bit words forming a circular bitstream (MSB first within a word). Value p (0..255) is the
// codebook entry of the 16-bit window that ends at bit (p + 1) K, and sits at row 2(L%4) + (j&1) + 8((j>>1)&1),
// column L/4 + 8(j>>2) of the tile, where L = p / 8, j = p % 8 (row = k, column = n).
//
// Lane layout used here ("8 lanes a tile"): lane i (0..7) of a tile owns values 32i..32i+31 = words Ki..Ki+K-1 and
// needs the low bits of word Ki-1 (the previous lane's last word; lane 0 wraps to lane 7). Those 32 values are
// columns i and i+8 of all 16 rows, so one lane produces two output columns' worth of products per k tile.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gfr {

constexpr float HAD_SCALE = 0.08838834764831845f;  // 1 / sqrt(128)

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t h2_bits(h2_t v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ h2_t bits_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }

// The scrambled state: two fp16 halves whose sum is the codebook value (experts.rs:43-46).
__device__ __forceinline__ uint32_t mcg_x(uint32_t s) { return ((s * 0xCBAC1FEDu) & 0x8FFF8FFFu) ^ 0x3B603B60u; }

// Codebook values of two 16-bit states as packed fp16 (first state in the low half). The per-state sum lo + hi is
// one fp16 round-to-nearest add, as the reference's half2 add.
__device__ __forceinline__ h2_t mcg2(uint32_t s0, uint32_t s1) {
    const uint32_t x0 = mcg_x(s0), x1 = mcg_x(s1);
    const uint32_t lo = __builtin_amdgcn_perm(x1, x0, 0x05040100u);  // x0.lo | x1.lo << 16
    const uint32_t hi = __builtin_amdgcn_perm(x1, x0, 0x07060302u);  // x0.hi | x1.hi << 16
    return bits_h2(lo) + bits_h2(hi);
}

// The 16-bit state of the lane's value q (0..31): window ending at bit (q + 1) K of the lane's bit range, whose
// first word is w[0]; prev = the word before w[0] in the circular stream. All positions are compile-time.
template <int K, int Q>
__device__ __forceinline__ uint32_t lane_state(const uint32_t (&w)[K], uint32_t prev) {
    constexpr int e = (Q + 1) * K;               // window end, in bits from the lane's first bit
    constexpr int hiw = (e - 1) >> 5;            // word holding the window's last bit
    constexpr int shift = 32 * (hiw + 1) - e;    // right shift that brings the window end to bit 0
    if constexpr (shift + 16 <= 32) {
        return (w[hiw] >> shift) & 0xffffu;
    } else {
        const uint32_t hi = hiw == 0 ? prev : w[hiw > 0 ? hiw - 1 : 0];
        return __builtin_amdgcn_alignbit(hi, w[hiw], shift) & 0xffffu;
    }
}

// Decode the lane's 32 values into 16 packed pairs: d[c][h][l] = rows (2l + 8h, 2l + 8h + 1) of column i + 8c.
template <int K>
__device__ __forceinline__ void decode_lane(const uint32_t (&w)[K], uint32_t prev, h2_t (&d)[2][2][4]) {
#define GFR_DEC(L)                                                                                         \
    d[0][0][L] = mcg2(lane_state<K, 8 * L + 0>(w, prev), lane_state<K, 8 * L + 1>(w, prev));                \
    d[0][1][L] = mcg2(lane_state<K, 8 * L + 2>(w, prev), lane_state<K, 8 * L + 3>(w, prev));                \
    d[1][0][L] = mcg2(lane_state<K, 8 * L + 4>(w, prev), lane_state<K, 8 * L + 5>(w, prev));                \
    d[1][1][L] = mcg2(lane_state<K, 8 * L + 6>(w, prev), lane_state<K, 8 * L + 7>(w, prev));
    GFR_DEC(0) GFR_DEC(1) GFR_DEC(2) GFR_DEC(3)
#undef GFR_DEC
}

// The previous word for lane i of an 8-lane tile group: lane - 1, or lane + 7 for i == 0 (DPP within a 16-lane row).
__device__ __forceinline__ uint32_t prev_word(uint32_t last, int i) {
    const uint32_t shr1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)last, 0x111, 0xf, 0xf, false);  // row_shr:1
    const uint32_t shl7 = (uint32_t)__builtin_amdgcn_mov_dpp((int)last, 0x107, 0xf, 0xf, false);  // row_shl:7
    return i == 0 ? shl7 : shr1;
}

__device__ __forceinline__ float bf16r(float x) {
    // round to nearest even to bf16 (experts.rs:19-21 bit form; finite inputs)
    uint32_t b = __builtin_bit_cast(uint32_t, x);
    b = (b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u;
    return __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

// 128-point unnormalised Walsh-Hadamard transform of a wave64 row, two values a lane (v[j] = element 2 lane + j):
// butterflies at strides 1, 2, ..., 64, each (lower + upper, lower - upper) -- experts.rs:25-42's order, so every
// element gets the same fp32 sums as there.
__device__ __forceinline__ void fwht128_w64(float (&v)[2], int lane) {
    {
        const float a = v[0], b = v[1];
        v[0] = a + b;
        v[1] = a - b;
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const float o = __shfl_xor(v[j], m, 64);
            v[j] = (lane & m) ? o - v[j] : v[j] + o;
        }
    }
}

}  // namespace gfr
