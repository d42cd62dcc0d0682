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
// Value q (0..31) of lane i is tile value p = 32i + q: row 2(q/8) + (j&1) + 8((j>>1)&1), column i + 8(j>>2), j = q%8.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <utility>

namespace gfr {

constexpr float HAD_SCALE = 0.08838834764831845f;  // 1 / sqrt(128)

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t h2_bits(h2_t v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ h2_t bits_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }

// Codebook values of two 16-bit states packed in one register (S = s_a | s_b << 16), as packed fp16 (w_a, w_b).
// experts.rs:43-46 per state: x = s * 0xCBAC1FED mod 2^32, (x & 0x8FFF8FFF) ^ 0x3B603B60, value = fp16(x.lo) +
// fp16(x.hi) rounded to fp16. Computed two states at a time in 16-bit lanes: x.lo = (s * 0x1FED) mod 2^16 and
// x.hi = (s * 0xCBAC + ((s * 0x1FED) >> 16)) mod 2^16, with s * 0x1FED < 2^29 exact in a 24-bit multiply.
// hipcc emits 8 VALU ops a pair: 2 v_mul_u32_u24 (SDWA word select), 2 v_perm, v_pk_mad_u16, 2 v_bitop3, v_pk_add_f16.
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
// (x & m) ^ f as one v_bitop3 (truth table over src0 = 0xF0, src1 = 0xCC, src2 = 0xAA: (0xF0 & 0xCC) ^ 0xAA = 0x6A)
__device__ __forceinline__ uint32_t mask_flip(uint32_t x, uint32_t m, uint32_t f) {
    return __builtin_amdgcn_bitop3_b32(x, m, f, 0x6A);
}
__device__ __forceinline__ h2_t decode_pair(uint32_t S) {
    const uint32_t pa = (S & 0xffffu) * 0x1FEDu;
    const uint32_t pb = (S >> 16) * 0x1FEDu;
    const uint32_t lo = __builtin_amdgcn_perm(pb, pa, 0x05040100u);   // (x_a.lo, x_b.lo)
    const uint32_t cy = __builtin_amdgcn_perm(pb, pa, 0x07060302u);   // carries into the high halves
    const u16x2_t hv = __builtin_bit_cast(u16x2_t, S) * (u16x2_t){0xCBAC, 0xCBAC} + __builtin_bit_cast(u16x2_t, cy);
    const uint32_t hi = __builtin_bit_cast(uint32_t, hv);                   // (x_a.hi, x_b.hi)
    const uint32_t lm = (lo & 0x8FFF8FFFu) ^ 0x3B603B60u;
    const uint32_t hm = (hi & 0x8FFF8FFFu) ^ 0x3B603B60u;
    return bits_h2(lm) + bits_h2(hm);
}

// Right funnel shift of the lane's bit stream so that the window of value Q ends at bit 0 (junk above bit 15).
template <int K, int Q>
__device__ __forceinline__ uint32_t lane_window(const uint32_t (&w)[K], uint32_t prev) {
    constexpr int e = (Q + 1) * K;               // window end, in bits from the lane's first bit
    constexpr int hiw = (e - 1) >> 5;            // word holding the window's last bit
    constexpr int shift = 32 * (hiw + 1) - e;    // right shift that brings the window end to bit 0
    if constexpr (shift + 16 <= 32) {
        return w[hiw] >> shift;
    } else {
        const uint32_t hi = hiw == 0 ? prev : w[hiw > 0 ? hiw - 1 : 0];
        return __builtin_amdgcn_alignbit(hi, w[hiw], shift);
    }
}

// Row pairs: decode_lane produces, for each of the lane's two columns (i, i + 8), 8 packed weight pairs
// d[c][m] = (W[ra(m)][col], W[rb(m)][col]) (low, high half). The pairing depends on K so that the two states of a
// pair come out of one register cheaply; rows are those of the tile (0..15). These fp16 weights (the reference's
// rounding) serve the decoded-weight probe (gfr_exl3_decode_tiles) and, in the K != 2 pairing, the prefill MFMA's A
// fragments, whose token rows are staged in the same pair order. The decode GEMV uses lane_words / tile_dot below.
//   K != 2: m = 2l + h  -> rows (2l + 8 + h, 2l + h)             values (8l + j + 2, 8l + j), j = h or 4 + h
//   K == 2: m = 4v + u  -> rows (r + 2, r), r = 4v + (u&1) + 8(u>>1)  values (16v + j + 8, 16v + j), j = u or 4 + u
__host__ __device__ constexpr int pair_row(int K, int m, int half) {
    return K == 2 ? (4 * (m >> 2) + ((m & 3) & 1) + 8 * ((m & 3) >> 1) + (half ? 0 : 2))
                  : (2 * (m >> 1) + (m & 1) + (half ? 0 : 8));
}

// The lane's 32 values, each from its own funnel-shifted window, in the K != 2 pairing (pair_row with K != 2).
template <int K>
__device__ __forceinline__ void decode_lane_windows(const uint32_t (&w)[K], uint32_t prev, h2_t (&d)[2][8]) {
#define GFR_PAIR(L, J)                                                                                       \
    d[(J) >> 2][2 * (L) + ((J) & 1)] = decode_pair(__builtin_amdgcn_perm(                                     \
        lane_window<K, 8 * (L) + (J)>(w, prev), lane_window<K, 8 * (L) + (J) + 2>(w, prev), 0x05040100u));
#define GFR_WORDS(L) GFR_PAIR(L, 0) GFR_PAIR(L, 1) GFR_PAIR(L, 4) GFR_PAIR(L, 5)
    GFR_WORDS(0) GFR_WORDS(1) GFR_WORDS(2) GFR_WORDS(3)
#undef GFR_WORDS
#undef GFR_PAIR
}

// Decode the lane's 32 values into d[c][m] (see pair_row).
template <int K>
__device__ __forceinline__ void decode_lane(const uint32_t (&w)[K], uint32_t prev, h2_t (&d)[2][8]) {
    if constexpr (K == 4) {
        // four words, each holding the windows of values 8l .. 8l + 7 at right shifts 28 - 4j of (p : w); pairs
        // (j + 2, j) sit 8 bits apart, so one byte permute of (p : w) or of (p : w) >> 4 packs a pair
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t p = l == 0 ? prev : w[l > 0 ? l - 1 : 0];
            const uint32_t a = __builtin_amdgcn_alignbit(p, w[l], 4);
            const uint32_t b = p >> 4;
            d[1][2 * l + 1] = decode_pair(__builtin_amdgcn_perm(p, w[l], 0x02010100u));  // (s7, s5)
            d[0][2 * l + 1] = decode_pair(__builtin_amdgcn_perm(p, w[l], 0x04030302u));  // (s3, s1)
            d[1][2 * l] = decode_pair(__builtin_amdgcn_perm(b, a, 0x02010100u));         // (s6, s4)
            d[0][2 * l] = decode_pair(__builtin_amdgcn_perm(b, a, 0x04030302u));         // (s2, s0)
        }
    } else if constexpr (K == 2) {
        // two words; values q and q + 8 are 16 bits apart: one funnel shift holds the pair (q + 8 low, q high)
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            const uint32_t p = v == 0 ? prev : w[0];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                d[j >> 2][4 * v + (j & 3)] = decode_pair(__builtin_amdgcn_alignbit(p, w[v], 14 - 2 * j));
        }
    } else {
        decode_lane_windows<K>(w, prev, d);
    }
}


// ---- the decode GEMV's dot: codebook words against activations, without the fp16 weight in between -------------
// For one state s (16 bits, in half SEL of r), the masked codebook word m = (s * 0xCBAC1FED mod 2^32 & 0x8FFF8FFF) ^
// 0x3B603B60 (experts.rs:43-46) holds the two fp16 halves whose sum is the weight. The GEMV adds both halves times
// the activation in one v_dot2_f32_f16 against the activation staged twice, (x, x): acc + x * m.lo + x * m.hi in
// fp32. The reference rounds m.lo + m.hi to fp16 first; this sum keeps that rounding
// out (a difference of at most half an fp16 ulp of each weight). Four VALU operations a weight at K = 4:
//   v_and_b32 / v_lshrrev_b32   the state's half of r, alone in a register
//   v_mul_lo_u32                s * 0xCBAC1FED mod 2^32
//   v_bitop3                    mask, flip
//   v_dot2_f32_f16              acc += x * m.lo + x * m.hi
// Every constant is a VGPR operand (CodewordConsts): on gfx950 an SGPR or literal operand makes a VALU operation of
// two issue passes where the all-VGPR v_and / v_lshrrev / v_bitop3 take one. Measured per decoded state and SIMD,
// three waves a SIMD: 8.62 ns for the earlier form (v_pk_mul_lo_u16 + v_mad_u32_u16 with SGPR constants, SGPR mask),
// 7.82 ns for this one. The other widths: v_pk_mul_lo_u16 (0, s * 0xCBAC) and v_mad_u32_u16 s * 0x1FED + that, then
// the mask and the dot. (op_sel on the v_dot2 operands is not encodable on gfx950, hence the doubled activations.)
struct CodewordConsts {
    uint32_t lo16, mul, mask, flip;
};
// Made once per kernel: at K = 4 the asm hides the values, so the compiler keeps them in VGPRs and does not fold
// them (the other widths' codeword does not read them).
template <int K>
__device__ __forceinline__ CodewordConsts codeword_consts() {
    CodewordConsts c{0xffffu, 0xCBAC1FEDu, 0x8FFF8FFFu, 0x3B603B60u};
    if constexpr (K == 4) __asm__ volatile("" : "+v"(c.lo16), "+v"(c.mul), "+v"(c.mask), "+v"(c.flip));
    return c;
}
// K = 4 (config 2's width) takes the v_mul_lo_u32 form with VGPR constants; the other widths keep v_pk_mul_lo_u16 +
// v_mad_u32_u16, whose op_sel picks the state's half without a mask (measured: the mul form is 2 % faster on
// config 2's layer, and 1-2 % slower at K = 2 and 3, whose kernels lose a resident wave to its two extra VGPRs).
template <int SEL, int K>
__device__ __forceinline__ uint32_t codeword(uint32_t r, const CodewordConsts& c) {
    uint32_t x;
    if constexpr (K == 4) {
        const uint32_t s = SEL == 0 ? (r & c.lo16) : (r >> 16);
        x = s * c.mul;
    } else {
        uint32_t t;
        if constexpr (SEL == 0) {
            __asm__("v_pk_mul_lo_u16 %0, %1, %2 op_sel:[0,0] op_sel_hi:[0,1]" : "=v"(t) : "v"(r), "s"(0xCBAC0000u));
            __asm__("v_mad_u32_u16 %0, %1, %2, %3" : "=v"(x) : "v"(r), "s"(0x1FEDu), "v"(t));
        } else {
            __asm__("v_pk_mul_lo_u16 %0, %1, %2 op_sel:[1,0] op_sel_hi:[1,1]" : "=v"(t) : "v"(r), "s"(0xCBAC0000u));
            __asm__("v_mad_u32_u16 %0, %1, %2, %3 op_sel:[1,0,0,0]" : "=v"(x) : "v"(r), "s"(0x1FEDu), "v"(t));
        }
        return (x & 0x8FFF8FFFu) ^ 0x3B603B60u;
    }
    return mask_flip(x, c.mask, c.flip);
}
// The lane's stream shifted right so that the window of value Q ends at bit 0, all 32 bits (bits 16-31: the 16
// stream bits before the window).
template <int K, int Q>
__device__ __forceinline__ uint32_t lane_window32(const uint32_t (&w)[K], uint32_t prev) {
    constexpr int e = (Q + 1) * K, hiw = (e - 1) >> 5, shift = 32 * (hiw + 1) - e;
    if constexpr (shift == 0) return w[hiw];
    else return __builtin_amdgcn_alignbit(hiw == 0 ? prev : w[hiw > 0 ? hiw - 1 : 0], w[hiw], shift);
}

// Masked codebook words of the lane's 32 values, value order. K = 2 and 4: one 32-bit window holds the states of
// values Q (low half) and Q - 16 / K (high half).
template <int K, int Q>
__device__ __forceinline__ void lane_word(const uint32_t (&w)[K], uint32_t prev, uint32_t (&m)[32],
                                          const CodewordConsts& c) {
    if constexpr (K == 2 || K == 4) {
        constexpr int D = 16 / K;
        if constexpr (Q % (2 * D) >= D) {
            const uint32_t r = lane_window32<K, Q>(w, prev);
            m[Q] = codeword<0, K>(r, c);
            m[Q - D] = codeword<1, K>(r, c);
        }
    } else {
        m[Q] = codeword<0, K>(lane_window<K, Q>(w, prev), c);
    }
}
template <int K, int... Q>
__device__ __forceinline__ void lane_words_(const uint32_t (&w)[K], uint32_t prev, uint32_t (&m)[32],
                                            const CodewordConsts& c, std::integer_sequence<int, Q...>) {
    (lane_word<K, Q>(w, prev, m, c), ...);
}
template <int K>
__device__ __forceinline__ void lane_words(const uint32_t (&w)[K], uint32_t prev, uint32_t (&m)[32],
                                           const CodewordConsts& c) {
    lane_words_<K>(w, prev, m, c, std::make_integer_sequence<int, 32>{});
}

// Tile row of value q of a lane (the format's row 2 (q / 8) + (j & 1) + 8 ((j >> 1) & 1), j = q % 8) and its column
// (0: i, 1: i + 8).
__host__ __device__ constexpr int value_row(int q) { return 2 * ((q >> 3) & 3) + (q & 1) + 8 * ((q >> 1) & 1); }
__host__ __device__ constexpr int value_col(int q) { return (q & 7) >> 2; }

// One k tile of the lane's two columns against the tile's 16 activations, each staged twice (xd[r] = (x_r, x_r)):
// acc[c] += the column's 16 weights times their rows, added in value order.
template <int Q>
__device__ __forceinline__ void value_dot(const uint32_t (&m)[32], const uint32_t (&xd)[16], float (&acc)[2]) {
    acc[value_col(Q)] = __builtin_amdgcn_fdot2(bits_h2(m[Q]), bits_h2(xd[value_row(Q)]), acc[value_col(Q)], false);
}
template <int... Q>
__device__ __forceinline__ void tile_dot_(const uint32_t (&m)[32], const uint32_t (&xd)[16], float (&acc)[2],
                                          std::integer_sequence<int, Q...>) {
    (value_dot<Q>(m, xd, acc), ...);
}
__device__ __forceinline__ void tile_dot(const uint32_t (&m)[32], const uint32_t (&xd)[16], float (&acc)[2]) {
    tile_dot_(m, xd, acc, std::make_integer_sequence<int, 32>{});
}


// The previous word for lane i of an 8-lane tile group: lane - 1, or lane + 7 for i == 0 (DPP within a 16-lane row).
__device__ __forceinline__ uint32_t prev_word(uint32_t last, int i) {
    const uint32_t shr1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)last, 0x111, 0xf, 0xf, false);  // row_shr:1
    const uint32_t shl7 = (uint32_t)__builtin_amdgcn_mov_dpp((int)last, 0x107, 0xf, 0xf, false);  // row_shl:7
    return i == 0 ? shl7 : shr1;
}

__device__ __forceinline__ float bf16r(float x) {
    // round to nearest even to bf16 (experts.rs:19-21 bit form; the same value for finite inputs): gfx950's
    // v_cvt_pk_bf16_f32 and a shift back
    return (float)(__bf16)x;
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
// fp16(a * b) with the product rounded to fp32 first, as the reference does (hipcc would otherwise fuse the multiply
// and the conversion into one v_fma_mix rounding, which differs in rare double-rounding cases).
__device__ __forceinline__ uint16_t f16_of_product(float a, float b) {
    float p = a * b;
    __asm__ volatile("" : "+v"(p));
    return f32_to_f16(p);
}
// (fp16(a0 * b) low, fp16(a1 * b) high): the same roundings as f16_of_product, both conversions in one
// v_cvt_pk_f16_f32 (round to nearest even).
__device__ __forceinline__ uint32_t f16x2_of_products(float a0, float a1, float b) {
    typedef float f2_t __attribute__((ext_vector_type(2)));
    typedef _Float16 hh2_t __attribute__((ext_vector_type(2)));
    float p0 = a0 * b, p1 = a1 * b;
    __asm__ volatile("" : "+v"(p0), "+v"(p1));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2_t){p0, p1}, hh2_t));
}
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

// The value of lane (lane ^ M) for M in {1, 2, 4, 8, 16, 32}, without LDS memory: DPP quad permutes, row shifts and
// rotations inside 16-lane rows, a ds_swizzle across rows of a 32-lane half, the gfx950 permlane32 swap across halves.
template <int M>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
    const int x = (int)v;
    if constexpr (M == 1) {
        return (uint32_t)__builtin_amdgcn_mov_dpp(x, 0xB1, 0xf, 0xf, false);   // quad_perm [1, 0, 3, 2]
    } else if constexpr (M == 2) {
        return (uint32_t)__builtin_amdgcn_mov_dpp(x, 0x4E, 0xf, 0xf, false);   // quad_perm [2, 3, 0, 1]
    } else if constexpr (M == 8) {
        return (uint32_t)__builtin_amdgcn_mov_dpp(x, 0x128, 0xf, 0xf, false);  // row_ror:8 (inside a 16-lane row)
    } else if constexpr (M == 4) {
        const int up = __builtin_amdgcn_mov_dpp(x, 0x100 + M, 0xf, 0xf, false);  // row_shl: lane + M
        const int dn = __builtin_amdgcn_mov_dpp(x, 0x110 + M, 0xf, 0xf, false);  // row_shr: lane - M
        return (uint32_t)((__lane_id() & M) ? dn : up);
    } else if constexpr (M == 16) {
        // ds_swizzle bit mode (and 0x1f, or 0, xor 0x10): the LDS crossbar, no memory and no VALU slot
        return (uint32_t)__builtin_amdgcn_ds_swizzle(x, 0x1f | (0x10 << 10));
    } else {
        static_assert(M == 32, "lane_xor: M in {1, 2, 4, 8, 16, 32}");
        const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        return (uint32_t)((__lane_id() & 32) ? r[0] : r[1]);
    }
}
template <int M>
__device__ __forceinline__ float lane_xor_f(float v) {
    return __builtin_bit_cast(float, lane_xor<M>(__builtin_bit_cast(uint32_t, v)));
}

// One butterfly stage between lanes l and l ^ M, as one fma a value: v' = v * m + partner with m = +1 in the lower
// lane (lower + upper) and -1 in the upper lane (lower - upper); fma by +-1 rounds exactly as the add or subtract.
// Partners: DPP inside a 16-lane row (xor 4 as two bank-masked row shifts into one register), the gfx950 permlane16 /
// permlane32 swaps across rows (no LDS round trip, which sits on the decode launches' latency chain). A swap of
// (x, x) leaves the lower lane's own value in r[0] and the partner in r[1], the upper lane's the other way round, so
// r[0] + m r[1] is (lower + upper) in the lower lane and (lower - upper) in the upper one.
template <int M>
__device__ __forceinline__ void fwht_stage(float (&v)[2], int lane) {
    const float m = (lane & M) ? -1.f : 1.f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        if constexpr (M == 16 || M == 32) {
            const uint32_t b = __builtin_bit_cast(uint32_t, v[j]);
            const auto r = M == 16 ? __builtin_amdgcn_permlane16_swap(b, b, false, false)
                                   : __builtin_amdgcn_permlane32_swap(b, b, false, false);
            v[j] = __builtin_fmaf(__builtin_bit_cast(float, (uint32_t)r[1]), m,
                                  __builtin_bit_cast(float, (uint32_t)r[0]));
        } else if constexpr (M == 4) {
            const int x = __builtin_bit_cast(int, v[j]);
            int p = __builtin_amdgcn_update_dpp(x, x, 0x104, 0xf, 0x5, false);   // lanes 0-3, 8-11: row_shl 4
            p = __builtin_amdgcn_update_dpp(p, x, 0x114, 0xf, 0xA, false);       // lanes 4-7, 12-15: row_shr 4
            v[j] = __builtin_fmaf(v[j], m, __builtin_bit_cast(float, p));
        } else {
            v[j] = __builtin_fmaf(v[j], m, lane_xor_f<M>(v[j]));
        }
    }
}

// 128-point unnormalised Walsh-Hadamard transform of a wave64 row, two values a lane (v[j] = element 2 lane + j):
// butterflies at strides 1, 2, ..., 64, each (lower + upper, lower - upper) -- experts.rs:25-42's order, so every
// element gets the same fp32 sums as there.
__device__ __forceinline__ void fwht128_w64(float (&v)[2], int lane) {
    {
        const float a = v[0], b = v[1];
        v[0] = a + b;
        v[1] = a - b;
    }
    fwht_stage<1>(v, lane);
    fwht_stage<2>(v, lane);
    fwht_stage<4>(v, lane);
    fwht_stage<8>(v, lane);
    fwht_stage<16>(v, lane);
    fwht_stage<32>(v, lane);
}

__device__ __forceinline__ float max_nn(float a, float b) {
    float r;
    __asm__("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
// The wave-wide maximum (every lane gets it) of inputs that are never NaN, in 8 VALU operations on the shortest
// chain: v_max_f32 with the DPP operand (quad swaps, then the half-row and row mirrors: any pairing that joins the
// two halves gives every lane the maximum), then the permlane16 and permlane32 swaps. (fmaxf's NaN quieting would add
// a canonicalising max per operand.)
__device__ __forceinline__ float wave_max_nn(float v) {
    __asm__("s_nop 1\n\t"
            "v_max_f32_dpp %0, %0, %0 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
            "s_nop 1\n\t"
            "v_max_f32_dpp %0, %0, %0 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"
            "s_nop 1\n\t"
            "v_max_f32_dpp %0, %0, %0 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
            "s_nop 1\n\t"
            "v_max_f32_dpp %0, %0, %0 row_mirror row_mask:0xf bank_mask:0xf"
            : "+v"(v));
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    v = max_nn(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
    const uint32_t c = __builtin_bit_cast(uint32_t, v);
    const auto q = __builtin_amdgcn_permlane32_swap(c, c, false, false);
    return max_nn(__builtin_bit_cast(float, (uint32_t)q[0]), __builtin_bit_cast(float, (uint32_t)q[1]));
}

}  // namespace gfr
