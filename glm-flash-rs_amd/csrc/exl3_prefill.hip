// Prefill-chunk experts on gfx950: grouped trellis GEMMs on fp16 MFMA with the reference's fused epilogues.
//
// Same contract as glm-flash-rs FastExperts (src/fast_experts.rs:91-208) and its kernels (native/exl3_prefill.cu):
//   gate/up  xd[p] = fp16(H(act * suh_d)), act = limited SwiGLU(H(Xg[p] @ Wg) * svh_g, H(Xu[p] @ Wu) * svh_u)
//   down     y[p]  = H(xd[p] @ Wd) * svh_d                                                       (fp32)
// for every routed pair p (H = the 128-block Hadamard / sqrt(128)), each output one full-K fp32 accumulation chain
// (exl3_prefill.cu:14-23: no split-K partials), deterministic and row-independent.
//
// MI355X design:
//   * Y^T = W^T X^T on v_mfma_f32_16x16x32_f16: the trellis-decoded weights are the A operand, decoded straight into
//     MFMA registers. A lane that owns column c of a 16x16 tile and one pair of its words (4i + 2g, 4i + 2g + 1)
//     holds exactly 8 values of that column -- rows {2l + 8 + h, 2l + h} -- which is one A-fragment lane
//     (16 n x 8 k) once k is taken in the pair order of exl3_format.hpp (pair_row); the token rows (B operand) are
//     staged in LDS in that same order, so no weight ever goes through LDS and none is decoded twice in a workgroup.
//   * workgroup = 4 waves, a tile of BM member rows of one expert x 128 (gate/up: both matrices) or 256 (down)
//     output columns, two workgroups a CU; each wave owns 64 columns x BM rows (4 BM / 16 MFMA 16x16 accumulators),
//     K in steps of 32, multi-stage direct-to-LDS staging and a register pipeline (next step's decode during this
//     step's MFMAs). BM = 176 for K = 4: the trellis decode (VALU) is amortised over more rows, an expert of 512
//     members takes 3 passes instead of 4, and 244 VGPRs and two workgroups' stages (2 x 80.6 KB) still fit.
//     K = 2, 3 and 5 decode their fragments directly as well (176, 160 and 144 rows, the most without spills).
//   * the 128 columns of a gate/up item, and each 128 of a down item, are one Hadamard block, so the epilogue
//     (transforms, scales, SwiGLU) runs in the workgroup: accumulators -> LDS (32 rows at a time) -> registers with
//     8 consecutive values a lane and four rows a wave, so that three of the seven butterfly stages stay in registers.
//   * work items (distinct expert u, pass of BM members) come from a plan kernel (member counts by parallel search,
//     scan); grid = items x column groups, no empty launches past the plan.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>
#include "exl3_format.hpp"
#include "launch.hpp"
#include "prefill.hpp"
#include "grouping_body.hpp"

namespace gfr {

// Member rows a full-K item at each width: the most that keep two workgroups' stages in LDS and the kernel within
// 256 VGPRs without spills (K = 4: 244 VGPRs at 176 rows, 2 x 80.6 KB of LDS; K = 3 at 160 rows: 252; K = 5 at
// 144: 256; K = 2 at 176: 239). Larger items decode each weight tile for more rows.
#ifndef PF_BM2_ROWS
#define PF_BM2_ROWS 176
#endif
#ifndef PF_BM3_ROWS
#define PF_BM3_ROWS 160
#endif
#ifndef PF_BM4_ROWS
#define PF_BM4_ROWS 176
#endif
#ifndef PF_BM5_ROWS
#define PF_BM5_ROWS 144
#endif
constexpr int PF_BM2 = PF_BM2_ROWS, PF_BM3 = PF_BM3_ROWS, PF_BM4 = PF_BM4_ROWS, PF_BM5 = PF_BM5_ROWS;
constexpr int pf_bm_for(int bits) { return bits == 2 ? PF_BM2 : bits == 3 ? PF_BM3 : bits == 4 ? PF_BM4 : PF_BM5; }
constexpr int PF_MAXU = 1024;       // distinct experts a window (grid / plan bound)

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

// ---- plan -----------------------------------------------------------------------------------------------------
// ucnt[u] = members of distinct expert u (the first -1 of its members row, found by a parallel search: 64 probes a
// round); items[k] = (u << 16) | pass for the passes of BM members, in u order; plan[0] = item count.
__global__ void __launch_bounds__(1024) prefill_plan_kernel(const int* __restrict__ uids,
                                                            const int* __restrict__ ucount,
                                                            const int* __restrict__ members, int maxm, int E,
                                                            int maxu, int bm, int* __restrict__ ucnt,
                                                            int* __restrict__ items, int* __restrict__ plan) {
    __shared__ int passes[PF_MAXU];
    __shared__ int scan_w[16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwv = blockDim.x >> 6;
    const int count = ucount[0];
    for (int u = wave; u < maxu; u += nwv) {
        int n = 0;
        if (u < count && uids[u] < E) {
            const int* m = members + (size_t)u * maxm;
            int lo = 0, hi = maxm;                       // the first -1 lies in [lo, hi]
            while (hi - lo > 1) {
                const int stride = (hi - lo + 63) / 64;
                const int pos = lo + lane * stride;
                const bool ok = pos < hi && m[pos] >= 0;
                const uint64_t bal = __ballot(ok);
                const int last = bal ? 63 - __builtin_clzll(bal) : -1;   // members come first
                if (last < 0) { hi = lo; break; }        // m[lo] < 0
                const int nlo = lo + last * stride;
                hi = min(hi, nlo + stride);
                lo = nlo + 1;
                if (lo >= hi) break;
            }
            // lo = first unprobed position after the last member found, hi = bound; settle the last one
            n = (lo < maxm && lo < hi && m[lo] >= 0) ? lo + 1 : lo;
            if (hi == 0) n = 0;
        }
        if (lane == 0) {
            ucnt[u] = n;
            passes[u] = (n + bm - 1) / bm;
        }
    }
    __syncthreads();
    // exclusive scan of passes over u (blocks of blockDim.x)
    int base = 0;
    for (int u0 = 0; u0 < maxu; u0 += blockDim.x) {
        const int u = u0 + threadIdx.x;
        int x = u < maxu ? passes[u] : 0;
        int v = x;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int o = __shfl_up(v, d, 64);
            if (lane >= d) v += o;
        }
        if (lane == 63) scan_w[wave] = v;
        __syncthreads();
        int off = 0, all = 0;
        for (int w = 0; w < nwv; ++w) {
            const int s = scan_w[w];
            if (w < wave) off += s;
            all += s;
        }
        __syncthreads();
        const int first = base + off + v - x;
        for (int k = 0; k < x; ++k) items[first + k] = (u << 16) | k;
        base += all;
    }
    if (threadIdx.x == 0) plan[0] = base;
}

// ---- rows of 128 values, 8 contiguous values a lane (the rotation and the GEMM epilogues) -----------------------
// Lane l holds elements 8 j .. 8 j + 7 of a row, j = (l & 3) | ((l >> 3) & 3) << 2; lane bits 2 and 5 pick one of
// four rows, so a wave transforms four rows at once. Element bits 0-2 are in registers, bits 3, 4, 5, 6 are lane
// bits 0, 1, 3, 4 (lane xor 1, 2, 8, 16: DPP quad permutes, row_ror:8 and a permlane16 swap).
__device__ __forceinline__ int l8_j(int lane) { return (lane & 3) | ((lane >> 3) & 3) << 2; }
__device__ __forceinline__ int l8_row(int lane) { return ((lane >> 2) & 1) | ((lane >> 5) & 1) << 1; }

// One butterfly stage across lanes (lane xor M) on values held with a lane sign: every lane computes u + m p, with
// p the partner's value and m = -1 on the upper lane of the pair, +1 on the lower. The lower lane gets the true
// lower + upper; the upper lane gets lower - upper negated. Partners of a stage share their sign so far (they differ
// only in this stage's lane bit), so the plain +-1 multiplier is right at every stage, and after the four stages the
// lane holds sigma * H(x) with sigma = (-1)^popcount(lane & 0b11011) (lane_sign). Negation is exact, so every value is
// bit for bit +- the reference's butterfly result. Stages xor 1, 2, 8 are one v_fmac_f32_dpp a value (the DPP read of
// a VGPR written by the VALU just before needs two wait states: the s_nop); xor 16 goes through ds_swizzle.
#define GFR_DPP8(CTRL)                                                                                          \
    __asm__ volatile("s_nop 1\n\t"                                                                            \
                     "v_fmac_f32_dpp %0, %0, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                        \
                     "v_fmac_f32_dpp %1, %1, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                        \
                     "v_fmac_f32_dpp %2, %2, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                        \
                     "v_fmac_f32_dpp %3, %3, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                        \
                     "v_fmac_f32_dpp %4, %4, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                        \
                     "v_fmac_f32_dpp %5, %5, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                        \
                     "v_fmac_f32_dpp %6, %6, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                        \
                     "v_fmac_f32_dpp %7, %7, %8 " CTRL " row_mask:0xf bank_mask:0xf"                              \
                     : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]),        \
                       "+v"(v[7])                                                                                \
                     : "v"(m))
// The 8 values of a stage in one block: a DPP read of a VGPR written by the VALU just before needs two wait states
// (the s_nop); inside the block each value was last written 8 instructions earlier.
template <int M>
__device__ __forceinline__ void fwht_l8_cross(float (&v)[8], float m) {
    if constexpr (M == 1) {
        GFR_DPP8("quad_perm:[1,0,3,2]");
    } else if constexpr (M == 2) {
        GFR_DPP8("quad_perm:[2,3,0,1]");
    } else if constexpr (M == 8) {
        GFR_DPP8("row_ror:8");
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = __builtin_fmaf(lane_xor_f<M>(v[i]), m, v[i]);
    }
}
#undef GFR_DPP8
// sigma of the lane (see fwht_l8_cross): the sign a transformed value carries
__device__ __forceinline__ float lane_sign(int lane) { return (__popc(lane & 0x1b) & 1) ? -1.f : 1.f; }

// 128-point unnormalised Walsh-Hadamard transform of four rows a wave (butterflies at strides 1, 2, ..., 64, each
// (lower + upper, lower - upper) in fp32, as experts.rs:25-42), returned times lane_sign(lane).
__device__ __forceinline__ void fwht128_l8(float (&v)[8], int lane) {
#pragma unroll
    for (int st = 1; st < 8; st <<= 1)
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (!(i & st)) {
                const float a = v[i], b = v[i + st];
                v[i] = a + b;
                v[i + st] = a - b;
            }
    fwht_l8_cross<1>(v, (lane & 1) ? -1.f : 1.f);
    fwht_l8_cross<2>(v, (lane & 2) ? -1.f : 1.f);
    fwht_l8_cross<8>(v, (lane & 8) ? -1.f : 1.f);
    fwht_l8_cross<16>(v, (lane & 16) ? -1.f : 1.f);
}

// Round two values to bf16 (round to nearest even) with one v_cvt_pk_bf16_f32.
typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
typedef float f2v_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void bf16r2(float& a, float& b) {
    const uint32_t d = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2v_t){a, b}, bf2_t));
    a = __builtin_bit_cast(float, d << 16);
    b = __builtin_bit_cast(float, d & 0xffff0000u);
}

// fp16(v * scale) of a row held as above (scale = lane_sign / sqrt(128) undoes the transform's lane sign), stored in the pair order of pair_row (K != 2) into a 128-value block:
// pair m of k tile kt = (x[m + 8] low, x[m] high), so the lane of the tile's first half (j even) pairs with its
// neighbour (lane xor 1) that holds the second; the even lane stores pairs 0-3, the odd lane pairs 4-7.
__device__ __forceinline__ void store_pairs_l8(uint16_t* block, const float (&v)[8], int lane, float scale) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        w[i] = f16x2_of_products(v[2 * i], v[2 * i + 1], scale);
    const int j = l8_j(lane);
    const bool odd = j & 1;
    const uint32_t r0 = lane_xor<1>(odd ? w[0] : w[2]), r1 = lane_xor<1>(odd ? w[1] : w[3]);
    const uint32_t L0 = odd ? w[2] : r0, L1 = odd ? w[3] : r1;   // the x[m + 8] (low halves)
    const uint32_t H0 = odd ? r0 : w[0], H1 = odd ? r1 : w[1];   // the x[m] (high halves)
    uint4 o;
    o.x = __builtin_amdgcn_perm(H0, L0, 0x05040100u);
    o.y = __builtin_amdgcn_perm(H0, L0, 0x07060302u);
    o.z = __builtin_amdgcn_perm(H1, L1, 0x05040100u);
    o.w = __builtin_amdgcn_perm(H1, L1, 0x07060302u);
    *reinterpret_cast<uint4*>(block + (j >> 1) * 16 + (j & 1) * 8) = o;
}


// rot_in for prefill chunks (exl3.cu:224-241, bit for bit): one wave a (token, 128-block), every (EXL3 slot, matrix)
// row of it four at a time in the 8-values-a-lane layout of fwht128_l8 (the reference's butterfly order, so the
// bits are rot_in's); x read once, the rotated rows written in pair order (the MFMA B operand's k order).
template <int MAXR>   // rounds of four (slot, matrix) rows: exl3_slots * mats <= 4 MAXR
__global__ void __launch_bounds__(256) prefill_rot_kernel(const uint16_t* __restrict__ x, int x_stride,
                                                          const int* __restrict__ pick,
                                                          const uint16_t* __restrict__ suh0,
                                                          const uint16_t* __restrict__ suh1, uint16_t* __restrict__ out0,
                                                          uint16_t* __restrict__ out1, int K, int rows, int slots,
                                                          int exl3_slots, int mats) {
    const int lane = threadIdx.x & 63;
    const int task = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int KB = K / 128, row = task / KB, blk = task % KB;
    if (row >= rows) return;
    const int j8 = l8_j(lane), r4 = l8_row(lane);
    const int k = blk * 128 + 8 * j8;
    float xf[8];
    {
        const uint4 xv = *reinterpret_cast<const uint4*>(x + (size_t)row * x_stride + k);
        const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xf[2 * i] = bf16_to_f32((uint16_t)xw[i]);
            xf[2 * i + 1] = bf16_to_f32((uint16_t)(xw[i] >> 16));
        }
    }
    // every round's expert and scales in flight before the first transform (rows = (slot, matrix), four a round)
    const int nrow = exl3_slots * mats;
    const int pk = lane < exl3_slots ? pick[row * slots + lane] : 0;
    uint4 sv[MAXR];
#pragma unroll
    for (int rd = 0; rd < MAXR; ++rd) {
        const int ri = rd * 4 + r4;
        const int sl = ri < nrow ? (mats == 2 ? ri >> 1 : ri) : 0, m = ri < nrow ? (mats == 2 ? ri & 1 : 0) : 0;
        const int e = __shfl(pk, sl, 64);
        if (rd * 4 < nrow) sv[rd] = *reinterpret_cast<const uint4*>((m ? suh1 : suh0) + (size_t)e * K + k);
    }
#pragma unroll
    for (int rd = 0; rd < MAXR; ++rd) {
        if (rd * 4 >= nrow) break;
        const int ri = rd * 4 + r4;
        const bool valid = ri < nrow;
        const int sl = valid ? (mats == 2 ? ri >> 1 : ri) : 0, m = valid ? (mats == 2 ? ri & 1 : 0) : 0;
        const int p = row * slots + sl;
        const uint32_t sw[4] = {sv[rd].x, sv[rd].y, sv[rd].z, sv[rd].w};
        float v[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = xf[2 * i] * f16_to_f32((uint16_t)sw[i]);
            v[2 * i + 1] = xf[2 * i + 1] * f16_to_f32((uint16_t)(sw[i] >> 16));
        }
        fwht128_l8(v, lane);
        if (valid) store_pairs_l8((m ? out1 : out0) + (size_t)p * K + blk * 128, v, lane, lane_sign(lane) * HAD_SCALE);
    }
}

// The same rotation with two 128-blocks of a token a wave and no idle rows: lanes of rows 0, 1 (lane bits 2 and 5,
// see l8_row) take block 2 b and rows 2, 3 block 2 b + 1, and a lane keeps its matrix (MATS = 2: row & 1) in every
// round, so the (slot, matrix) rows of a block fill the rounds exactly: round r is slot r (MATS = 2) or slots 2 r and
// 2 r + 1 (MATS = 1). x * suh is exact in fp32 (bf16 times fp16), so it is one v_fma_mix_f32 from the fp16 scale;
// the rest is rot_in's arithmetic as above, bit for bit. K / 128 even.
// One wave's task (row, block pair bp); picks() returns the row's expert of slot `lane` on lanes below exl3_slots,
// called once the token's loads are issued.
template <int MATS, typename Picks>
__device__ __forceinline__ void rot2_task(const uint16_t* __restrict__ x, int x_stride, Picks picks,
                                          const uint16_t* __restrict__ suh0, const uint16_t* __restrict__ suh1,
                                          uint16_t* __restrict__ out0, uint16_t* __restrict__ out1, int K, int row,
                                          int bp, int slots, int exl3_slots) {
    const int lane = threadIdx.x & 63;
    const int j8 = l8_j(lane), r4 = l8_row(lane);
    const int blk = 2 * bp + (r4 >> 1), k = blk * 128 + 8 * j8;
    const int m = MATS == 2 ? (r4 & 1) : 0;
    const uint16_t* suh = m ? suh1 : suh0;
    uint16_t* outm = (m ? out1 : out0) + (size_t)blk * 128;
    const uint4 xv = *reinterpret_cast<const uint4*>(x + (size_t)row * x_stride + k);
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
    float xf[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        xf[2 * i] = bf16_to_f32((uint16_t)xw[i]);
        xf[2 * i + 1] = bf16_to_f32((uint16_t)(xw[i] >> 16));
    }
    const int nrd = MATS == 2 ? exl3_slots : (exl3_slots + 1) / 2;
    const int pk = picks();
    const float st = lane_sign(lane) * HAD_SCALE;
    constexpr int RC = 8;                                   // rounds a chunk: their scales in flight together
    for (int r0 = 0; r0 < nrd; r0 += RC) {
        uint4 sv[RC];
#pragma unroll
        for (int q = 0; q < RC; ++q) {
            const int rd = min(r0 + q, nrd - 1);
            const int sl = MATS == 2 ? rd : min(2 * rd + (r4 & 1), exl3_slots - 1);
            const int e = MATS == 2 ? __builtin_amdgcn_readlane(pk, sl) : __shfl(pk, sl, 64);
            sv[q] = *reinterpret_cast<const uint4*>(suh + (size_t)e * K + k);
        }
        // keep the chunk's scale loads together: left alone, the compiler sinks each into its round, one memory
        // round trip a round
#pragma unroll
        for (int q = 0; q < RC; ++q) __asm__ volatile("" : "+v"(sv[q].x), "+v"(sv[q].y), "+v"(sv[q].z), "+v"(sv[q].w));
#pragma unroll
        for (int q = 0; q < RC; ++q) {
            const int rd = r0 + q;
            if (rd >= nrd) break;
            const int sl = MATS == 2 ? rd : 2 * rd + (r4 & 1);
            const uint32_t sw[4] = {sv[q].x, sv[q].y, sv[q].z, sv[q].w};
            float v[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                __asm__("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[0,1,0]" : "=v"(v[2 * i]) : "v"(xf[2 * i]), "v"(sw[i]));
                __asm__("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]"
                        : "=v"(v[2 * i + 1]) : "v"(xf[2 * i + 1]), "v"(sw[i]));
            }
            fwht128_l8(v, lane);
            if (MATS == 2 || sl < exl3_slots) store_pairs_l8(outm + (size_t)(row * slots + sl) * K, v, lane, st);
        }
    }
}

template <int MATS>
__global__ void __launch_bounds__(256) prefill_rot2_kernel(const uint16_t* __restrict__ x, int x_stride,
                                                           const int* __restrict__ pick,
                                                           const uint16_t* __restrict__ suh0,
                                                           const uint16_t* __restrict__ suh1,
                                                           uint16_t* __restrict__ out0, uint16_t* __restrict__ out1,
                                                           int K, int rows, int slots, int exl3_slots) {
    const int lane = threadIdx.x & 63;
    const int task = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int KP = K / 256, row = task / KP, bp = task % KP;
    if (row >= rows) return;
    rot2_task<MATS>(x, x_stride, [&] { return lane < exl3_slots ? pick[row * slots + lane] : 0; }, suh0, suh1, out0,
                    out1, K, row, bp, slots, exl3_slots);
}

// Route + group + item plan and the rotation of every EXL3 pair in one launch, for the windows route_group_kernel
// takes (K / 128 even). Workgroup 0 does route_group_kernel's work (route_group_body; its dynamic LDS); the others
// take prefill_rot2_kernel's tasks, a wave's task routing its token with the same router (route_load / route_pick on
// the same logits, so the same picks as workgroup 0 writes) while its token loads are in flight. Nothing of one
// part waits for the other.
template <int MATS>
__global__ void __launch_bounds__(512) route_group_rot_kernel(const float* __restrict__ logits, int rows, int routed,
                                                              int topk, int* __restrict__ picks,
                                                              float* __restrict__ weights, int* __restrict__ ids,
                                                              int* __restrict__ count, int* __restrict__ members,
                                                              int maxm, int bm, int* __restrict__ plan_ucnt,
                                                              int* __restrict__ plan_items, int* __restrict__ plan,
                                                              int plan_E, RouteGate gate,
                                                              const uint16_t* __restrict__ x, int x_stride,
                                                              const uint16_t* __restrict__ suh0,
                                                              const uint16_t* __restrict__ suh1,
                                                              uint16_t* __restrict__ out0, uint16_t* __restrict__ out1,
                                                              int K, int exl3_slots) {
    extern __shared__ uint32_t lds[];
    __shared__ __attribute__((aligned(16))) int scan_scratch[16];
    if (blockIdx.x == 0) {
        route_group_body(lds, scan_scratch, logits, rows, routed, topk, picks, weights, ids, count, members, maxm, bm,
                         plan_ucnt, plan_items, plan, plan_E, gate);
        return;
    }
    const int task = (blockIdx.x - 1) * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int KP = K / 256, row = task / KP, bp = task % KP;
    if (row >= rows) return;
    const int lane = threadIdx.x & 63;
    rot2_task<MATS>(x, x_stride,
                    [&] {
                        int pick;
                        float weight;
                        route_token_regs(logits + (size_t)row * routed, routed, topk, routed, pick, weight, gate,
                                         false);
                        return lane < exl3_slots ? pick : 0;
                    },
                    suh0, suh1, out0, out1, K, row, bp, topk + 1, exl3_slots);
}

// The large-window grouping's scatter launch (group_scatter_body, workgroups 0 .. E - 1) and the rotation
// (prefill_rot2_kernel's tasks, the workgroups after them) in one launch: both read only the picks of the launches
// before, and neither waits for the other.
template <int MATS>
__global__ void __launch_bounds__(256) group_scatter_rot_kernel(const int* __restrict__ picks, int rows, int slots,
                                                                int E, const uint32_t* __restrict__ bits,
                                                                const uint8_t* __restrict__ first,
                                                                const int* __restrict__ prefix,
                                                                const int* __restrict__ counts,
                                                                int* __restrict__ ids, int* __restrict__ count,
                                                                int* __restrict__ members, int maxm, int bm,
                                                                int* __restrict__ plan_ucnt,
                                                                int* __restrict__ plan_items, int* __restrict__ plan,
                                                                int plan_E, const uint16_t* __restrict__ x,
                                                                int x_stride, const uint16_t* __restrict__ suh0,
                                                                const uint16_t* __restrict__ suh1,
                                                                uint16_t* __restrict__ out0,
                                                                uint16_t* __restrict__ out1, int K, int exl3_slots) {
    __shared__ __attribute__((aligned(16))) int scan_scratch[16];
    __shared__ int tot_sh[4];
    if ((int)blockIdx.x < E) {
        group_scatter_body(blockIdx.x, scan_scratch, tot_sh, picks, rows, slots, E, bits, first, prefix, counts, ids,
                           count, members, maxm, bm, plan_ucnt, plan_items, plan, plan_E);
        return;
    }
    const int lane = threadIdx.x & 63;
    const int task = ((int)blockIdx.x - E) * 4 + (threadIdx.x >> 6);
    const int KP = K / 256, row = task / KP, bp = task % KP;
    if (row >= rows) return;
    rot2_task<MATS>(x, x_stride, [&] { return lane < exl3_slots ? picks[row * slots + lane] : 0; }, suh0, suh1, out0,
                    out1, K, row, bp, slots, exl3_slots);
}

// ---- GEMM --------------------------------------------------------------------------------------------------------
struct PrefillArgs {
    const uint16_t* x0;      // rows [P][Kin] fp16 in pair order, matrix 0 (gate, or the down input xd)
    const uint16_t* x1;      // of matrix 1 (up); == x0 when the input rotations are shared
    const uint32_t* t0;      // trellis [E][Kin/16][N/16][32]
    const uint32_t* t1;
    const int* uids;
    const int* members;
    const int* ucnt;
    const int* items;
    const int* plan;
    int Kin, N, maxm, slots;
    const uint16_t* sv0;     // gate/up: svh_g, svh_u, suh_d; down: svh_d
    const uint16_t* sv1;
    const uint16_t* sd;
    uint16_t* xd;            // gate/up output [P][N] fp16 in pair order
    float* y;                // down output [P][N]
    float limit;
    int sk, P;               // split-K launches: K splits, pairs
    float* z;                // split-K output: partial sums [mats][sk][P][N] fp32 (no epilogue)
};

// The A fragment of one 16-column trellis tile over two k tiles (K = 4): lane l owns column c = l % 16 of the tile
// (format lane i = c % 8, value half c / 8) for k tile q / 2 and word pair g = q % 2 (q = l / 16): words 4i + 2g and
// 4i + 2g + 1 hold its 8 values, rows (2l + 8 + h, 2l + h) for l = 2g, 2g + 1 -- the pair order of pair_row, the order
// the token rows are staged in. tw: the tile's words of the two k tiles in LDS, [2][32].
// The words of that fragment: the previous word and the lane's word pair of its k tile.
__device__ __forceinline__ void frag4_words(const uint32_t* tw, int lane, uint32_t& p0, uint32_t& w0, uint32_t& w1) {
    const int c = lane & 15, i = c & 7, q = lane >> 4, kt = q >> 1, g = q & 1;
    const uint32_t* w = tw + kt * 32;
    const int w0i = 4 * i + 2 * g;
    p0 = w[(w0i + 31) & 31];
    const uint2 ww = *reinterpret_cast<const uint2*>(w + w0i);
    w0 = ww.x;
    w1 = ww.y;
}
// Its four packed state pairs (each two 16-bit windows of one column, pair order).
__device__ __forceinline__ void frag4_states(uint32_t p0, uint32_t w0, uint32_t w1, int lane, uint32_t (&s)[4]) {
    const uint32_t sel = ((lane & 15) >> 3) ? 0x02010100u : 0x04030302u;   // value half: (s6,s4)/(s7,s5) or (s2,s0)/(s3,s1)
    {
        const uint32_t a = __builtin_amdgcn_alignbit(p0, w0, 4), b = p0 >> 4;
        s[0] = __builtin_amdgcn_perm(b, a, sel);
        s[1] = __builtin_amdgcn_perm(p0, w0, sel);
    }
    {
        const uint32_t a = __builtin_amdgcn_alignbit(w0, w1, 4), b = w0 >> 4;
        s[2] = __builtin_amdgcn_perm(b, a, sel);
        s[3] = __builtin_amdgcn_perm(w0, w1, sel);
    }
}
__device__ __forceinline__ h8_t a_fragment4(const uint32_t* tw, int lane) {
    uint32_t p0, w0, w1, s[4];
    frag4_words(tw, lane, p0, w0, w1);
    frag4_states(p0, w0, w1, lane, s);
    h8_t f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const h2_t v = decode_pair(s[j]);
        f[2 * j] = v[0];
        f[2 * j + 1] = v[1];
    }
    return f;
}

// The same fragment for K = 2, 3 and 5 (the prefill path stages its rows in the K != 2 pair order of pair_row at
// every width). The lane's two value
// groups (l = 2g and 2g + 1) are each 4 consecutive values 8 l + 4 half .. + 3 of format lane i; their windows end
// at bits (v + 1) K of the lane's stream and span 3 K + 16 <= 31 bits, so one funnel shift of two adjacent words
// (alignbit by a per-lane amount, the same for every tile) holds all four: value v0 + d at bits (3 - d) K.
// fragk_words: the 2 x 2 words of the lane's groups (the word before the group's last bit wraps within the k tile,
// as lane 0's previous word is lane 7's last); fragk_shifts: the two funnel shifts.
template <int K>
__device__ __forceinline__ void fragk_groups(int lane, int t, int& lo, int& sh) {
    const int c = lane & 15, half = c >> 3, g = (lane >> 4) & 1, i = c & 7;
    const int v0 = 8 * (2 * g + t) + 4 * half;
    const int e = (v0 + 4) * K, hiw = (e - 1) >> 5;
    lo = K * i + hiw;                                   // the word holding the group's last bit
    sh = 32 * (hiw + 1) - e;
}
template <int K>
__device__ __forceinline__ void fragk_shifts(int lane, uint32_t (&sh)[2]) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        int lo, s;
        fragk_groups<K>(lane, t, lo, s);
        sh[t] = (uint32_t)s;
    }
}
template <int K>
__device__ __forceinline__ void fragk_words(const uint32_t* tw, int lane, uint32_t (&wd)[4]) {
    const uint32_t* w = tw + (lane >> 5) * (8 * K);     // k tile q / 2
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        int lo, s;
        fragk_groups<K>(lane, t, lo, s);
        wd[2 * t] = w[(lo + 8 * K - 1) % (8 * K)];
        wd[2 * t + 1] = w[lo];
    }
}
// Its four packed state pairs, st[2 t + h] = (window of v0 + h + 2 low, window of v0 + h high).
template <int K>
__device__ __forceinline__ void fragk_states(const uint32_t (&wd)[4], const uint32_t (&sh)[2], uint32_t (&st)[4]) {
    static_assert(3 * K + 16 <= 32, "four windows in one funnel word");
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const uint32_t W = __builtin_amdgcn_alignbit(wd[2 * t], wd[2 * t + 1], sh[t]);
        st[2 * t] = ((W << (16 - 3 * K)) & 0xFFFF0000u) | ((W >> K) & 0xFFFFu);
        st[2 * t + 1] = ((W << (16 - 2 * K)) & 0xFFFF0000u) | (W & 0xFFFFu);
    }
}
template <int K>
__device__ __forceinline__ h8_t a_fragmentk(const uint32_t* tw, int lane, const uint32_t (&sh)[2]) {
    uint32_t wd[4], s[4];
    fragk_words<K>(tw, lane, wd);
    fragk_states<K>(wd, sh, s);
    h8_t f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const h2_t v = decode_pair(s[j]);
        f[2 * j] = v[0];
        f[2 * j + 1] = v[1];
    }
    return f;
}

// 16-byte direct-to-LDS load: lane i's 16 bytes land at lds_base + 16 i (lds_base uniform). Written as inline asm:
// the compiler treats its builtin as an LDS store of unknown address and puts s_waitcnt vmcnt(0) before every later
// LDS read, which drains the whole load pipeline each step; here the kernels wait for their stages themselves
// (wait_vmcnt), and loads complete in order, so any wait the compiler adds for its own loads only waits longer.
__device__ __forceinline__ void load_lds16(const void* g, void* lds_base) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds_base);
    __asm__ volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" :: "v"(g), "{m0}"(m0) : "memory");
}

// The same load in the scalar-base form: lane i reads sbase + voff_i (32-bit unsigned per-lane offset), so a
// per-step advance is one 64-bit scalar add and the LDS destination (m0) stays in scalar registers.
__device__ __forceinline__ void load_lds16_s(uint64_t sbase, uint32_t voff, uint32_t m0) {
    __asm__ volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" :: "v"(voff), "s"(sbase), "{m0}"(m0) : "memory");
}
__device__ __forceinline__ uint64_t uniform64(uint64_t v) {
    // readfirstlane returns int: through uint32_t, so that the low word is not sign-extended into the high one
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (uint64_t)lo | ((uint64_t)hi << 32);
}

// Workgroup barrier for LDS-only hand-offs: this wave's LDS operations complete, then s_barrier. Unlike
// __syncthreads() it does not wait for outstanding global loads (the staged direct-to-LDS loads of later steps).
__device__ __forceinline__ void lds_barrier() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// s_waitcnt vmcnt(n), other counters unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Item (u, pass) x column group cg. MATS = 2: gate + up, 128 columns of each (waves 0-1 gate, 2-3 up); MATS = 1:
// down, 256 columns (wave w: columns 64 w ..). Rows: the pass's BM members of expert u (pairs). Each wave owns 64
// columns (4 trellis tiles) x BM rows: a step of 32 k is 4 A fragments decoded in registers against BM / 16 B
// fragments, so every decoded fragment feeds BM / 16 MFMAs. Software pipeline: while step s multiplies, the wave
// decodes step s + 1's A fragments into a second register set and keeps a ring of B fragments D reads ahead of the
// MFMAs; direct-to-LDS loads run NS - 1 steps ahead of the step that reads them. With BM = 128 two workgroups share
// a CU, so one wave's decode (VALU) overlaps the other's MFMAs on each SIMD. A staged row keeps its four 16-byte
// chunks XOR-swizzled by (row >> 1) & 3 to spread the B-fragment reads over the banks.
// SPLIT: (item, column group, K split) programs over a.sk contiguous k ranges, each writing its raw partial sums to
// a.z in the decode path's split layout (its epilogue kernels add the splits in order); for windows too small to
// fill the GPU with full-K items.
template <int MATS, int K, int BM, bool SPLIT = false>
__global__ void __launch_bounds__(256, BM == 256 ? 1 : 2) prefill_gemm_kernel(const PrefillArgs a) {
    constexpr int NCOLS = MATS == 2 ? 128 : 256, RB = BM / 16;
    constexpr int OCC = BM == 256 ? 1 : 2;
    constexpr int NS = SPLIT ? 4 : OCC == 1 ? (MATS == 2 ? 4 : 6) : (MATS == 2 ? 3 : 4);
    constexpr int XBUF = BM * 64;                        // one matrix's rows of a step (2 k tiles, pair order)
    constexpr int TBUF = 16 * 2 * 32 * K;                // the workgroup's 16 tiles x 2 k tiles of words
    constexpr int STAGE = MATS * XBUF + TBUF;
    constexpr int ER = BM % 64 ? 32 : BM / 4, EPITCH = 256 + 8;   // epilogue: ER rows of 256 fp32 columns at a time
    constexpr int LDS_EPI = SPLIT ? 0 : ER * EPITCH * 4;
    constexpr int LDS_BYTES = NS * STAGE > LDS_EPI ? NS * STAGE : LDS_EPI;
    constexpr int XLOADS = (MATS * RB + 3) / 4;          // direct loads of rows a wave a step (the last repeated)
    constexpr int TL = (K + 3) / 4;                      // direct loads of trellis words a wave a step
    constexpr int LOADS = XLOADS + TL;
    static_assert((BM == 256 || BM == 176 || BM == 160 || BM == 144 || BM == 128 || BM == 32) && NS <= 8, "tile shape");
    __shared__ __attribute__((aligned(16))) unsigned char lds[LDS_BYTES];
    __shared__ int rows_sh[BM];

    const int ncg = a.N / NCOLS;
    // XCD-aware order: the hardware deals consecutive workgroups to the 8 XCDs in turn; renumber so that each XCD gets
    // a contiguous range of (item, column group[, split]) -- an item's column groups then share one L2 (its token
    // rows). The grid is sized for the most items a window can have; the window's real programs (nact, known once
    // the plan has run) are spread over all 8 XCDs, taken by the first-dispatched workgroups.
    const int nsk = SPLIT ? a.sk : 1;
    const int nact = a.plan[0] * ncg * nsk, per = (nact + 7) >> 3;
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    const int full = nact & 7 ? nact & 7 : 8;            // XCDs holding `per` programs (the rest hold per - 1)
    if (slot >= (xcd < full ? per : per - 1)) return;
    const int logical = (xcd < full ? xcd * per : full * per + (xcd - full) * (per - 1)) + slot;
    const int item = logical / (ncg * nsk), cg = logical / nsk % ncg, split = logical % nsk;
    const int it = a.items[item];
    const int u = it >> 16, pass = it & 0xffff;
    const int e = a.uids[u];
    // the expert's members split evenly over its ceil(cnt / BM) passes; row blocks past nrows skip their MFMAs
    const int ucnt = a.ucnt[u], npass = (ucnt + BM - 1) / BM;
    const int rbeg = pass * ucnt / npass, nrows = (pass + 1) * ucnt / npass - rbeg;
    const int nblk = (nrows + 15) >> 4;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    {
        const int* mrow = a.members + (size_t)u * a.maxm + rbeg;
        const int c0 = mrow[0];
        const int p0 = (c0 >> 5) * a.slots + (c0 & 31);
        const int code = tid < nrows ? mrow[tid] : -1;
        if (tid < BM) rows_sh[tid] = code >= 0 ? (code >> 5) * a.slots + (code & 31) : p0;   // padding: member 0
    }
    __syncthreads();

    const int KT = a.Kin >> 4, NT = a.N >> 4, S = KT / 2 / nsk, s0 = split * S;   // this program's steps s0 ..
    const int col0 = cg * NCOLS;
    const int mat = MATS == 2 ? wave >> 1 : 0;
    const int wtile0 = MATS == 2 ? (wave & 1) * 4 : wave * 4;   // the wave's first tile within its matrix's columns
    const int stile0 = MATS == 2 ? mat * 8 + wtile0 : wtile0;    // ... within the staged tiles

    // the lane's direct loads: rows (XLOADS of them, 16 rows a load) and one trellis chunk, each as a uniform 64-bit
    // base (advanced per step with scalar adds) and a per-lane 32-bit byte offset (the host keeps every offset below
    // 2^32); the LDS destinations are uniform too
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t lds_u = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds;
    uint64_t xbase[XLOADS];
    uint32_t xoff[XLOADS];
#pragma unroll
    for (int j = 0; j < XLOADS; ++j) {
        const int t = min(wv * XLOADS + j, MATS * RB - 1);     // 16-row block of the stage (MATS * RB of them)
        const int m = t / RB, row = (t % RB) * 16 + lane / 4, pos = lane & 3;
        const int c = pos ^ ((row >> 1) & 3);              // the global chunk this LDS position holds
        xbase[j] = uniform64((uint64_t)(uintptr_t)(m ? a.x1 : a.x0) + (uint64_t)s0 * 64);
        xoff[j] = (uint32_t)rows_sh[row] * (uint32_t)(a.Kin * 2) + (uint32_t)((c >> 1) * 32 + (c & 1) * 16);
    }
    // trellis words: 32 blocks (tile, k tile) of 32 K bytes, K loads of 64 16-byte chunks; wave w issues loads
    // w, w + 4, ... (the last one repeated where K is not a multiple of 4: the same bytes to the same place). The
    // matrix of a load is uniform unless a load straddles the gate / up halves (MATS = 2, K = 3 or 5): then the
    // lanes keep 64-bit addresses.
    constexpr bool TUNI = MATS == 1 || K == 2 || K == 4;
    const uint32_t* tsrc[TL];
    uint64_t tbase[TL];
    uint32_t toff[TL];
    int tdst[TL];
#pragma unroll
    for (int j = 0; j < TL; ++j) {
        const int li = wv + 4 * j < K ? wv + 4 * j : K - 1;
        const int c = li * 64 + lane, blk = c / (2 * K), ch = c % (2 * K);
        const int tile = blk >> 1, kt = blk & 1;
        const int tmat = MATS == 2 ? tile >> 3 : 0;
        const int ntile = col0 / 16 + (MATS == 2 ? (tile & 7) : tile);
        const uint32_t* tm = tmat ? a.t1 : a.t0;
        if constexpr (TUNI) {
            tbase[j] = uniform64((uint64_t)(uintptr_t)tm + (uint64_t)s0 * 2 * NT * (8 * K) * 4);
            toff[j] = (uint32_t)((((e * KT + kt) * NT + ntile) * (8 * K) + ch * 4) * 4);
        } else {
            tsrc[j] = tm + (((size_t)e * KT + 2 * s0 + kt) * NT + ntile) * (8 * K) + ch * 4;
        }
        tdst[j] = MATS * XBUF + li * 1024;
    }
    auto issue = [&](int s) {
        const uint32_t st = lds_u + (uint32_t)((s % NS) * STAGE);
#pragma unroll
        for (int j = 0; j < XLOADS; ++j)
            load_lds16_s(xbase[j] + (uint64_t)s * 64, xoff[j], st + min(wv * XLOADS + j, MATS * RB - 1) * 1024);
#pragma unroll
        for (int j = 0; j < TL; ++j) {
            if constexpr (TUNI)
                load_lds16_s(tbase[j] + (uint64_t)s * 2 * NT * (8 * K) * 4, toff[j], st + tdst[j]);
            else
                load_lds16(tsrc[j] + (size_t)s * 2 * NT * (8 * K), lds + (s % NS) * STAGE + tdst[j]);
        }
    };
    // wait until at most n stages' loads of this wave are outstanding
    static_assert(NS - 2 <= 6 && 6 * LOADS < 64, "vmcnt range");
    auto wait_stages = [&](int n) {
        if (n >= 6) wait_vmcnt<6 * LOADS>();
        else if (n == 5) wait_vmcnt<5 * LOADS>();
        else if (n == 4) wait_vmcnt<4 * LOADS>();
        else if (n == 3) wait_vmcnt<3 * LOADS>();
        else if (n == 2) wait_vmcnt<2 * LOADS>();
        else if (n == 1) wait_vmcnt<LOADS>();
        else wait_vmcnt<0>();
    };
    const int q = lane >> 4;
    // B fragment b from LDS stage buffer `slot`; the 4 decoded A fragments of the step in `slot` (the slot is a
    // compile-time constant in the unrolled main loop, so the stage offset folds into the LDS instructions)
    auto read_b = [&](int slot, int b) {
        const unsigned char* xb = lds + slot * STAGE + mat * XBUF;
        const int row = 16 * b + (lane & 15);
        return *reinterpret_cast<const h8_t*>(xb + row * 64 + ((q ^ ((row >> 1) & 3)) << 4));
    };
    // K = 3, 5: the direct fragment decode's two per-lane funnel shifts (the same for every tile and step)
    uint32_t ksh[2] = {0u, 0u};
    if constexpr (K != 4) fragk_shifts<K>(lane, ksh);
    auto decode_a = [&](int slot, h8_t (&af)[4]) {
        const uint32_t* tw = reinterpret_cast<const uint32_t*>(lds + slot * STAGE + MATS * XBUF);
        if constexpr (K == 4) {
#pragma unroll
            for (int t4 = 0; t4 < 4; ++t4) af[t4] = a_fragment4(tw + (stile0 + t4) * 64, lane);
        } else {
#pragma unroll
            for (int t4 = 0; t4 < 4; ++t4) af[t4] = a_fragmentk<K>(tw + (stile0 + t4) * (16 * K), lane, ksh);
        }
    };

    f4_t acc[4][RB];
#pragma unroll
    for (int t4 = 0; t4 < 4; ++t4)
#pragma unroll
        for (int b = 0; b < RB; ++b) acc[t4][b] = (f4_t){0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int s = 0; s < NS - 1; ++s)
        if (s < S) issue(s);
    wait_stages(min(S, NS - 1) - 1);                      // stage 0 landed
    lds_barrier();
    constexpr int D = RB % 4 == 0 ? 4 : (RB % 2 == 0 ? 2 : 1);   // B fragments read ahead (a ring; RB % D == 0
    static_assert(RB % D == 0, "ring");                   // so that step s + 1's first fragments land in ring[0 ..])
    h8_t ring[D], a0[4], a1[4];
#pragma unroll
    for (int b = 0; b < D; ++b) ring[b] = read_b(0, b);
    decode_a(0, a0);
    // one step: multiply (ac, B fragments of the ring) while an is decoded for step s + 1 and the ring is refilled
    // D fragments ahead (the last D of them from step s + 1's stage)
    // FAST (a trip of steps known to be in the steady state, s + NS - 1 < S for each): the stage wait is the steady
    // one and every step issues
    auto step = [&](int s, int slot, const h8_t (&ac)[4], h8_t (&an)[4], auto fast) {
        constexpr bool FAST = decltype(fast)::value;
        // stage s + 1 landed (at most the stages after it in flight) and every wave is done with stage s - 1
        if constexpr (FAST) wait_vmcnt<(NS - 3) * LOADS>();
        else wait_stages(min(S - 1, s + NS - 2) - (s + 1));
        lds_barrier();
        if (FAST || s + NS - 1 < S) issue(s + NS - 1);   // into stage s - 1's buffer, now free
        const int sn = (slot + 1) % NS;                   // the next step's slot (the last step reads a stale one,
                                                          // unused)
        {
            // the next step's decode spread over this step's MFMA groups (sched_barrier keeps each group together,
            // so the VALU of the decode issues while the matrix core works)
            const uint32_t* twn = reinterpret_cast<const uint32_t*>(lds + sn * STAGE + MATS * XBUF);
            uint32_t wp[4], w0[4], w1[4], st[4];
            uint32_t wk[2][K == 4 ? 1 : 4];                // K = 3, 5: words of two tiles, one read ahead
            // the row-block count as an SGPR value opaque to the compiler at every step: each block's test is then
            // one s_cmp / s_cbranch_scc; left visible, the tests are hoisted out of the loop as lane masks and each
            // is rebuilt in the loop with a v_cndmask and a v_cmp (22 VALU instructions a step at 11 blocks)
            int nbs = nblk;
            __asm__ volatile("" : "+s"(nbs));
            if constexpr (K == 4) {
#pragma unroll
                for (int t4 = 0; t4 < 4; ++t4) frag4_words(twn + (stile0 + t4) * 64, lane, wp[t4], w0[t4], w1[t4]);
            } else {
                fragk_words<K>(twn + stile0 * (16 * K), lane, wk[0]);
            }
#pragma unroll
            for (int b = 0; b < RB; ++b) {
                const h8_t bc = ring[b % D];
                ring[b % D] = b + D < RB ? read_b(slot, b + D) : read_b(sn, b + D - RB);
                if (b < nbs) {
#pragma unroll
                    for (int t4 = 0; t4 < 4; ++t4)
                        acc[t4][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ac[t4], bc, acc[t4][b], 0, 0, 0);
                }
#pragma unroll
                for (int pr = b * 16 / RB; pr < (b + 1) * 16 / RB; ++pr) {   // the 16 decoded pairs spread evenly
                    const int t = pr >> 2, j = pr & 3;
                    if (j == 0) {
                        if constexpr (K == 4) {
                            frag4_states(wp[t], w0[t], w1[t], lane, st);
                        } else {
                            fragk_states<K>(wk[t & 1], ksh, st);
                            if (t < 3) fragk_words<K>(twn + (stile0 + t + 1) * (16 * K), lane, wk[(t + 1) & 1]);
                        }
                    }
                    const h2_t v = decode_pair(st[j]);
                    an[t][2 * j] = v[0];
                    an[t][2 * j + 1] = v[1];
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // keep the decode inside this step (the compiler would otherwise sink it next to its use)
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) __asm__ volatile("" : "+v"(an[t4]));
    };
    // UNR steps a trip (a multiple of NS and of 2): every stage slot is a constant, and the two fragment sets trade
    // roles instead of being copied
    constexpr int UNR = NS % 2 == 0 ? NS : 2 * NS;
    int s = 0;
    const std::integral_constant<bool, true> fast;
    const std::integral_constant<bool, false> general;
    for (; s + UNR + NS - 2 < S; s += UNR) {
#pragma unroll
        for (int u = 0; u < UNR; u += 2) {
            step(s + u, u % NS, a0, a1, fast);
            step(s + u + 1, (u + 1) % NS, a1, a0, fast);
        }
    }
    for (; s + UNR <= S; s += UNR) {
#pragma unroll
        for (int u = 0; u < UNR; u += 2) {
            step(s + u, u % NS, a0, a1, general);
            step(s + u + 1, (u + 1) % NS, a1, a0, general);
        }
    }
    for (; s < S; ++s) {
        step(s, s % NS, a0, a1, general);
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) a0[t4] = a1[t4];
    }
    if constexpr (SPLIT) {
        // raw partial sums, no epilogue: lane (row 16 b + lane % 16) holds columns 16 t4 + 4 (lane / 16) + 0..3 of
        // the wave's tiles
        const int cbase = col0 + wtile0 * 16 + 4 * (lane >> 4);
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            const int row = 16 * b + (lane & 15);
            if (row < nrows) {
                float* zr = a.z + ((size_t)(mat * nsk + split) * a.P + rows_sh[row]) * a.N + cbase;
#pragma unroll
                for (int t4 = 0; t4 < 4; ++t4) *reinterpret_cast<f4_t*>(zr + t4 * 16) = acc[t4][b];
            }
        }
        return;
    }
    __syncthreads();

    // ---- epilogue: ER rows at a time through LDS; each wave takes ER / 4 rows, four at a time (lane layout of
    // fwht128_l8). The column scales are the same for every row: loaded once.
    float* ep = reinterpret_cast<float*>(lds);
    const int j8 = l8_j(lane), r4 = l8_row(lane);
    float sc[3][8];   // MATS = 2: svh gate, svh up, suh down of columns 8 j8 ..; MATS = 1: svh of both halves
    {
        const size_t o = (size_t)e * a.N + col0 + 8 * j8;
        const uint16_t* src[3] = {a.sv0 + o, MATS == 2 ? a.sv1 + o : a.sv0 + o + 128, MATS == 2 ? a.sd + o : nullptr};
#pragma unroll
        for (int m = 0; m < (MATS == 2 ? 3 : 2); ++m) {
            const uint4 v = *reinterpret_cast<const uint4*>(src[m]);
            const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sc[m][2 * i] = f16_to_f32((uint16_t)vv[i]);
                sc[m][2 * i + 1] = f16_to_f32((uint16_t)(vv[i] >> 16));
            }
        }
        // the transformed accumulators carry lane_sign: fold it into the scales that multiply them (exact), and the
        // transform's 1/sqrt(128) as well (one multiply a value instead of two: v * (HAD svh) rounds where the
        // reference's (v * HAD) * svh may differ in the last fp32 bit, ahead of a bf16 or fp32 result)
        const float sg = lane_sign(lane) * HAD_SCALE;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            sc[0][i] *= sg;
            sc[1][i] *= sg;
        }
    }
    const float had_sg = lane_sign(lane) * HAD_SCALE;
    const int ncol = (MATS == 2 ? mat * 128 : 0) + wtile0 * 16 + 4 * (lane >> 4);
    auto ld8 = [&](int row, int col, float (&v)[8]) {
        const float4 x = *reinterpret_cast<const float4*>(ep + row * EPITCH + col);
        const float4 y = *reinterpret_cast<const float4*>(ep + row * EPITCH + col + 4);
        v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w; v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
    };
    // one chunk of ER rows; c is a compile-time constant so that acc stays in registers
    auto chunk = [&](auto cc) {
        constexpr int c = decltype(cc)::value;
        if constexpr (c * ER >= BM) return;
        if (c * ER >= nrows) return;
#pragma unroll
        for (int bb = 0; bb < ER / 16; ++bb)
            if (c * (ER / 16) + bb < RB)                // the last chunk of a BM that is not a multiple of ER
#pragma unroll
                for (int t4 = 0; t4 < 4; ++t4) {
                    const int row = 16 * bb + (lane & 15);
                    *reinterpret_cast<f4_t*>(ep + row * EPITCH + ncol + t4 * 16) =
                        acc[t4][min(c * (ER / 16) + bb, RB - 1)];
                }
        __syncthreads();
#pragma unroll
        for (int g = 0; g < ER / 16; ++g) {
            const int rr = wave * (ER / 4) + 4 * g + r4;        // this lane's row of the chunk
            if (c * ER + wave * (ER / 4) + 4 * g >= nrows) break;
            const int row = c * ER + rr;
            if constexpr (MATS == 2) {
                float gv[8], uv[8];
                ld8(rr, 8 * j8, gv);
                ld8(rr, 128 + 8 * j8, uv);
                fwht128_l8(gv, lane);
                fwht128_l8(uv, lane);
#pragma unroll
                for (int i = 0; i < 8; i += 2) {
                    // bf16 roundings two values at a time (g with u, then element i with i + 1)
                    float g0 = gv[i] * sc[0][i], u0 = uv[i] * sc[1][i];
                    float g1 = gv[i + 1] * sc[0][i + 1], u1 = uv[i + 1] * sc[1][i + 1];
                    bf16r2(g0, u0);
                    bf16r2(g1, u1);
                    // min(g, limit) for the finite g here, as a med3 against a huge negative bound (fminf, or a med3
                    // against -inf that the compiler turns back into it, adds a NaN-quieting v_max of each input)
                    const float gg0 = __builtin_amdgcn_fmed3f(g0, -3.0e38f, a.limit);
                    const float gg1 = __builtin_amdgcn_fmed3f(g1, -3.0e38f, a.limit);
                    const float uu0 = __builtin_amdgcn_fmed3f(u0, -a.limit, a.limit);
                    const float uu1 = __builtin_amdgcn_fmed3f(u1, -a.limit, a.limit);
                    // silu through the hardware exp2 / reciprocal (within an ulp or two of expf and the IEEE divide;
                    // the bf16 rounding that follows absorbs the difference)
                    const float ex0 = __builtin_amdgcn_exp2f(gg0 * -1.4426950408889634f);
                    const float ex1 = __builtin_amdgcn_exp2f(gg1 * -1.4426950408889634f);
                    float s0 = gg0 * __builtin_amdgcn_rcpf(1.f + ex0), s1 = gg1 * __builtin_amdgcn_rcpf(1.f + ex1);
                    bf16r2(s0, s1);
                    float a0 = s0 * uu0, a1 = s1 * uu1;
                    bf16r2(a0, a1);
                    gv[i] = a0 * sc[2][i];
                    gv[i + 1] = a1 * sc[2][i + 1];
                }
                fwht128_l8(gv, lane);
                if (row < nrows) store_pairs_l8(a.xd + (size_t)rows_sh[row] * a.N + col0, gv, lane, had_sg);
            } else {
                float v[2][8];
                ld8(rr, 8 * j8, v[0]);
                ld8(rr, 128 + 8 * j8, v[1]);
                fwht128_l8(v[0], lane);
                fwht128_l8(v[1], lane);
                if (row < nrows) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        float4* dst = reinterpret_cast<float4*>(a.y + (size_t)rows_sh[row] * a.N + col0 + h * 128 + 8 * j8);
                        dst[0] = make_float4(v[h][0] * sc[h][0], v[h][1] * sc[h][1], v[h][2] * sc[h][2],
                                             v[h][3] * sc[h][3]);
                        dst[1] = make_float4(v[h][4] * sc[h][4], v[h][5] * sc[h][5], v[h][6] * sc[h][6],
                                             v[h][7] * sc[h][7]);
                    }
                }
            }
        }
        __syncthreads();
    };
    static_assert(ER % 16 == 0 && (BM + ER - 1) / ER <= 6, "epilogue chunks");
    chunk(std::integral_constant<int, 0>{});
    chunk(std::integral_constant<int, 1>{});
    chunk(std::integral_constant<int, 2>{});
    chunk(std::integral_constant<int, 3>{});
    chunk(std::integral_constant<int, 4>{});
    chunk(std::integral_constant<int, 5>{});
}

}  // namespace gfr

struct gfr_fast_experts {
    gfr::PrefillDims d;
    uint16_t *xg, *xu, *xd;
    float* out;
    int *ucnt, *items, *plan;
    float *zgu, *zd;          // split-K partials of windows of at most PF_SPLIT_PAIRS pairs (else null)
};

namespace gfr {

// Windows of at most PF_SPLIT_PAIRS pairs (verify windows, short chunks) run split-K: 32-row items, each K range
// of PF_SPLIT_K a program, partial sums added in order by the decode path's epilogue kernels. Their full-K items
// would leave most CUs idle behind a few long programs.
#ifndef PF_SPLIT_PAIRS_MAX
#define PF_SPLIT_PAIRS_MAX 2048
#endif
constexpr int PF_SPLIT_PAIRS = PF_SPLIT_PAIRS_MAX;
constexpr int PF_SPLIT_K = 512;
// The gate/up programs take 1024 k where the hidden size allows: measured against 512 at config 3's window (103.6–
// 105.7 vs 105.1–107.4 us), the reference geometry's 40-row window (178.7–186.0 vs 183.1–188.9 us) and a 32-row
// window of config 5's shape (386.8–403.3 vs 398.6–417.8 us), three alternating runs each on two boxes; 2048 lost.
static int split_k_gateup(int hidden) { return hidden % (2 * PF_SPLIT_K) == 0 ? 2 * PF_SPLIT_K : PF_SPLIT_K; }
constexpr int PF_SPLIT_BM = 32;
static bool split_ok(int hidden, int inter) { return hidden % PF_SPLIT_K == 0 && inter % PF_SPLIT_K == 0; }
static_assert(PF_SPLIT_BM <= PF_BM2 && PF_SPLIT_BM <= PF_BM3 && PF_SPLIT_BM <= PF_BM4 && PF_SPLIT_BM <= PF_BM5,
              "items are bounded at the smallest item size");
// The most items a window of P pairs over at most maxu distinct experts can plan, at any item size the engine uses.
static size_t item_bound(size_t P, size_t maxu) {
    const size_t b = P / PF_SPLIT_BM + maxu;
    return b < P ? b : P;
}

hipError_t prefill_create(gfr_fast_experts** out, int hidden, int inter, int slots, int exl3_slots, int experts,
                          int max_rows) {
    gfr_fast_experts* fx = new gfr_fast_experts{{hidden, inter, slots, exl3_slots, experts, max_rows},
                                                nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                                nullptr, nullptr};
    const size_t P = (size_t)max_rows * slots;
    // items = sum over experts of ceil(members / bm) <= min(P, P / bm + distinct experts), largest at the smallest
    // item size (the split-K programs' PF_SPLIT_BM rows)
    const size_t max_items = item_bound(P, PF_MAXU) + 1;
    hipError_t e;
    if ((e = hipMalloc(&fx->xg, P * hidden * 2)) != hipSuccess || (e = hipMalloc(&fx->xu, P * hidden * 2)) != hipSuccess ||
        (e = hipMalloc(&fx->xd, P * inter * 2)) != hipSuccess || (e = hipMalloc(&fx->out, P * hidden * 4)) != hipSuccess ||
        (e = hipMalloc(&fx->ucnt, PF_MAXU * 4)) != hipSuccess || (e = hipMalloc(&fx->items, max_items * 4)) != hipSuccess ||
        (e = hipMalloc(&fx->plan, 16)) != hipSuccess
    ) {
        prefill_destroy(fx);
        return e;
    }
    if (split_ok(hidden, inter)) {
        const size_t Ps = P < (size_t)PF_SPLIT_PAIRS ? P : (size_t)PF_SPLIT_PAIRS;
        if ((e = hipMalloc(&fx->zgu, 2 * (size_t)(hidden / PF_SPLIT_K) * Ps * inter * 4)) != hipSuccess ||
            (e = hipMalloc(&fx->zd, (size_t)(inter / PF_SPLIT_K) * Ps * hidden * 4)) != hipSuccess) {
            prefill_destroy(fx);
            return e;
        }
    }
    *out = fx;
    return hipSuccess;
}

PrefillDims prefill_dims(const gfr_fast_experts* fx) { return fx->d; }

template <int MATS>
static hipError_t launch_gemm_split(int bits, dim3 grid, hipStream_t s, const PrefillArgs& a) {
    switch (bits) {
        case 2: prefill_gemm_kernel<MATS, 2, PF_SPLIT_BM, true><<<grid, 256, 0, s>>>(a); break;
        case 3: prefill_gemm_kernel<MATS, 3, PF_SPLIT_BM, true><<<grid, 256, 0, s>>>(a); break;
        case 4: prefill_gemm_kernel<MATS, 4, PF_SPLIT_BM, true><<<grid, 256, 0, s>>>(a); break;
        case 5: prefill_gemm_kernel<MATS, 5, PF_SPLIT_BM, true><<<grid, 256, 0, s>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int MATS>
static hipError_t launch_gemm(int bits, dim3 grid, hipStream_t s, const PrefillArgs& a) {
    switch (bits) {
        case 2: prefill_gemm_kernel<MATS, 2, PF_BM2><<<grid, 256, 0, s>>>(a); break;
        case 3: prefill_gemm_kernel<MATS, 3, PF_BM3><<<grid, 256, 0, s>>>(a); break;
        case 4: prefill_gemm_kernel<MATS, 4, PF_BM4><<<grid, 256, 0, s>>>(a); break;
        case 5: prefill_gemm_kernel<MATS, 5, PF_BM5><<<grid, 256, 0, s>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t prefill_run(gfr_fast_experts* fx, hipStream_t s, const gfr_exl3_experts* w, const uint16_t* input,
                       int input_stride, const int* picks, const int* ids, const int* count, const int* members,
                       int rows, int maxm, bool shared_x, const float* combine_weights, float* combine_out,
                       bool* combined, bool planned, const float* combine_shared, int shared_stride,
                       hipEvent_t shared_ready, bool rotated) {
    const PrefillDims& d = fx->d;
    if (combined) *combined = false;
    if (w->bits < 2 || w->bits > 5) return hipErrorInvalidValue;
    const int P = rows * d.slots;
    const int maxu = P < w->experts ? P : w->experts;
    if (maxu > PF_MAXU) return hipErrorInvalidValue;
    // the GEMM's direct loads address rows and trellis words by 32-bit byte offsets from their matrix
    const uint64_t lim = 1ull << 32;
    if ((uint64_t)P * d.hidden * 2 >= lim || (uint64_t)P * d.inter * 2 >= lim ||
        (uint64_t)w->experts * d.hidden * d.inter * w->bits / 8 >= lim)
        return hipErrorInvalidValue;
    hipError_t e;
    // rotated rows of every EXL3 pair (one copy when the two input rotations are the same)
    if (rotated) {
        if (shared_x || (d.hidden / 128) % 2) return hipErrorInvalidValue;   // not launch_route_group_rot's rows
    } else if ((d.hidden / 128) % 2 == 0) {
        const int tasks = rows * (d.hidden / 256), grid = (tasks + 3) / 4;
        if (!shared_x)
            prefill_rot2_kernel<2><<<grid, 256, 0, s>>>(input, input_stride, picks, w->suh_g, w->suh_u, fx->xg, fx->xu,
                                                        d.hidden, rows, d.slots, d.exl3_slots);
        else
            prefill_rot2_kernel<1><<<grid, 256, 0, s>>>(input, input_stride, picks, w->suh_g, w->suh_u, fx->xg, fx->xu,
                                                        d.hidden, rows, d.slots, d.exl3_slots);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    } else {
        const int tasks = rows * (d.hidden / 128);
        const int mats = shared_x ? 1 : 2;
        if (d.exl3_slots * mats <= 16)   // fewer scale registers: more resident waves
            prefill_rot_kernel<4><<<(tasks + 3) / 4, 256, 0, s>>>(input, input_stride, picks, w->suh_g, w->suh_u,
                                                                  fx->xg, fx->xu, d.hidden, rows, d.slots,
                                                                  d.exl3_slots, mats);
        else if (d.exl3_slots * mats <= 32)
            prefill_rot_kernel<8><<<(tasks + 3) / 4, 256, 0, s>>>(input, input_stride, picks, w->suh_g, w->suh_u,
                                                                  fx->xg, fx->xu, d.hidden, rows, d.slots,
                                                                  d.exl3_slots, mats);
        else
            prefill_rot_kernel<16><<<(tasks + 3) / 4, 256, 0, s>>>(input, input_stride, picks, w->suh_g, w->suh_u,
                                                                   fx->xg, fx->xu, d.hidden, rows, d.slots,
                                                                   d.exl3_slots, mats);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    const bool split = fx->zgu && P <= PF_SPLIT_PAIRS;
    const int bm = split ? PF_SPLIT_BM : pf_bm_for(w->bits);
    if (!planned) {
        prefill_plan_kernel<<<1, 1024, 0, s>>>(ids, count, members, maxm, w->experts, maxu, bm, fx->ucnt, fx->items,
                                               fx->plan);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    // grid bound on the plan's items (sum of ceil(members / bm) <= min(P, P / bm + maxu)); the allocation holds
    // item_bound(max P, PF_MAXU), which is at least this
    const int max_items = P / bm + maxu < P ? P / bm + maxu : P;
    PrefillArgs a{};
    a.uids = ids; a.members = members; a.ucnt = fx->ucnt; a.items = fx->items; a.plan = fx->plan;
    a.maxm = maxm; a.slots = d.slots; a.limit = 10.f;
    if (split) {
        // gate / up partials -> epilogue (xd in pair order) -> down partials -> epilogue -> output
        const int skg = d.hidden / split_k_gateup(d.hidden), skd = d.inter / PF_SPLIT_K;
        a.sk = skg; a.P = P; a.z = fx->zgu;
        a.x0 = fx->xg; a.x1 = shared_x ? fx->xg : fx->xu; a.t0 = w->gt; a.t1 = w->ut; a.Kin = d.hidden; a.N = d.inter;
        if ((e = launch_gemm_split<2>(w->bits, dim3(max_items * (d.inter / 128) * skg), s, a)) != hipSuccess) return e;
        if ((e = launch_gateup_epilogue(s, fx->zgu, picks, w->svh_g, w->svh_u, w->suh_d, fx->xd, P, d.inter, skg,
                                        d.slots, d.exl3_slots, 10.f, true)) != hipSuccess)
            return e;
        a.sk = skd; a.z = fx->zd;
        a.x0 = fx->xd; a.x1 = fx->xd; a.t0 = w->dt; a.t1 = w->dt; a.Kin = d.inter; a.N = d.hidden;
        if ((e = launch_gemm_split<1>(w->bits, dim3(max_items * (d.hidden / 256) * skd), s, a)) != hipSuccess) return e;
        if (combine_weights && combine_out && d.exl3_slots <= 16) {
            // the down epilogue and the layer's slot-ordered combine in one launch (the decode path's finish)
            if (combined) *combined = true;
            if (shared_ready && (e = hipStreamWaitEvent(s, shared_ready, 0)) != hipSuccess) return e;
            return launch_down_finish(s, fx->zd, picks, w->svh_d, fx->out, rows, P, d.hidden, skd, d.slots,
                                      d.exl3_slots, combine_weights, combine_shared, shared_stride, combine_out);
        }
        return launch_down_epilogue(s, fx->zd, picks, w->svh_d, fx->out, P, d.hidden, skd, d.slots, d.exl3_slots);
    }
    // gate / up -> xd
    a.x0 = fx->xg; a.x1 = shared_x ? fx->xg : fx->xu; a.t0 = w->gt; a.t1 = w->ut; a.Kin = d.hidden; a.N = d.inter;
    a.sv0 = w->svh_g; a.sv1 = w->svh_u; a.sd = w->suh_d; a.xd = fx->xd; a.y = fx->out;
    if ((e = launch_gemm<2>(w->bits, dim3(max_items * (d.inter / 128)), s, a)) != hipSuccess) return e;
    // down -> output
    a.x0 = fx->xd; a.x1 = fx->xd; a.t0 = w->dt; a.t1 = w->dt; a.Kin = d.inter; a.N = d.hidden;
    a.sv0 = w->svh_d; a.sv1 = nullptr; a.sd = nullptr; a.xd = nullptr; a.y = fx->out;
    return launch_gemm<1>(w->bits, dim3(max_items * (d.hidden / 256)), s, a);
}

float* prefill_output(const gfr_fast_experts* fx) { return fx->out; }
int prefill_item_rows(const gfr_fast_experts* fx, int rows, int bits) {
    const bool split = fx->zgu && rows * fx->d.slots <= PF_SPLIT_PAIRS;
    return split ? PF_SPLIT_BM : pf_bm_for(bits);
}
hipError_t launch_route_group_rot(gfr_fast_experts* fx, hipStream_t s, const gfr_exl3_experts* w,
                                  const uint16_t* input, int input_stride, const float* logits, int rows, int routed,
                                  int topk, int* picks, float* weights, int* ids, int* count, int* members, int maxm,
                                  const float* bias, float scale) {
    const PrefillDims& d = fx->d;
    const int slots = topk + 1;
    const size_t lds = route_group_lds(rows, slots, routed + 1);
    if (rows < 1 || rows > GROUP_SMALL_ROWS || rows > d.max_rows || routed + 1 > 1024 || slots != d.slots ||
        lds > GROUP_LDS_MAX || (d.hidden / 128) % 2 || w->bits < 2 || w->bits > 5)
        return hipErrorNotSupported;
    constexpr int WG = 512;                              // route_group measured the same at 512 and 1024 threads
    const int tasks = rows * (d.hidden / 256), grid = 1 + (tasks + WG / 64 - 1) / (WG / 64);
    route_group_rot_kernel<2><<<grid, WG, lds, s>>>(logits, rows, routed, topk, picks, weights, ids, count, members,
                                                    maxm, prefill_item_rows(fx, rows, w->bits), fx->ucnt, fx->items,
                                                    fx->plan, w->experts, RouteGate{bias, scale}, input, input_stride,
                                                    w->suh_g, w->suh_u, fx->xg, fx->xu, d.hidden, d.exl3_slots);
    return hipGetLastError();
}

hipError_t launch_group_large_rot(gfr_fast_experts* fx, hipStream_t s, const gfr_exl3_experts* w,
                                  const uint16_t* input, int input_stride, const int* picks, int rows, int slots,
                                  int E, uint32_t* bits, uint8_t* first, int* prefix, int* counts, int* ids,
                                  int* count, int* members, int maxm) {
    const PrefillDims& d = fx->d;
    if (rows < 1 || rows > d.max_rows || slots != d.slots || (d.hidden / 128) % 2 || w->bits < 2 || w->bits > 5)
        return hipErrorNotSupported;
    const int bm = prefill_item_rows(fx, rows, w->bits);
    hipError_t e = launch_group_large(s, picks, rows, slots, E, bits, first, prefix, counts, ids, count, members,
                                      maxm, bm, fx->ucnt, fx->items, fx->plan, w->experts, false);
    if (e != hipSuccess) return e;
    const int tasks = rows * (d.hidden / 256);
    group_scatter_rot_kernel<2><<<E + (tasks + 3) / 4, 256, 0, s>>>(picks, rows, slots, E, bits, first, prefix,
                                                                    counts, ids, count, members, maxm, bm, fx->ucnt,
                                                                    fx->items, fx->plan, w->experts, input,
                                                                    input_stride, w->suh_g, w->suh_u, fx->xg, fx->xu,
                                                                    d.hidden, d.exl3_slots);
    return hipGetLastError();
}

void prefill_plan_buffers(gfr_fast_experts* fx, int** ucnt, int** items, int** plan) {
    *ucnt = fx->ucnt;
    *items = fx->items;
    *plan = fx->plan;
}
uint16_t* prefill_xd(const gfr_fast_experts* fx) { return fx->xd; }
uint16_t* prefill_rotated(const gfr_fast_experts* fx, int mat) { return mat ? fx->xu : fx->xg; }

void prefill_destroy(gfr_fast_experts* fx) {
    if (!fx) return;
    for (void* p : {(void*)fx->xg, (void*)fx->xu, (void*)fx->xd, (void*)fx->out, (void*)fx->ucnt, (void*)fx->items,
                    (void*)fx->plan, (void*)fx->zgu, (void*)fx->zd})
        if (p) (void)hipFree(p);
    delete fx;
}

}  // namespace gfr
