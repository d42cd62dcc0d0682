// EXL3 routed experts for decode and verify windows on gfx950: input rotation, grouped trellis GEMV, epilogues.
//
// Same contract as glm-flash-rs native/exl3.cu (rot_in_kernel :224-241, exl3_grouped_8_4 :145-170 / :325-330,
// gateup_epilogue_kernel :260-296, down_epilogue_kernel :300-321), designed for CDNA4:
//   * the GEMV streams each k tile of a 128-column block as one contiguous 8 * (32 K)-byte run per wave (lane l
//     loads K consecutive words with one vector load), decodes the trellis in VALU (exl3_format.hpp) and
//     accumulates with v_dot2_f32_f16 (fp16 x fp16 products, fp32 accumulate);
//   * a workgroup covers one (expert, matrix, 128-column block, K split); its waves own fixed contiguous k ranges
//     that are added in wave order through LDS; splits go to Z[mat][split][pair][n] and are added in split order
//     by the epilogue, so every output is deterministic and depends only on its own row;
//   * weights are decoded once per workgroup and reused for all member rows of the expert (up to RB at a time).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "exl3_format.hpp"
#include "route.hpp"
#include "launch.hpp"

namespace gfr {

template <int K>
__device__ __forceinline__ void load_words(const uint32_t* __restrict__ p, uint32_t (&w)[K]) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    if constexpr (K == 4) {
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else if constexpr (K == 2) {
        const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
        w[0] = v.x; w[1] = v.y;
    } else {
#pragma unroll
        for (int j = 0; j < K; ++j) w[j] = __builtin_nontemporal_load(p + j);
    }
}

// Debug / parity: the decoded fp16 weights of a whole matrix, row-major [kin][n] (gfr_exl3_decode_tiles).
// One wave decodes 8 tiles of one k tile row.
template <int K>
__global__ void __launch_bounds__(64) decode_tiles_kernel(const uint32_t* __restrict__ T, int kin, int n,
                                                           uint16_t* __restrict__ out) {
    const int lane = threadIdx.x, t = lane >> 3, i = lane & 7;
    const int NT = n >> 4, kt = blockIdx.y, nt = blockIdx.x * 8 + t;
    const bool ok = nt < NT;
    uint32_t w[K];
    const uint32_t* src = T + ((size_t)kt * NT + (ok ? nt : 0)) * (8 * K) + i * K;
#pragma unroll
    for (int j = 0; j < K; ++j) w[j] = src[j];
    const uint32_t prev = prev_word(w[K - 1], i);
    h2_t d[2][8];
    decode_lane<K>(w, prev, d);
    if (!ok) return;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const int col = nt * 16 + i + 8 * c;
            const uint32_t v = h2_bits(d[c][m]);
            out[(size_t)(kt * 16 + pair_row(K, m, 0)) * n + col] = (uint16_t)v;
            out[(size_t)(kt * 16 + pair_row(K, m, 1)) * n + col] = (uint16_t)(v >> 16);
        }
}

// rot_in (exl3.cu:224-241): Xh[mat][p][blk] = fp16(had(bf16 x[row] * suh[mat][e]) * HAD) for every pair
// p = row * slots + slot with slot < exl3_slots. One wave a (pair, 128-block, matrix). F16IN: x is fp16 (the
// single-linear config) instead of bf16.
template <bool F16IN>
__global__ void __launch_bounds__(64) rot_in_kernel(const uint16_t* __restrict__ x, int x_stride,
                                                     const int* __restrict__ pick, const uint16_t* __restrict__ suh0,
                                                     const uint16_t* __restrict__ suh1, uint16_t* __restrict__ out0,
                                                     uint16_t* __restrict__ out1, int K, int slots, int exl3_slots) {
    const int p = blockIdx.x, blk = blockIdx.y, mat = blockIdx.z;
    const int row = p / slots, slot = p % slots;
    if (slot >= exl3_slots) return;
    const int lane = threadIdx.x;
    const int e = pick[row * slots + slot];
    const int k = blk * 128 + 2 * lane;
    const uint16_t* suh = (mat ? suh1 : suh0) + (size_t)e * K + k;
    const uint16_t* xr = x + (size_t)row * x_stride + k;
    float v[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) v[j] = (F16IN ? f16_to_f32(xr[j]) : bf16_to_f32(xr[j])) * f16_to_f32(suh[j]);
    fwht128_w64(v, lane);
    uint16_t* o = (mat ? out1 : out0) + (size_t)p * K + k;
    const uint32_t packed = (uint32_t)f16_of_product(v[0], HAD_SCALE) | ((uint32_t)f16_of_product(v[1], HAD_SCALE) << 16);
    *reinterpret_cast<uint32_t*>(o) = packed;
}


// Arguments of the decode GEMV (one struct in the kernarg segment).
struct GemvArgs {
    const uint16_t* x0;      // XSRC 0: fp16 rotated rows [P][Kin] (matrix 0); XSRC 1: bf16 input rows [rows][x_stride]
    const uint16_t* x1;      // XSRC 0: fp16 rotated rows of matrix 1
    int x_stride;
    const uint16_t* suh0;    // XSRC 1: input scales [E][Kin] of the two matrices; XSRC 2: suh_d [E][Kin]
    const uint16_t* suh1;
    const uint32_t* t0;      // trellis [E][Kin/16][N/16][8K]
    const uint32_t* t1;
    const int* uids;
    const int* ucount;
    const int* members;      // [E][maxm]
    float* z;                // [MATS][SK][P][N] split partials (output)
    int Kin, N, P, SK, maxm, slots, E;
    const float* zgu;        // XSRC 2: the gate/up split partials [2][SKgu][P][Kin]
    int SKgu;
    const uint16_t* svh_g;   // XSRC 2: gate / up output scales [E][Kin]
    const uint16_t* svh_u;
    float limit;
    uint16_t* xd;            // XSRC 2: the down input, also stored (column block 0 only) [P][Kin] fp16
    const float* logits;     // ROUTE1: the token's router logits [routed]
    const float* route_bias; // ROUTE1: the gate (route.hpp RouteGate): nullptr = softmax
    float route_scale;
    int routed;
    int* pick_out;           // ROUTE1 outputs (program 0): picks / weights [slots], ids [slots], count, members
    float* weight_out;
    int* ids_out;
    int* count_out;
    int* members_out;
    int x_f16;               // XSRC 1: the input rows are fp16 (the single linear) instead of bf16
    int ucap;                // programs x = chunk * ucap + u: distinct-expert slots of the grid (RB members a chunk)
};

// The 128 activations of one Hadamard block for one member, already in fp32 lanes v[0..1] = elements 2 lane + j,
// rounded to fp16 and staged twice in a word, (x, x), into the wave's LDS slots (tile row order) of k tiles kk0 ..
// kk0 + 7: the operand tile_dot takes.
__device__ __forceinline__ void store_block(uint32_t* slots, const float (&v)[2], int lane) {
    const uint32_t h0 = f16_of_product(v[0], HAD_SCALE), h1 = f16_of_product(v[1], HAD_SCALE);
    *reinterpret_cast<uint2*>(slots + 2 * lane) = make_uint2(h0 | h0 << 16, h1 | h1 << 16);
}
// One k tile's 16 staged activations (rows 0..15, each twice) into registers.
__device__ __forceinline__ void load_tile_acts(const uint32_t* tile, uint32_t (&xd)[16]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint4 v = reinterpret_cast<const uint4*>(tile)[q];
        xd[4 * q] = v.x;
        xd[4 * q + 1] = v.y;
        xd[4 * q + 2] = v.z;
        xd[4 * q + 3] = v.w;
    }
}

// Grouped trellis GEMV of the decode path. Program (chunk * ucap + distinct expert u, 128-column block cb, mat * SK +
// split): members [chunk RB, chunk RB + RB) of expert uids[u] times W_q[mat] over k tiles [split * NW KTW,
// (split + 1) * NW KTW) for the block's 128 columns; wave w owns k tiles split * NW KTW + w KTW + [0, KTW),
// ascending, one v_dot2_f32_f16 chain a column (codeword halves against the activation, exl3_format.hpp lane_words /
// tile_dot); the waves are added in order through LDS into Z[mat][split][pair][n] (every sum has a fixed order, so a
// row's result never depends on the other rows or on RB).
//   Prologue: the window's count, the expert id and the member codes in one round trip (ROUTE1: computed here
//   instead), then the activation loads, then the trellis words, so that the activations are built while the
//   trellis streams in. Activation sources (each bit for bit the reference's formula), staged per wave in LDS:
//   XSRC 0  rotated fp16 rows (exl3.cu's grouped kernel input);
//   XSRC 1  rot_in fused (exl3.cu:224-241): bf16 input row * suh -> 128-point transform -> fp16; KTW = 8, one block;
//   XSRC 2  the gate/up epilogue fused (exl3.cu:260-296): the gate / up split partials of one 128-block summed in
//           order -> transforms, scales, limited SwiGLU, suh_d, transform -> fp16 (the down projection's input).
//   ROUTE1  (one-token windows) the wave routes the token itself (route.hpp) from a.logits: the window's experts
//           are the token's slots; program (0, 0, 0) stores picks / weights / ids / count / members for the later
//           launches.
template <int K, int KTW, int NW, int MATS, int XSRC, int RB, bool ROUTE1>
__global__ void __launch_bounds__(NW * 64) expert_gemv_kernel(const GemvArgs a) {
    constexpr int KC = NW * KTW;
    static_assert(XSRC == 0 || KTW == 8, "a wave that builds its activations covers one 128-point block");
    static_assert(XSRC != 0 || RB * KTW <= 64, "one lane a (member, k tile) when staging rotated rows");
    __shared__ __attribute__((aligned(16))) uint32_t xs[NW][RB][KTW * 16];   // activations, each twice
    __shared__ float red[NW][RB][128];

    const int u = blockIdx.x % a.ucap, cb = blockIdx.y, c0 = (int)(blockIdx.x / a.ucap) * RB;
    const int split = blockIdx.z % a.SK, mat = MATS == 1 ? 0 : blockIdx.z / a.SK;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, t = lane >> 3, i = lane & 7;
    const int KT = a.Kin >> 4, NT = a.N >> 4;
    const int kt0 = split * KC + wave * KTW;

    int e, code;
    if constexpr (ROUTE1) {
        int pick;
        float weight;
        route_token_regs(a.logits, a.routed, a.slots - 1, a.routed, pick, weight, RouteGate{a.route_bias, a.route_scale});
        int rank = 0;                                    // ascending order of the token's slots' experts
        for (int j = 0; j < a.slots; ++j) rank += __builtin_amdgcn_readlane(pick, j) < pick;
        const uint64_t mine = __ballot(lane < a.slots && rank == u);
        if (mine == 0) return;                           // u >= slots: no such expert
        const int slot = __builtin_ctzll(mine);
        e = __builtin_amdgcn_readlane(pick, slot);
        code = lane == 0 ? slot : -1;                    // row 0, this slot
        if (u == 0 && cb == 0 && blockIdx.z == 0 && wave == 0 && lane < a.slots) {
            a.pick_out[lane] = pick;
            a.weight_out[lane] = weight;
            a.ids_out[rank] = pick;
            a.members_out[(size_t)rank * a.maxm] = lane;
            for (int j = 1; j < a.maxm; ++j) a.members_out[(size_t)rank * a.maxm + j] = -1;
            if (lane == 0) a.count_out[0] = a.slots;
        }
        if (e >= a.E) return;
    } else {
        const int cntu = a.ucount[0];
        e = a.uids[u];
        code = lane < a.maxm ? a.members[(size_t)u * a.maxm + lane] : -1;
        // past the window's experts, not an EXL3 expert, or this program's chunk is past the expert's members (the
        // check sits here: a later exit, after the ballot, cost the RB > 1 forms most of their registers)
        if (u >= cntu || e >= a.E || (c0 > 0 && __builtin_amdgcn_readlane(code, c0 & 63) < 0)) return;
    }
    const int cnt = __popcll(__ballot(code >= 0));        // members come first
    const int pair_l = code >= 0 ? (code >> 5) * a.slots + (code & 31) : 0;

    // ---- activation loads of this program's chunk of members (before the trellis words)
    uint32_t xv[RB], sv = 0, sg = 0, su = 0;             // XSRC 1: bf16 pairs; scale pairs
    uint4 va = {0, 0, 0, 0}, vb = {0, 0, 0, 0};           // XSRC 0: this lane's k tile of one member
    float gsum[RB][2], usum[RB][2];
    // XSRC 2, one member at a time: the first four gate / up partials are only loaded here (so that the trellis
    // loads issue right behind them) and added in build_acts, in split order as the later ones
    constexpr int EARLY = (XSRC == 2 && RB == 1) ? 4 : 0;
    float2 zg0[RB][EARLY > 0 ? EARLY : 1], zu0[RB][EARLY > 0 ? EARLY : 1];
    auto load_acts = [&](int r0, int nr) {
        if constexpr (XSRC == 1) {
            sv = *reinterpret_cast<const uint32_t*>((mat ? a.suh1 : a.suh0) + (size_t)e * a.Kin + kt0 * 16 + 2 * lane);
#pragma unroll
            for (int m = 0; m < RB; ++m) {
                const int row = __builtin_amdgcn_readlane(code, r0 + (m < nr ? m : 0)) >> 5;
                xv[m] = *reinterpret_cast<const uint32_t*>(a.x0 + (size_t)row * a.x_stride + kt0 * 16 + 2 * lane);
            }
        } else if constexpr (XSRC == 2) {
            const size_t o = (size_t)e * a.Kin + kt0 * 16 + 2 * lane;
            sg = *reinterpret_cast<const uint32_t*>(a.svh_g + o);
            su = *reinterpret_cast<const uint32_t*>(a.svh_u + o);
            sv = *reinterpret_cast<const uint32_t*>(a.suh0 + o);
#pragma unroll
            for (int m = 0; m < RB; ++m) gsum[m][0] = gsum[m][1] = usum[m][0] = usum[m][1] = 0.f;
            const int n = kt0 * 16 + 2 * lane;
            if constexpr (EARLY > 0) {
                const int p = __builtin_amdgcn_readlane(pair_l, r0);
#pragma unroll
                for (int q = 0; q < EARLY; ++q) {
                    const int sq = q < a.SKgu ? q : 0;
                    zg0[0][q] = *reinterpret_cast<const float2*>(a.zgu + ((size_t)sq * a.P + p) * a.Kin + n);
                    zu0[0][q] = *reinterpret_cast<const float2*>(a.zgu + ((size_t)(a.SKgu + sq) * a.P + p) * a.Kin + n);
                }
                return;                                   // the rest is added in build_acts
            }
            for (int s0 = 0; s0 < a.SKgu; s0 += 4) {      // partials in split order, four in flight
                float2 zg[RB][4], zu[RB][4];
#pragma unroll
                for (int m = 0; m < RB; ++m) {
                    const int p = __builtin_amdgcn_readlane(pair_l, r0 + (m < nr ? m : 0));
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        if (s0 + q < a.SKgu) {
                            zg[m][q] = *reinterpret_cast<const float2*>(a.zgu + ((size_t)(s0 + q) * a.P + p) * a.Kin + n);
                            zu[m][q] = *reinterpret_cast<const float2*>(
                                a.zgu + ((size_t)(a.SKgu + s0 + q) * a.P + p) * a.Kin + n);
                        }
                }
#pragma unroll
                for (int m = 0; m < RB; ++m)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        if (s0 + q < a.SKgu) {
                            gsum[m][0] += zg[m][q].x; gsum[m][1] += zg[m][q].y;
                            usum[m][0] += zu[m][q].x; usum[m][1] += zu[m][q].y;
                        }
            }
        } else {
            const int m = lane / KTW, kk = lane % KTW;
            const int p = __shfl(pair_l, (r0 + m) & 63, 64);
            if (m < nr) {
                const uint16_t* X = mat ? a.x1 : a.x0;
                const uint4* src = reinterpret_cast<const uint4*>(X + (size_t)p * a.Kin + (size_t)(kt0 + kk) * 16);
                va = src[0];
                vb = src[1];
            }
        }
    };
    // ---- the loaded activations of a chunk -> this wave's LDS slots (tile row order, each value twice)
    auto build_acts = [&](int r0, int nr) {
        if constexpr (XSRC == 1) {
            const float s0 = f16_to_f32((uint16_t)sv), s1 = f16_to_f32((uint16_t)(sv >> 16));
#pragma unroll
            for (int m = 0; m < RB; ++m)
                if (m < nr) {
                    const uint16_t x0 = (uint16_t)xv[m], x1 = (uint16_t)(xv[m] >> 16);
                    float v[2] = {(a.x_f16 ? f16_to_f32(x0) : bf16_to_f32(x0)) * s0,
                                  (a.x_f16 ? f16_to_f32(x1) : bf16_to_f32(x1)) * s1};
                    fwht128_w64(v, lane);
                    store_block(&xs[wave][m][0], v, lane);
                }
        } else if constexpr (XSRC == 2) {
            if constexpr (EARLY > 0) {
                // the early partials, then the rest four at a time, all in split order
                const int n = kt0 * 16 + 2 * lane;
#pragma unroll
                for (int q = 0; q < EARLY; ++q)
                    if (q < a.SKgu) {
                        gsum[0][0] += zg0[0][q].x; gsum[0][1] += zg0[0][q].y;
                        usum[0][0] += zu0[0][q].x; usum[0][1] += zu0[0][q].y;
                    }
                const int p = __builtin_amdgcn_readlane(pair_l, r0);
                for (int s0 = EARLY; s0 < a.SKgu; s0 += 4) {
                    float2 zg[4], zu[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        if (s0 + q < a.SKgu) {
                            zg[q] = *reinterpret_cast<const float2*>(a.zgu + ((size_t)(s0 + q) * a.P + p) * a.Kin + n);
                            zu[q] = *reinterpret_cast<const float2*>(
                                a.zgu + ((size_t)(a.SKgu + s0 + q) * a.P + p) * a.Kin + n);
                        }
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        if (s0 + q < a.SKgu) {
                            gsum[0][0] += zg[q].x; gsum[0][1] += zg[q].y;
                            usum[0][0] += zu[q].x; usum[0][1] += zu[q].y;
                        }
                }
            }
            const float svg[2] = {f16_to_f32((uint16_t)sg), f16_to_f32((uint16_t)(sg >> 16))};
            const float svu[2] = {f16_to_f32((uint16_t)su), f16_to_f32((uint16_t)(su >> 16))};
            const float sdd[2] = {f16_to_f32((uint16_t)sv), f16_to_f32((uint16_t)(sv >> 16))};
            const int n = kt0 * 16 + 2 * lane;
#pragma unroll
            for (int m = 0; m < RB; ++m)
                if (m < nr) {
                    float gv[2] = {gsum[m][0], gsum[m][1]}, uv[2] = {usum[m][0], usum[m][1]};
                    fwht128_w64(gv, lane);
                    fwht128_w64(uv, lane);
                    float v[2];
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const float gg = fminf(bf16r(gv[j] * HAD_SCALE * svg[j]), a.limit);
                        const float uu = fminf(fmaxf(bf16r(uv[j] * HAD_SCALE * svu[j]), -a.limit), a.limit);
                        const float act = bf16r(bf16r(gg / (1.f + expf(-gg))) * uu);
                        v[j] = act * sdd[j];
                    }
                    fwht128_w64(v, lane);
                    store_block(&xs[wave][m][0], v, lane);
                    if (cb == 0 && a.xd) {
                        const int p = __builtin_amdgcn_readlane(pair_l, r0 + m);
                        *reinterpret_cast<uint32_t*>(a.xd + (size_t)p * a.Kin + n) =
                            (uint32_t)f16_of_product(v[0], HAD_SCALE) | ((uint32_t)f16_of_product(v[1], HAD_SCALE) << 16);
                    }
                }
        } else {
            const int m = lane / KTW, kk = lane % KTW;
            if (m < nr) {
                const uint32_t x8[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
                uint4* dst = reinterpret_cast<uint4*>(&xs[wave][m][kk * 16]);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t a0 = x8[2 * q] & 0xffffu, a1 = x8[2 * q] >> 16;
                    const uint32_t b0 = x8[2 * q + 1] & 0xffffu, b1 = x8[2 * q + 1] >> 16;
                    dst[q] = make_uint4(a0 | a0 << 16, a1 | a1 << 16, b0 | b0 << 16, b1 | b1 << 16);
                }
            }
        }
        // the slots are this wave's own: a wave-level barrier orders the LDS stores before the reads
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    const int nr0 = cnt - c0 < RB ? cnt - c0 : RB;
    load_acts(c0, nr0);
    uint32_t wr[KTW][K];
    {
        const uint32_t* T = mat ? a.t1 : a.t0;
        const uint32_t* src = T + (((size_t)e * KT + kt0) * NT + cb * 8 + t) * (8 * K) + i * K;
#pragma unroll
        for (int kk = 0; kk < KTW; ++kk) load_words<K>(src + (size_t)kk * NT * (8 * K), wr[kk]);
    }
    // keep this order: activation loads, every trellis load, then the activations built (waiting only for their
    // own loads), then tile by tile decode + products as the words land. Left alone, the scheduler sinks the
    // activation loads below the decode and splits the trellis loads into dependent rounds.
    __builtin_amdgcn_sched_barrier(0);

    // the chunk of up to RB members (its activations are already loading)
    auto chunk = [&](int r0, int nr) {
        build_acts(r0, nr);
        __builtin_amdgcn_sched_barrier(0);
        float acc[RB][2];
#pragma unroll
        for (int m = 0; m < RB; ++m) acc[m][0] = acc[m][1] = 0.f;
#pragma unroll
        for (int kk = 0; kk < KTW; ++kk) {
            // tile kk's words, as a value of this iteration: its decode waits for its own load only and is not
            // hoisted above the activation build (the words are loop-invariant otherwise; hoisted, the decoded
            // tiles held 128 registers and cut the resident waves)
#pragma unroll
            for (int j = 0; j < K; ++j) __asm__ volatile("" : "+v"(wr[kk][j]));
            const uint32_t prev = prev_word(wr[kk][K - 1], i);
            uint32_t cw[32];
            lane_words<K>(wr[kk], prev, cw);
#pragma unroll
            for (int m = 0; m < RB; ++m) {
                if (m < nr) {
                    uint32_t xd[16];
                    load_tile_acts(&xs[wave][m][kk * 16], xd);
                    tile_dot(cw, xd, acc[m]);
                }
            }
        }
        if constexpr (NW == 1) {
#pragma unroll
            for (int m = 0; m < RB; ++m)
                if (m < nr) {
                    const int p = __builtin_amdgcn_readlane(pair_l, r0 + m);
                    float* zr = a.z + ((size_t)(mat * a.SK + split) * a.P + p) * a.N + cb * 128 + 16 * t + i;
                    zr[0] = acc[m][0];
                    zr[8] = acc[m][1];
                }
        } else {
#pragma unroll
            for (int m = 0; m < RB; ++m)
                if (m < nr) {
                    red[wave][m][16 * t + i] = acc[m][0];
                    red[wave][m][16 * t + i + 8] = acc[m][1];
                }
            __syncthreads();
            for (int idx = tid; idx < nr * 128; idx += NW * 64) {
                const int m = idx >> 7, col = idx & 127;
                float sum = red[0][m][col];
#pragma unroll
                for (int w = 1; w < NW; ++w) sum += red[w][m][col];
                const int p = __builtin_amdgcn_readlane(pair_l, r0 + m);
                a.z[((size_t)(mat * a.SK + split) * a.P + p) * a.N + cb * 128 + col] = sum;
            }
        }
    };
    chunk(c0, nr0);
}

// Down epilogue (exl3.cu:300-321) and, with weights, the slot-ordered combine of a token. Program (token row,
// 128-column block), one wave a slot (up to 16 at a time): pair p = row * slots + s, its SK down partials summed in
// order, transformed, scaled by svh_d -> y[p]; then out[row] = sum over the slots in order of weights * y.
__global__ void __launch_bounds__(1024) down_finish_kernel(const float* __restrict__ Z, const int* __restrict__ pick,
                                                            const uint16_t* __restrict__ svh_d, float* __restrict__ y,
                                                            int P, int D, int SK, int slots, int exl3_slots,
                                                            const float* __restrict__ weights,
                                                            float* __restrict__ out) {
    __shared__ float2 ys[16][64];
    const int row = blockIdx.x, blk = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nwv = blockDim.x >> 6;
    const int n = blk * 128 + 2 * lane;
    float o0 = 0.f, o1 = 0.f;
    for (int s0 = 0; s0 < exl3_slots; s0 += nwv) {
        const int s = s0 + wave;
        if (s < exl3_slots) {
            const int p = row * slots + s;
            const int e = pick[p];
            float2 zs[8];
            float v[2] = {0.f, 0.f};
            for (int k0 = 0; k0 < SK; k0 += 8) {            // partials in split order, eight in flight
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    if (k0 + k < SK) zs[k] = *reinterpret_cast<const float2*>(Z + ((size_t)(k0 + k) * P + p) * D + n);
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    if (k0 + k < SK) {
                        v[0] += zs[k].x;
                        v[1] += zs[k].y;
                    }
            }
            const uint32_t sv = *reinterpret_cast<const uint32_t*>(svh_d + (size_t)e * D + n);
            fwht128_w64(v, lane);
            float2 yv;
            yv.x = v[0] * HAD_SCALE * f16_to_f32((uint16_t)sv);
            yv.y = v[1] * HAD_SCALE * f16_to_f32((uint16_t)(sv >> 16));
            *reinterpret_cast<float2*>(y + (size_t)p * D + n) = yv;
            ys[wave][lane] = yv;
        }
        if (weights) {
            __syncthreads();
            if (wave == 0)
                for (int q = 0; q < nwv && s0 + q < exl3_slots; ++q) {
                    const float w = weights[row * slots + s0 + q];
                    o0 += w * ys[q][lane].x;
                    o1 += w * ys[q][lane].y;
                }
            __syncthreads();
        }
    }
    if (weights && wave == 0) *reinterpret_cast<float2*>(out + (size_t)row * D + n) = make_float2(o0, o1);
}

// gateup epilogue (exl3.cu:260-296): ordered split sums of gate and up, rotation, svh scales, GLM's limited SwiGLU
// with its bf16 roundings, suh_d scale, rotation -> xd fp16. One wave a (pair, 128-column block).
__global__ void __launch_bounds__(64) gateup_epilogue_kernel(const float* __restrict__ Z, const int* __restrict__ pick,
                                                              const uint16_t* __restrict__ svh_g,
                                                              const uint16_t* __restrict__ svh_u,
                                                              const uint16_t* __restrict__ suh_d,
                                                              uint16_t* __restrict__ xd, int P, int N, int SK,
                                                              int slots, int exl3_slots, float limit, int pairs) {
    const int p = blockIdx.x, blk = blockIdx.y;
    const int row = p / slots, slot = p % slots;
    if (slot >= exl3_slots) return;
    const int lane = threadIdx.x;
    const int e = pick[row * slots + slot];
    const int n = blk * 128 + 2 * lane;
    float gv[2], uv[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        float sg = 0.f, su = 0.f;
        for (int s = 0; s < SK; ++s) {
            sg += Z[((size_t)(0 * SK + s) * P + p) * N + n + j];
            su += Z[((size_t)(1 * SK + s) * P + p) * N + n + j];
        }
        gv[j] = sg;
        uv[j] = su;
    }
    fwht128_w64(gv, lane);
    fwht128_w64(uv, lane);
    float v[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const float gg = fminf(bf16r(gv[j] * HAD_SCALE * f16_to_f32(svh_g[(size_t)e * N + n + j])), limit);
        const float uu =
            fminf(fmaxf(bf16r(uv[j] * HAD_SCALE * f16_to_f32(svh_u[(size_t)e * N + n + j])), -limit), limit);
        const float act = bf16r(bf16r(gg / (1.f + expf(-gg))) * uu);
        v[j] = act * f16_to_f32(suh_d[(size_t)e * N + n + j]);
    }
    fwht128_w64(v, lane);
    const uint16_t h0 = f16_of_product(v[0], HAD_SCALE), h1 = f16_of_product(v[1], HAD_SCALE);
    if (pairs) {
        // the MFMA path's pair order: within each 16-value tile, x[m + 8] then x[m] for m = 0..7
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int k = n + j, m = k & 15;
            xd[(size_t)p * N + (k & ~15) + (m < 8 ? 2 * m + 1 : 2 * (m - 8))] = j ? h1 : h0;
        }
    } else {
        *reinterpret_cast<uint32_t*>(xd + (size_t)p * N + n) = (uint32_t)h0 | ((uint32_t)h1 << 16);
    }
}

// down epilogue (exl3.cu:300-321): ordered split sum, rotation, svh_d -> y fp32. One wave a (pair, 128-block).
__global__ void __launch_bounds__(64) down_epilogue_kernel(const float* __restrict__ Z, const int* __restrict__ pick,
                                                            const uint16_t* __restrict__ svh_d, float* __restrict__ y,
                                                            int P, int D, int SK, int slots, int exl3_slots) {
    const int p = blockIdx.x, blk = blockIdx.y;
    const int row = p / slots, slot = p % slots;
    if (slot >= exl3_slots) return;
    const int lane = threadIdx.x;
    const int e = pick[row * slots + slot];
    const int n = blk * 128 + 2 * lane;
    float v[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        float s = 0.f;
        for (int k = 0; k < SK; ++k) s += Z[((size_t)k * P + p) * D + n + j];
        v[j] = s;
    }
    fwht128_w64(v, lane);
    float2 o;
    o.x = v[0] * HAD_SCALE * f16_to_f32(svh_d[(size_t)e * D + n]);
    o.y = v[1] * HAD_SCALE * f16_to_f32(svh_d[(size_t)e * D + n + 1]);
    *reinterpret_cast<float2*>(y + (size_t)p * D + n) = o;
}


// ---- one-token MoE layer in one persistent launch ----------------------------------------------------------------
// The bs = 1 layer (Moe::run_prefetched, moe.rs:66-182, for the benchmark's router) as one launch instead of three:
// route -> gate/up GEMV (rot_in fused) -> gate/up epilogue -> down GEMV -> down epilogue -> combine. Workgroup b takes
// units b, b + grid, b + 2 grid, ... in order, every gate/up unit before any down unit; the grid is at most the
// number of workgroups the GPU holds at once, so a workgroup that waits (a down unit waiting for gate/up partials)
// only waits for gate/up units of resident workgroups that never wait themselves. The down units' trellis words
// stream in while gate/up units still run; a bounded wait sets an error word instead of hanging.
//   gate/up unit (slot s, 128-column block cb, K split, matrix): 4 waves, one 128-k block each, added in wave order
//     -> Zgu partial row, then one count on the (s, cb) arrival counter.
//   down unit (slot s, split pair q, 128-column block hb of the hidden size): waves 0-1 split 2q, waves 2-3 split
//     2q + 1, 2 waves a split, one 128-k block cb each. Once the (s, cb) counters show all 2 SKgu gate/up partials,
//     each wave runs the gate/up epilogue of its own block (exl3.cu:260-296) into its activations, as the
//     three-launch path's down GEMV does; the two waves of a split are added in order -> Zd partial rows.
//   finish: the last down unit of column block hb (counted over every slot and split) runs the down epilogue
//     (exl3.cu:300-321) of every slot and the slot-ordered weighted combine -> out[hb].
// Every sum has the order of the three-launch path (same wave, split and slot order), so the output is bit for bit
// that path's. Data that other workgroups read goes through agent-scope (L2-coherent) stores and loads; a hand-off
// is: stores, s_waitcnt (the stores are complete), then the counter's atomic add. The gate/up counters only grow
// (ready = 2 SKgu arrivals past the launch's generation); the finish counters are cleared by their last arriver, and
// the very last one advances the generation, so nothing needs clearing between launches (graph replays included).
__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t add_agent(uint32_t* p, uint32_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// this wave's agent-scope stores are complete (visible to every workgroup's agent-scope loads)
__device__ __forceinline__ void stores_done() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

#ifdef GFR_TOKEN_TRACE
#define TOKEN_MARK(k) do { if (threadIdx.x == 0) a.trace[blockIdx.x * 16 + (k)] = __builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define TOKEN_MARK(k) do { } while (0)
#endif
constexpr int TOKEN_SPIN_LIMIT = 1 << 22;     // polls of a counter before the launch gives up (error word)
constexpr int TOKEN_MAX_SLOTS = 16;
constexpr int TOKEN_MAX_SPLITS = 16;           // K splits of either GEMV (hidden <= 8192, inter <= 4096)

// this wave's 128 k x 16 columns of one trellis block row against its staged activations xs (each twice)
template <int K>
__device__ __forceinline__ void token_dot(const uint32_t (&wr)[8][K], const uint32_t* xs, int i, float& acc0,
                                          float& acc1) {
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
        const uint32_t prev = prev_word(wr[kk][K - 1], i);
        uint32_t cw[32];
        lane_words<K>(wr[kk], prev, cw);
        uint32_t xd[16];
        load_tile_acts(xs + kk * 16, xd);
        float acc[2] = {acc0, acc1};
        tile_dot(cw, xd, acc);
        acc0 = acc[0];
        acc1 = acc[1];
    }
}

__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int K>
__global__ void __launch_bounds__(256) moe_token_kernel(const TokenArgs a) {
    __shared__ __attribute__((aligned(16))) uint32_t xs[4][128];   // activations, each twice
    __shared__ float red[4][128];
    __shared__ float2 ys[TOKEN_MAX_SLOTS][64];
    __shared__ uint32_t sh[2];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, t8 = lane >> 3, i = lane & 7;
    const int S = a.slots, NCB = a.N >> 7, NHB = a.D >> 7, SKgu = a.D >> 9, SKd = a.N >> 8, QD = (SKd + 1) >> 1;
    const uint32_t Tgu = (uint32_t)(S * NCB * SKgu * 2), T = Tgu + (uint32_t)(S * QD * NHB);
    uint32_t* const genp = a.sync + 1;
    uint32_t* const fcnt = a.sync + 2;
    uint32_t* const err = a.sync + 3;
    uint32_t* const gcnt = a.sync + 4;               // [S][NCB], grows by 2 SKgu a launch
    uint32_t* const hcnt = gcnt + S * NCB;           // [NHB], cleared by its last arriver
    TOKEN_MARK(0);

    int pick;                                        // lane s < S: slot s's expert and weight
    float weight;
    route_token_regs(a.logits, a.routed, S - 1, a.routed, pick, weight, RouteGate{a.route_bias, a.route_scale});
    int rank = 0;                                    // ascending order of the slots' experts
    for (int j = 0; j < S; ++j) rank += __builtin_amdgcn_readlane(pick, j) < pick;
    const uint32_t gen = ld_agent(genp);
    const uint32_t gu_ready = (gen + 1) * (uint32_t)(2 * SKgu);
    TOKEN_MARK(1);

    for (uint32_t t = blockIdx.x; t < T; t += (uint32_t)a.grid) {
        if (t == 0 && wave == 0 && lane < S) {       // the window's routing and grouping for the caller
            a.pick_out[lane] = pick;
            a.weight_out[lane] = weight;
            a.ids_out[rank] = pick;
            a.members_out[(size_t)rank * a.maxm] = lane;
            for (int j = 1; j < a.maxm; ++j) a.members_out[(size_t)rank * a.maxm + j] = -1;
            if (lane == 0) a.count_out[0] = S;
        }
        if (t < Tgu) {
            // ---- gate/up unit
            const int g = t / (2 * SKgu), r = t % (2 * SKgu);
            const int s = g / NCB, cb = g % NCB, split = r >> 1, mat = r & 1;
            const int e = __builtin_amdgcn_readlane(pick, s);
            const int KT = a.D >> 4, NT = a.N >> 4, kblk = split * 4 + wave;
            uint32_t wr[8][K];
            {
                const uint32_t* src = (mat ? a.ut : a.gt) + (((size_t)e * KT + kblk * 8) * NT + cb * 8 + t8) * (8 * K) + i * K;
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) load_words<K>(src + (size_t)kk * NT * (8 * K), wr[kk]);
            }
            const uint32_t xv = *reinterpret_cast<const uint32_t*>(a.x + kblk * 128 + 2 * lane);
            const uint32_t sv =
                *reinterpret_cast<const uint32_t*>((mat ? a.suh_u : a.suh_g) + (size_t)e * a.D + kblk * 128 + 2 * lane);
            {
                float v[2] = {bf16_to_f32((uint16_t)xv) * f16_to_f32((uint16_t)sv),
                              bf16_to_f32((uint16_t)(xv >> 16)) * f16_to_f32((uint16_t)(sv >> 16))};
                fwht128_w64(v, lane);
                store_block(xs[wave], v, lane);
                wave_sync_lds();
            }
            float acc0 = 0.f, acc1 = 0.f;
            token_dot<K>(wr, xs[wave], i, acc0, acc1);
            red[wave][16 * t8 + i] = acc0;
            red[wave][16 * t8 + i + 8] = acc1;
            __syncthreads();
            if (tid < 128) {
                const float sum = red[0][tid] + red[1][tid] + red[2][tid] + red[3][tid];
                st_agent(a.zgu + ((size_t)(mat * SKgu + split) * S + s) * a.N + cb * 128 + tid, sum);
            }
            stores_done();
            __syncthreads();
            if (tid == 0) add_agent(gcnt + s * NCB + cb, 1);
            TOKEN_MARK(2);
        } else {
            // ---- down unit
            const uint32_t td = t - Tgu;
            const int s = td / (QD * NHB), r = td % (QD * NHB), q = r / NHB, hb = r % NHB;
            const int e = __builtin_amdgcn_readlane(pick, s);
            const int sp = 2 * q + (wave >> 1), nsp = SKd - 2 * q < 2 ? SKd - 2 * q : 2;
            const bool active = sp < SKd;
            const int cb = 2 * sp + (wave & 1);          // this wave's 128-k block of the intermediate size
            const int KT = a.N >> 4, NT = a.D >> 4;
            float acc0 = 0.f, acc1 = 0.f;
            uint32_t wr[8][K];
            uint32_t sg = 0, su = 0, sd = 0;
            if (active) {
                const uint32_t* src = a.dt + (((size_t)e * KT + cb * 8) * NT + hb * 8 + t8) * (8 * K) + i * K;
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) load_words<K>(src + (size_t)kk * NT * (8 * K), wr[kk]);
                const size_t o = (size_t)e * a.N + cb * 128 + 2 * lane;
                sg = *reinterpret_cast<const uint32_t*>(a.svh_g + o);
                su = *reinterpret_cast<const uint32_t*>(a.svh_u + o);
                sd = *reinterpret_cast<const uint32_t*>(a.suh_d + o);
                // wait for the 2 SKgu gate/up partials of (s, cb), then the gate/up epilogue of the block
                int spins = 0;
                while (__builtin_amdgcn_readfirstlane(ld_agent(gcnt + s * NCB + cb)) != gu_ready) {
                    if (++spins > TOKEN_SPIN_LIMIT) {
                        if (lane == 0) __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(4);
                }
                TOKEN_MARK(5);
                const int n = cb * 128 + 2 * lane;
                float gv[2] = {0.f, 0.f}, uv[2] = {0.f, 0.f};
                {
                    float zz[TOKEN_MAX_SPLITS][4];      // every partial in flight at once, then added in order
#pragma unroll
                    for (int k = 0; k < TOKEN_MAX_SPLITS; ++k)
                        if (k < SKgu) {
                            const float* zg = a.zgu + ((size_t)k * S + s) * a.N + n;
                            const float* zu = a.zgu + ((size_t)(SKgu + k) * S + s) * a.N + n;
                            zz[k][0] = ld_agent(zg);
                            zz[k][1] = ld_agent(zg + 1);
                            zz[k][2] = ld_agent(zu);
                            zz[k][3] = ld_agent(zu + 1);
                        }
#pragma unroll
                    for (int k = 0; k < TOKEN_MAX_SPLITS; ++k)
                        if (k < SKgu) {
                            gv[0] += zz[k][0];
                            gv[1] += zz[k][1];
                            uv[0] += zz[k][2];
                            uv[1] += zz[k][3];
                        }
                }
                const float svg[2] = {f16_to_f32((uint16_t)sg), f16_to_f32((uint16_t)(sg >> 16))};
                const float svu[2] = {f16_to_f32((uint16_t)su), f16_to_f32((uint16_t)(su >> 16))};
                const float sdd[2] = {f16_to_f32((uint16_t)sd), f16_to_f32((uint16_t)(sd >> 16))};
                fwht128_w64(gv, lane);
                fwht128_w64(uv, lane);
                float v[2];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float gg = fminf(bf16r(gv[j] * HAD_SCALE * svg[j]), a.limit);
                    const float uu = fminf(fmaxf(bf16r(uv[j] * HAD_SCALE * svu[j]), -a.limit), a.limit);
                    const float act = bf16r(bf16r(gg / (1.f + expf(-gg))) * uu);
                    v[j] = act * sdd[j];
                }
                fwht128_w64(v, lane);
                store_block(xs[wave], v, lane);
                if (hb == 0)                              // the down input, for the caller (engine xd)
                    *reinterpret_cast<uint32_t*>(a.xd + (size_t)s * a.N + n) =
                        (uint32_t)f16_of_product(v[0], HAD_SCALE) | ((uint32_t)f16_of_product(v[1], HAD_SCALE) << 16);
                wave_sync_lds();
                token_dot<K>(wr, xs[wave], i, acc0, acc1);
            }
            red[wave][16 * t8 + i] = acc0;
            red[wave][16 * t8 + i + 8] = acc1;
            __syncthreads();
            TOKEN_MARK(6);
            {
                const int h = tid >> 7, col = tid & 127;     // the split pair's half h = split 2q + h
                if (h < nsp) {
                    const float sum = red[2 * h][col] + red[2 * h + 1][col];
                    st_agent(a.zd + ((size_t)(2 * q + h) * S + s) * a.D + hb * 128 + col, sum);
                }
            }
            stores_done();
            __syncthreads();
            if (tid == 0) {
                const uint32_t total = (uint32_t)(S * SKd);
                const bool last = add_agent(hcnt + hb, (uint32_t)nsp) + nsp == total;
                if (last) st_agent(hcnt + hb, 0u);
                sh[1] = last;
            }
            __syncthreads();
            if (sh[1]) {
                TOKEN_MARK(8);
                // finish of hb: every slot's down epilogue (split partials in order, transform, svh_d), then the
                // slots in order, weighted
                const int n = hb * 128 + 2 * lane;
                for (int s2 = wave; s2 < S; s2 += 4) {
                    const int e2 = __builtin_amdgcn_readlane(pick, s2);
                    float v[2] = {0.f, 0.f};
                    float zz[TOKEN_MAX_SPLITS][2];
#pragma unroll
                    for (int k = 0; k < TOKEN_MAX_SPLITS; ++k)
                        if (k < SKd) {
                            const float* z = a.zd + ((size_t)k * S + s2) * a.D + n;
                            zz[k][0] = ld_agent(z);
                            zz[k][1] = ld_agent(z + 1);
                        }
#pragma unroll
                    for (int k = 0; k < TOKEN_MAX_SPLITS; ++k)
                        if (k < SKd) {
                            v[0] += zz[k][0];
                            v[1] += zz[k][1];
                        }
                    const uint32_t sv = *reinterpret_cast<const uint32_t*>(a.svh_d + (size_t)e2 * a.D + n);
                    fwht128_w64(v, lane);
                    const float2 yv = make_float2(v[0] * HAD_SCALE * f16_to_f32((uint16_t)sv),
                                                  v[1] * HAD_SCALE * f16_to_f32((uint16_t)(sv >> 16)));
                    ys[s2][lane] = yv;
                    *reinterpret_cast<float2*>(a.y + (size_t)s2 * a.D + n) = yv;
                }
                __syncthreads();
                if (wave == 0) {
                    float o0 = 0.f, o1 = 0.f;
                    for (int s2 = 0; s2 < S; ++s2) {
                        const float w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, weight), s2));
                        o0 += w * ys[s2][lane].x;
                        o1 += w * ys[s2][lane].y;
                    }
                    *reinterpret_cast<float2*>(a.out + n) = make_float2(o0, o1);
                    TOKEN_MARK(9);
                    if (lane == 0 && add_agent(fcnt, 1) == (uint32_t)(NHB - 1)) {
                        st_agent(fcnt, 0u);
                        st_agent(genp, gen + 1);            // the layer is done: the next launch's generation
                    }
                }
            }
        }
    }
}

}  // namespace gfr

#include "launch.hpp"

namespace gfr {

hipError_t launch_decode_tiles(hipStream_t s, const uint32_t* T, int kin, int n, int bits, uint16_t* out) {
    const dim3 grid((n / 16 + 7) / 8, kin / 16);
    switch (bits) {
        case 2: decode_tiles_kernel<2><<<grid, 64, 0, s>>>(T, kin, n, out); break;
        case 3: decode_tiles_kernel<3><<<grid, 64, 0, s>>>(T, kin, n, out); break;
        case 4: decode_tiles_kernel<4><<<grid, 64, 0, s>>>(T, kin, n, out); break;
        case 5: decode_tiles_kernel<5><<<grid, 64, 0, s>>>(T, kin, n, out); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_rot_in(hipStream_t s, const uint16_t* x, int x_stride, bool in_f16, const int* pick,
                         const uint16_t* suh0, const uint16_t* suh1, uint16_t* out0, uint16_t* out1, int K, int P,
                         int slots, int exl3_slots, int mats) {
    const dim3 grid(P, K / 128, mats);
    if (in_f16)
        rot_in_kernel<true><<<grid, 64, 0, s>>>(x, x_stride, pick, suh0, suh1, out0, out1, K, slots, exl3_slots);
    else
        rot_in_kernel<false><<<grid, 64, 0, s>>>(x, x_stride, pick, suh0, suh1, out0, out1, K, slots, exl3_slots);
    return hipGetLastError();
}

// Split counts are fixed by the shape (never by the rows in the window), so a row's bits never depend on its window.
static int ktw_for(int Kin) {
    const int KT = Kin / 16;
    return KT % 16 == 0 ? 4 : KT % 8 == 0 ? 2 : 1;
}

int gemv_splits(int Kin) { return Kin / 16 / (4 * ktw_for(Kin)); }
// waves a workgroup of the block-building GEMVs: one 128-block each, as many as divide the blocks
static int nw_gateup(int D) { return (D / 128) % 4 == 0 ? 4 : 2; }   // hidden: a multiple of 256
static int nw_down(int) { return 2; }                                   // inter: a multiple of 256
int gemv_gateup_splits(int D) { return D / 128 / nw_gateup(D); }
int gemv_down_splits(int N) { return N / 128 / nw_down(N); }

template <int K, int KTW, int NW, int MATS, int XSRC, bool ROUTE1>
static hipError_t gemv_go(int rb, dim3 grid, hipStream_t s, const GemvArgs& a) {
    if (ROUTE1 || rb == 1) expert_gemv_kernel<K, KTW, NW, MATS, XSRC, 1, ROUTE1><<<grid, NW * 64, 0, s>>>(a);
    else if (rb == 2) expert_gemv_kernel<K, KTW, NW, MATS, XSRC, 2, false><<<grid, NW * 64, 0, s>>>(a);
    else if (rb == 4) expert_gemv_kernel<K, KTW, NW, MATS, XSRC, 4, false><<<grid, NW * 64, 0, s>>>(a);
    else expert_gemv_kernel<K, KTW, NW, MATS, XSRC, 8, false><<<grid, NW * 64, 0, s>>>(a);
    return hipGetLastError();
}

// member rows a chunk: the smallest of 1, 2, 4, 8 that holds the window's rows (an expert has at most `rows`)
static int rb_for(int rows) { return rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : 8; }
// programs along x: maxu experts times the chunks of rb members that an expert with `members` members needs
static unsigned chunks_x(int maxu, int members, int rb) { return (unsigned)maxu * (unsigned)((members + rb - 1) / rb); }

template <int KTW, int NW, int MATS, int XSRC, bool ROUTE1 = false>
static hipError_t gemv_bits(int bits, int rb, dim3 grid, hipStream_t s, const GemvArgs& a) {
    switch (bits) {
        case 2: return gemv_go<2, KTW, NW, MATS, XSRC, ROUTE1>(rb, grid, s, a);
        case 3: return gemv_go<3, KTW, NW, MATS, XSRC, ROUTE1>(rb, grid, s, a);
        case 4: return gemv_go<4, KTW, NW, MATS, XSRC, ROUTE1>(rb, grid, s, a);
        case 5: return gemv_go<5, KTW, NW, MATS, XSRC, ROUTE1>(rb, grid, s, a);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv(hipStream_t s, const uint16_t* X0, const uint16_t* X1, const uint32_t* T0, const uint32_t* T1,
                       const int* uids, const int* ucount, const int* members, float* Z, int Kin, int N, int P,
                       int maxm, int slots, int E, int bits, int mats, int maxu) {
    GemvArgs a{};
    a.x0 = X0; a.x1 = X1; a.t0 = T0; a.t1 = T1; a.uids = uids; a.ucount = ucount; a.members = members; a.z = Z;
    a.Kin = Kin; a.N = N; a.P = P; a.SK = gemv_splits(Kin); a.maxm = maxm; a.slots = slots; a.E = E;
    const int ktw = ktw_for(Kin), rb = rb_for(maxm);
    a.ucap = maxu;
    const dim3 grid(chunks_x(maxu, maxm, rb), N / 128, mats * a.SK);
    if (mats == 2) {
        if (ktw == 4) return gemv_bits<4, 4, 2, 0>(bits, rb, grid, s, a);
        if (ktw == 2) return gemv_bits<2, 4, 2, 0>(bits, rb, grid, s, a);
        return gemv_bits<1, 4, 2, 0>(bits, rb, grid, s, a);
    }
    if (ktw == 4) return gemv_bits<4, 4, 1, 0>(bits, rb, grid, s, a);
    if (ktw == 2) return gemv_bits<2, 4, 1, 0>(bits, rb, grid, s, a);
    return gemv_bits<1, 4, 1, 0>(bits, rb, grid, s, a);
}

hipError_t launch_expert_gateup(hipStream_t s, const uint16_t* x, int x_stride, const uint16_t* suh_g,
                                const uint16_t* suh_u, const uint32_t* gt, const uint32_t* ut, const int* uids,
                                const int* ucount, const int* members, float* Zgu, int D, int N, int P, int rows,
                                int maxm, int slots, int E, int bits, int maxu, const RouteOne* route) {
    GemvArgs a{};
    a.x0 = x; a.x_stride = x_stride; a.suh0 = suh_g; a.suh1 = suh_u; a.t0 = gt; a.t1 = ut;
    a.uids = uids; a.ucount = ucount; a.members = members; a.z = Zgu; a.Kin = D; a.N = N; a.P = P;
    a.SK = gemv_gateup_splits(D); a.maxm = maxm; a.slots = slots; a.E = E;
    const int nw = nw_gateup(D), rb = route ? 1 : rb_for(rows);
    a.ucap = maxu;
    const dim3 grid(chunks_x(maxu, rows < maxm ? rows : maxm, rb), N / 128, 2 * a.SK);
    if (route) {
        a.logits = route->logits; a.routed = route->routed; a.pick_out = route->picks; a.weight_out = route->weights;
        a.route_bias = route->bias; a.route_scale = route->scale;
        a.ids_out = route->ids; a.count_out = route->count; a.members_out = route->members;
        return nw == 4 ? gemv_bits<8, 4, 2, 1, true>(bits, 1, grid, s, a) : gemv_bits<8, 2, 2, 1, true>(bits, 1, grid, s, a);
    }
    return nw == 4 ? gemv_bits<8, 4, 2, 1>(bits, rb, grid, s, a) : gemv_bits<8, 2, 2, 1>(bits, rb, grid, s, a);
}

hipError_t launch_expert_down(hipStream_t s, const float* Zgu, int D, const uint16_t* svh_g, const uint16_t* svh_u,
                              const uint16_t* suh_d, float limit, uint16_t* xd, const uint32_t* dt, const int* uids,
                              const int* ucount, const int* members, float* Zd, int N, int P, int rows, int maxm,
                              int slots, int E, int bits, int maxu) {
    GemvArgs a{};
    a.zgu = Zgu; a.SKgu = gemv_gateup_splits(D); a.svh_g = svh_g; a.svh_u = svh_u; a.suh0 = suh_d; a.limit = limit;
    a.xd = xd; a.t0 = dt; a.t1 = dt; a.uids = uids; a.ucount = ucount; a.members = members; a.z = Zd;
    a.Kin = N; a.N = D; a.P = P; a.SK = gemv_down_splits(N); a.maxm = maxm; a.slots = slots; a.E = E;
    const int rb = rb_for(rows);
    a.ucap = maxu;
    return gemv_bits<8, 2, 1, 2>(bits, rb, dim3(chunks_x(maxu, rows < maxm ? rows : maxm, rb), D / 128, a.SK), s, a);
}

// One linear with its input rotation fused (XSRC 1, fp16 input): Z[split][n] partials of
// W_q[0] over one row, SK = kin / 128 / NW splits in fixed order (gemv_linear_splits).
static int nw_linear(int kin) { return (kin / 128) % 4 == 0 ? 4 : 2; }
int gemv_linear_splits(int kin) { return kin / 128 / nw_linear(kin); }
hipError_t launch_linear_fused(hipStream_t s, const uint16_t* x, const uint16_t* suh, const uint32_t* trellis,
                               const int* uids, const int* ucount, const int* members, float* z, int kin, int n,
                               int bits) {
    GemvArgs a{};
    a.x0 = x; a.x_stride = kin; a.x_f16 = 1; a.suh0 = suh; a.suh1 = suh; a.t0 = trellis; a.t1 = trellis;
    a.uids = uids; a.ucount = ucount; a.members = members; a.z = z; a.Kin = kin; a.N = n; a.P = 1;
    a.SK = gemv_linear_splits(kin); a.maxm = 1; a.slots = 1; a.E = 1; a.ucap = 1;
    const dim3 grid(1, n / 128, a.SK);
    const bool four = nw_linear(kin) == 4;
    switch (bits) {
#define GFR_LIN(KB)                                                                                                 \
        case KB:                                                                                                  \
            if (four) expert_gemv_kernel<KB, 8, 4, 1, 1, 1, false><<<grid, 256, 0, s>>>(a);                         \
            else expert_gemv_kernel<KB, 8, 2, 1, 1, 1, false><<<grid, 128, 0, s>>>(a);                              \
            break;
        GFR_LIN(2) GFR_LIN(3) GFR_LIN(4) GFR_LIN(5)
#undef GFR_LIN
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_down_finish(hipStream_t s, const float* Zd, const int* pick, const uint16_t* svh_d, float* y,
                              int rows, int P, int D, int SK, int slots, int exl3_slots, const float* weights,
                              float* out) {
    const int nwv = exl3_slots < 16 ? (exl3_slots > 0 ? exl3_slots : 1) : 16;
    down_finish_kernel<<<dim3(rows, D / 128), 64 * nwv, 0, s>>>(Zd, pick, svh_d, y, P, D, SK, slots, exl3_slots,
                                                                weights, out);
    return hipGetLastError();
}

hipError_t launch_gateup_epilogue(hipStream_t s, const float* Z, const int* pick, const uint16_t* svh_g,
                                  const uint16_t* svh_u, const uint16_t* suh_d, uint16_t* xd, int P, int N, int SK,
                                  int slots, int exl3_slots, float limit, bool pair_order) {
    gateup_epilogue_kernel<<<dim3(P, N / 128), 64, 0, s>>>(Z, pick, svh_g, svh_u, suh_d, xd, P, N, SK, slots,
                                                           exl3_slots, limit, pair_order ? 1 : 0);
    return hipGetLastError();
}

int token_sync_words(int slots, int D, int N) { return 4 + slots * (N / 128) + D / 128; }

int token_units(int slots, int D, int N) {
    const int SKd = N / 256;
    return slots * (N / 128) * (D / 512) * 2 + slots * ((SKd + 1) / 2) * (D / 128);
}

bool token_shape_ok(int D, int N) {
    return D % 512 == 0 && N % 256 == 0 && D / 512 <= TOKEN_MAX_SPLITS && N / 256 <= TOKEN_MAX_SPLITS;
}
int token_max_slots() { return TOKEN_MAX_SLOTS; }

int token_blocks_per_cu(int bits) {
    int nb = 0;
    hipError_t e = hipErrorInvalidValue;
    switch (bits) {
        case 2: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, moe_token_kernel<2>, 256, 0); break;
        case 3: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, moe_token_kernel<3>, 256, 0); break;
        case 4: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, moe_token_kernel<4>, 256, 0); break;
        case 5: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, moe_token_kernel<5>, 256, 0); break;
    }
    return e == hipSuccess ? nb : 0;
}

hipError_t launch_moe_token(hipStream_t s, const TokenArgs& a, int bits) {
    switch (bits) {
        case 2: moe_token_kernel<2><<<a.grid, 256, 0, s>>>(a); break;
        case 3: moe_token_kernel<3><<<a.grid, 256, 0, s>>>(a); break;
        case 4: moe_token_kernel<4><<<a.grid, 256, 0, s>>>(a); break;
        case 5: moe_token_kernel<5><<<a.grid, 256, 0, s>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_down_epilogue(hipStream_t s, const float* Z, const int* pick, const uint16_t* svh_d, float* y,
                                int P, int D, int SK, int slots, int exl3_slots) {
    down_epilogue_kernel<<<dim3(P, D / 128), 64, 0, s>>>(Z, pick, svh_d, y, P, D, SK, slots, exl3_slots);
    return hipGetLastError();
}

}  // namespace gfr
