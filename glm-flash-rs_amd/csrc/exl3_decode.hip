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
#include "shared_fp8.hpp"

#ifndef GFR_GEMV_PRE
#define GFR_GEMV_PRE 2   // trellis tiles a wave issues before it waits for its activations
#endif

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
    const uint32_t packed = f16x2_of_products(v[0], v[1], HAD_SCALE);
    *reinterpret_cast<uint32_t*>(o) = packed;
}


// Orders this wave's LDS stores before its own later LDS reads (the slots are the wave's own).
__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Arguments of the decode GEMV (one struct in the kernarg segment).
struct GemvArgs {
    const uint16_t* x0;      // XSRC 0: fp16 rotated rows [P][Kin] (matrix 0); XSRC 1: bf16 input rows [rows][x_stride]
    const uint16_t* x1;      // XSRC 0: fp16 rotated rows of matrix 1
    int x_stride;
    const uint16_t* suh0;    // XSRC 1: input scales [E][Kin] of the two matrices; down GEMV: suh_d [E][Kin]
    const uint16_t* suh1;
    const uint32_t* t0;      // trellis [E][Kin/16][N/16][8K]
    const uint32_t* t1;
    const int* uids;
    const int* ucount;
    const int* members;      // [E][maxm]
    float* z;                // [MATS][SK][P][N] split partials (output)
    int Kin, N, P, SK, maxm, slots, E;
    const float* zgu;        // down GEMV: the gate/up split partials [2][SKgu][P][Kin]
    int SKgu;
    const uint16_t* svh_g;   // down GEMV: gate / up output scales [E][Kin]
    const uint16_t* svh_u;
    float limit;
    uint16_t* xd;            // down GEMV: the down input, also stored (column block 0 only) [P][Kin] fp16
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
    const uint32_t* tnext;   // gate/up GEMV: the down trellis [E][...] read ahead by the gate waves, or nullptr
    size_t next_words;       // its words an expert
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
//   instead), then the activation loads and the first trellis words, then the rest of the trellis words once the
//   activation loads have landed. Activation sources (each bit for bit the reference's formula), staged per wave in
//   LDS:
//   XSRC 0  rotated fp16 rows (exl3.cu's grouped kernel input);
//   XSRC 1  rot_in fused (exl3.cu:224-241): bf16 input row * suh -> 128-point transform -> fp16; KTW = 8, one block.
//   ROUTE1  (one-token windows) the wave routes the token itself (route.hpp) from a.logits: the window's experts
//           are the token's slots; program (0, 0, 0) stores picks / weights / ids / count / members for the later
//           launches.
template <int K, int KTW, int NW, int MATS, int XSRC, int RB, bool ROUTE1, bool FP8>
__device__ __forceinline__ void expert_gemv_body(const GemvArgs& a, const Fp8Args& f) {
    constexpr int KC = NW * KTW;
    static_assert(XSRC == 0 || KTW == 8 || KTW == 4 || KTW == 2,
                  "a wave that builds its activations covers one 128-point block or a part of one");
    static_assert(XSRC != 0 || RB * KTW <= 64, "one lane a (member, k tile) when staging rotated rows");
    __shared__ __attribute__((aligned(16))) uint32_t xs[NW][RB][KTW * 16];   // activations, each twice
    __shared__ float red[NW][RB][128];

    const int u = blockIdx.x % a.ucap, cb = blockIdx.y, c0 = (int)(blockIdx.x / a.ucap) * RB;
    const int split = blockIdx.z % a.SK, mat = MATS == 1 ? 0 : blockIdx.z / a.SK;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, t = lane >> 3, i = lane & 7;
    const int KT = a.Kin >> 4, NT = a.N >> 4;
    const int kt0 = split * KC + wave * KTW;

    int e, code;
    uint32_t xearly = 0;   // ROUTE1 with the fused rotation: the token's input pair, loaded while it is routed
    if constexpr (ROUTE1) {
        if constexpr (FP8) {
            if (u == a.slots - 1) {
                // the layer's shared expert is FP8: this unit's workgroups run its gate/up programs (8 intermediate
                // indices each) instead of an EXL3 expert's
                __shared__ Fp8Part fp8_part;
                const int nb = gridDim.y * gridDim.z;
                for (int j = blockIdx.y + gridDim.y * blockIdx.z; j < f.inter / 8; j += nb) {
                    fp8_gu_program<8, NW, 4>(f.w, f.s, f.x, f.hidden, 1, 0, f.hidden, f.inter, j, wave, lane,
                                             fp8_part, f.gu, f.act);
                    __syncthreads();                      // fp8_part is the next program's
                }
                return;
            }
        }
        if constexpr (XSRC == 1)
            xearly = *reinterpret_cast<const uint32_t*>(a.x0 + (kt0 & ~7) * 16 + 2 * lane);
        if (u == a.slots - 1) {
            // the shared expert (id `routed`, above every routed id, in the last slot) is always the window's last
            // unit: its waves need no routing and start their trellis stream at once
            e = a.routed;
            code = lane == 0 ? a.slots - 1 : -1;
        } else {
            int pick;
            float weight;
            // only the wave that publishes the routing needs the weights (the others use the picks)
            const bool writer = u == 0 && cb == 0 && blockIdx.z == 0 && wave == 0;
            route_token_regs(a.logits, a.routed, a.slots - 1, a.routed, pick, weight,
                             RouteGate{a.route_bias, a.route_scale}, writer);
            int rank = 0;                                // ascending order of the token's slots' experts
            for (int j = 0; j < a.slots; ++j) rank += __builtin_amdgcn_readlane(pick, j) < pick;
            const uint64_t mine = __ballot(lane < a.slots && rank == u);
            if (mine == 0) return;                       // u >= slots: no such expert
            const int slot = __builtin_ctzll(mine);
            e = __builtin_amdgcn_readlane(pick, slot);
            code = lane == 0 ? slot : -1;                // row 0, this slot
            if (writer && lane < a.slots) {
                a.pick_out[lane] = pick;
                a.weight_out[lane] = weight;
                a.ids_out[rank] = pick;
                a.members_out[(size_t)rank * a.maxm] = lane;
                for (int j = 1; j < a.maxm; ++j) a.members_out[(size_t)rank * a.maxm + j] = -1;
                if (lane == 0) a.count_out[0] = a.slots;
            }
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
    uint32_t xv[RB], sv = 0;                              // XSRC 1: bf16 pairs; scale pair
    uint4 va = {0, 0, 0, 0}, vb = {0, 0, 0, 0};           // XSRC 0: this lane's k tile of one member
    auto load_acts = [&](int r0, int nr) {
        if constexpr (XSRC == 1) {
            // the whole 128-point block of the wave's k tiles (the transform needs all of it)
            sv = *reinterpret_cast<const uint32_t*>((mat ? a.suh1 : a.suh0) + (size_t)e * a.Kin + (kt0 & ~7) * 16 + 2 * lane);
            if constexpr (ROUTE1) {
                xv[0] = xearly;
            } else {
#pragma unroll
                for (int m = 0; m < RB; ++m) {
                    const int row = __builtin_amdgcn_readlane(code, r0 + (m < nr ? m : 0)) >> 5;
                    xv[m] = *reinterpret_cast<const uint32_t*>(a.x0 + (size_t)row * a.x_stride + (kt0 & ~7) * 16 + 2 * lane);
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
    // issue: called once the activations are built, to start the rest of the trellis words (issued any earlier,
    // under the other waves' streams, they delayed the activations more than they gained, measured on MI355X)
    auto build_acts = [&](int r0, int nr, auto&& issue) {
        if constexpr (XSRC == 1) {
            const float s0 = f16_to_f32((uint16_t)sv), s1 = f16_to_f32((uint16_t)(sv >> 16));
            float v[RB][2];
#pragma unroll
            for (int m = 0; m < RB; ++m) {
                const uint16_t x0 = (uint16_t)xv[m], x1 = (uint16_t)(xv[m] >> 16);
                v[m][0] = (a.x_f16 ? f16_to_f32(x0) : bf16_to_f32(x0)) * s0;
                v[m][1] = (a.x_f16 ? f16_to_f32(x1) : bf16_to_f32(x1)) * s1;
            }
#pragma unroll
            for (int m = 0; m < RB; ++m)
                if (m < nr) {
                    fwht128_w64(v[m], lane);
                    // this wave's k tiles of the block: its lanes [8 sub, 8 (sub + KTW)), at slot 0 onwards
                    const int sub = kt0 & 7;
                    if (KTW == 8 || (lane >= 8 * sub && lane < 8 * (sub + KTW)))
                        store_block(&xs[wave][m][0] - 16 * sub, v[m], lane);
                }
            __builtin_amdgcn_sched_barrier(0);
            issue();
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
            issue();
        }
        // the slots are this wave's own: a wave-level barrier orders the LDS stores before the reads
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    const int nr0 = cnt - c0 < RB ? cnt - c0 : RB;
    // Load order: the activations and the first PRE trellis tiles, then the activations built (waiting only for
    // their own loads and the tiles issued before them), then the rest of the trellis words. Every wave of the launch
    // issues its trellis stream at about the same time; activation loads queued behind that whole stream would arrive
    // only once most of it had landed, and no tile could be decoded before then. Issued ahead of the bulk, they land
    // early and the decode overlaps the stream.
    load_acts(c0, nr0);
    uint32_t wr[KTW][K];
    const uint32_t* tsrc = (mat ? a.t1 : a.t0) + (((size_t)e * KT + kt0) * NT + cb * 8 + t) * (8 * K) + i * K;
    constexpr int PRE = GFR_GEMV_PRE < KTW ? GFR_GEMV_PRE : KTW;
#pragma unroll
    for (int kk = 0; kk < PRE; ++kk) load_words<K>(tsrc + (size_t)kk * NT * (8 * K), wr[kk]);
    // keep this order (left alone, the scheduler sinks the activation loads below the decode and splits the trellis
    // loads into dependent rounds)
    __builtin_amdgcn_sched_barrier(0);

    const CodewordConsts cc = codeword_consts<K>();
    // the chunk of up to RB members (its activations are already loading)
    auto chunk = [&](int r0, int nr) {
        build_acts(r0, nr, [&]() {
#pragma unroll
            for (int kk = PRE; kk < KTW; ++kk) load_words<K>(tsrc + (size_t)kk * NT * (8 * K), wr[kk]);
        });
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
            lane_words<K>(wr[kk], prev, cw, cc);
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
    // Read-ahead of this expert's down matrix for the next launch. The gate waves (mat 0, first chunk) end about 2 us
    // before the up waves that share their CUs, with the HBM idle: each loads one dword of every 128-byte line of its
    // share (gridDim.y * SK * NW gate waves an expert, at most 4 lines a lane), so the down launch's trellis loads hit
    // the memory-side cache instead of HBM. A lane's loads and the wait for them are one asm statement with
    // early-clobber outputs: the loaded registers are never read, and no register the compiler allocates can be
    // written by a load still in flight (a late return into a reused address register sends the next load astray).
    if (MATS == 2 && a.tnext && mat == 0 && c0 == 0) {
        const int nwv = (int)gridDim.y * a.SK * NW, widx = ((int)blockIdx.y * a.SK + split) * NW + wave;
        const size_t lines = a.next_words / 32, per = (lines + nwv - 1) / nwv;
        const size_t l0 = (size_t)widx * per, l1 = l0 + per < lines ? l0 + per : lines;
        if (l0 < l1 && per <= 256) {
            const uint32_t* base = a.tnext + (size_t)e * a.next_words;
            // lines past the share re-read its last line (the count is the wave's, the same on every lane)
            auto at = [&](int j) {
                const size_t l = l0 + lane + 64 * j;
                return base + (l < l1 ? l : l1 - 1) * 32;
            };
            uint32_t d0, d1, d2, d3;
            const int nl = (int)((per + 63) / 64);
            if (nl == 1)
                __asm__ volatile("global_load_dword %0, %1, off\n\ts_waitcnt vmcnt(0)"
                                 : "=&v"(d0) : "v"(at(0)) : "memory");
            else if (nl == 2)
                __asm__ volatile("global_load_dword %0, %2, off\n\tglobal_load_dword %1, %3, off\n\t"
                                 "s_waitcnt vmcnt(0)"
                                 : "=&v"(d0), "=&v"(d1) : "v"(at(0)), "v"(at(1)) : "memory");
            else
                __asm__ volatile("global_load_dword %0, %4, off\n\tglobal_load_dword %1, %5, off\n\t"
                                 "global_load_dword %2, %6, off\n\tglobal_load_dword %3, %7, off\n\t"
                                 "s_waitcnt vmcnt(0)"
                                 : "=&v"(d0), "=&v"(d1), "=&v"(d2), "=&v"(d3)
                                 : "v"(at(0)), "v"(at(1)), "v"(at(2)), "v"(at(3)) : "memory");
        }
    }
}

template <int K, int KTW, int NW, int MATS, int XSRC, int RB, bool ROUTE1>
__global__ void __launch_bounds__(NW * 64) expert_gemv_kernel(const GemvArgs a) {
    expert_gemv_body<K, KTW, NW, MATS, XSRC, RB, ROUTE1, false>(a, Fp8Args{});
}
// The one-token form with the layer's FP8 shared expert in the shared unit's workgroups (kept apart so that the
// layers without one run the kernel above unchanged).
template <int K, int KTW, int NW, int MATS, int XSRC, int RB, bool ROUTE1>
__global__ void __launch_bounds__(NW * 64) expert_gemv_fp8_kernel(const GemvArgs a, const Fp8Args f) {
    expert_gemv_body<K, KTW, NW, MATS, XSRC, RB, ROUTE1, true>(a, f);
}

// ---- down GEMV of the decode path ------------------------------------------------------------------------------
// Program (unit, 128-column block hb of the hidden size, 128-k block kb of the intermediate size), NW waves. A unit is
// (member chunk, distinct expert u) of the grouping tables, or with TOKEN (a one-token window routed by the gate/up
// launch) the token's slot, whose expert is its pick and whose pair is the slot itself. The k block's activations are
// the gate/up epilogue (exl3.cu:260-296) of its 128 intermediate values: the gate / up split partials summed in split
// order, transforms, svh scales, GLM's limited SwiGLU with its bf16 roundings, suh_d, transform -> fp16 (stored to xd
// by the hb == 0 programs). Wave w builds the epilogue of members w and w + NW into LDS while every wave streams and
// decodes its own 8 / NW k tiles (kb * 8 + w * 8 / NW, ...) of the block's 8 column tiles into registers; after one
// barrier each wave dots its tiles, the waves are added in order and the k block's sum goes through the down
// epilogue's transform and svh_d scale (exl3.cu:300-321; linear, so it applies to each k block's part) into
// Zd[kb][pair][hidden]. The finish launch adds the k blocks in order. Every sum has a fixed order, and a row's result
// never depends on the other rows (NW, which sets the order of the waves' sums, is fixed by the shape and by TOKEN).
//   a.Kin = intermediate size (the down input), a.N = hidden size; a.suh0 = suh_d, a.svh_g / svh_u the gate / up
//   output scales, a.t0 the down trellis, a.zgu / SKgu the gate/up partials, a.z = Zd, a.x1 (reused) = svh_d.
// hidden sizes from which a down workgroup covers two 128-output blocks
constexpr int DOWN_HB2_MIN = 4096;

// The dispatcher hands workgroup L (linear launch order) to XCD L % 8, and each XCD has its own L2. Renumber the grid
// so that XCD x runs the logical range [x T/8, (x+1) T/8) with y (the output row block) fastest, then x, then z: the
// row blocks of one (unit, k block) then share one L2 for the partials and scales they all read. Grids whose size
// is not a multiple of 8 keep the launch order.
__device__ inline void xcd_grouped(int& bx, int& by, int& bz) {
    bx = blockIdx.x; by = blockIdx.y; bz = blockIdx.z;
    const int gx = gridDim.x, gy = gridDim.y, T = gx * gy * gridDim.z;
    if (T & 7) return;
    const int L = bx + gx * (by + gy * bz), g = (L & 7) * (T >> 3) + (L >> 3);
    by = g % gy;
    bx = (g / gy) % gx;
    bz = g / (gy * gx);
}

template <int K, int RB, int HB, bool TOKEN, int NW, int TZ, bool FP8>
__device__ __forceinline__ void down_gemv_body(const GemvArgs& a, const Fp8Args& f) {
    constexpr int TPW = 8 / NW;                          // k tiles a wave of the 128-k block
    static_assert(NW == 1 || NW == 4, "waves a workgroup");
    __shared__ __attribute__((aligned(16))) uint32_t xs[RB][128];   // the k block's activations, each twice
    __shared__ float red[NW][RB][128 * HB];
    __shared__ float2 psum[NW][RB][2][64];                           // each wave's share of the gate / up splits
    int bx, hb, kb;
    xcd_grouped(bx, hb, kb);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, t = lane >> 3, i = lane & 7;
    const int KT = a.Kin >> 4, NT = a.N >> 4;
    const int n = kb * 128 + 2 * lane;
    const int spw = (a.SKgu + NW - 1) / NW, s0 = wave * spw, s1 = s0 + spw < a.SKgu ? s0 + spw : a.SKgu;
    // the gate/up epilogue inputs: every wave loads its quarter of the K splits of every member (splits
    // [w * SPW, (w + 1) * SPW), four in flight, added in order) into LDS; the wave building member m then adds the
    // four quarters in wave order (members w and w + 4 are built by wave w)
    auto load_partials = [&](int m, int p) {
        float2 g = make_float2(0.f, 0.f), u = make_float2(0.f, 0.f);
        for (int k0 = s0; k0 < s1; k0 += 4) {
            float2 zg[4], zu[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int kk = k0 + k < s1 ? k0 + k : s0;
                zg[k] = *reinterpret_cast<const float2*>(a.zgu + ((size_t)kk * a.P + p) * a.Kin + n);
                zu[k] = *reinterpret_cast<const float2*>(a.zgu + ((size_t)(a.SKgu + kk) * a.P + p) * a.Kin + n);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (k0 + k < s1) {
                    g.x += zg[k].x; g.y += zg[k].y;
                    u.x += zu[k].x; u.y += zu[k].y;
                }
        }
        psum[wave][m][0][lane] = g;
        psum[wave][m][1][lane] = u;
    };
    int e, nr, c0, pair_l;
    float2 tzg[TZ], tzu[TZ];                            // TOKEN: this wave's split partials, in flight
    if constexpr (TOKEN) {
        // a one-token window routed by the gate/up launch (RB 1): program bx is the token's slot bx, pair bx. The
        // slot's partials need no table, so they are loaded at once, next to the slot's expert (the shared expert,
        // id `routed` in the last slot, needs no load at all); only the trellis and scale loads wait for the id.
        // (TZ >= the wave's share of the splits, set by the host; every wave issues TZ loads, past its share
        // re-reading its first split)
        const int slot = bx;
        if constexpr (FP8) {
            if (slot == a.slots - 1) {
                // the layer's shared expert is FP8: this slot's workgroups run its down programs (a 16-column tile
                // a wave) instead of an EXL3 expert's
                const int nb = gridDim.y * gridDim.z;
                for (int nt = (hb + gridDim.y * kb) * NW + wave; nt < f.hidden / 16; nt += nb * NW)
                    fp8_down_program<4>(f.w, f.s, f.x, 1, 0, f.inter, nt, lane, f.out, f.hidden);
                return;
            }
        }
        c0 = 0;
        nr = 1;
        pair_l = slot;
#pragma unroll
        for (int k = 0; k < TZ; ++k) {
            const int kk = s0 + k < s1 ? s0 + k : (s0 < a.SKgu ? s0 : 0);
            tzg[k] = *reinterpret_cast<const float2*>(a.zgu + ((size_t)kk * a.P + slot) * a.Kin + n);
            tzu[k] = *reinterpret_cast<const float2*>(a.zgu + ((size_t)(a.SKgu + kk) * a.P + slot) * a.Kin + n);
        }
        __builtin_amdgcn_sched_barrier(0);
        e = slot == a.slots - 1 ? a.routed : a.pick_out[slot];
        if (e >= a.E) return;
    } else {
        const int u = bx % a.ucap;
        c0 = (bx / a.ucap) * RB;
        const int cntu = a.ucount[0];
        e = a.uids[u];
        const int code = lane < a.maxm ? a.members[(size_t)u * a.maxm + lane] : -1;
        if (u >= cntu || e >= a.E || (c0 > 0 && __builtin_amdgcn_readlane(code, c0 & 63) < 0)) return;
        const int cnt = __popcll(__ballot(code >= 0));
        nr = cnt - c0 < RB ? cnt - c0 : RB;
        pair_l = code >= 0 ? (code >> 5) * a.slots + (code & 31) : 0;
    }

    constexpr int EM = RB > 4 ? 2 : 1;                  // members a wave builds
    const size_t so = (size_t)e * a.Kin + n;
    const bool builds = wave < nr;
    uint32_t sg = 0, su = 0, sd = 0;
    if (builds) {
        sg = *reinterpret_cast<const uint32_t*>(a.svh_g + so);
        su = *reinterpret_cast<const uint32_t*>(a.svh_u + so);
        sd = *reinterpret_cast<const uint32_t*>(a.suh0 + so);
    }
    // the down epilogue's output scales of this wave's (member, block) parts (wave q < nr HB takes part q), loaded
    // with the other scales instead of after the dots
    uint32_t svd = 0;
    if (wave < nr * HB) {
        const int h = wave % HB;
        svd = *reinterpret_cast<const uint32_t*>(a.x1 + (size_t)e * a.N + (hb * HB + h) * 128 + 2 * lane);
    }
    // HB output blocks of 128: the same two k tiles of each (column tiles (hb HB + h) 8 + t); the first block's
    // words decoded before the barrier, the others' kept as words and decoded after the first block's dots
    uint32_t wr[HB][TPW][K];
    {
        const uint32_t* src = a.t0 + (((size_t)e * KT + kb * 8 + TPW * wave) * NT + hb * HB * 8 + t) * (8 * K) + i * K;
#pragma unroll
        for (int h = 0; h < HB; ++h) {
#pragma unroll
            for (int kk = 0; kk < TPW; ++kk) load_words<K>(src + (size_t)kk * NT * (8 * K) + h * 8 * (8 * K), wr[h][kk]);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (TOKEN) {
        float2 g = make_float2(0.f, 0.f), u = make_float2(0.f, 0.f);
#pragma unroll
        for (int k = 0; k < TZ; ++k)
            if (s0 + k < s1) {
                g.x += tzg[k].x; g.y += tzg[k].y;
                u.x += tzu[k].x; u.y += tzu[k].y;
            }
        psum[wave][0][0][lane] = g;
        psum[wave][0][1][lane] = u;
    } else {
        for (int m = 0; m < nr; ++m) load_partials(m, __builtin_amdgcn_readlane(pair_l, (c0 + m) & 63));
    }
    __syncthreads();
    if (builds) {
        const float svg[2] = {f16_to_f32((uint16_t)sg), f16_to_f32((uint16_t)(sg >> 16))};
        const float svu[2] = {f16_to_f32((uint16_t)su), f16_to_f32((uint16_t)(su >> 16))};
        const float sdd[2] = {f16_to_f32((uint16_t)sd), f16_to_f32((uint16_t)(sd >> 16))};
#pragma unroll
        for (int q = 0; q < EM; ++q) {
            const int m = wave + NW * q;
            if (m < nr) {
                float gv[2] = {0.f, 0.f}, uv[2] = {0.f, 0.f};
#pragma unroll
                for (int w = 0; w < NW; ++w) {
                    const float2 g = psum[w][m][0][lane], u = psum[w][m][1][lane];
                    gv[0] += g.x; gv[1] += g.y;
                    uv[0] += u.x; uv[1] += u.y;
                }
                fwht128_w64(gv, lane);
                fwht128_w64(uv, lane);
                float v[2];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float gg = fminf(bf16r(gv[j] * HAD_SCALE * svg[j]), a.limit);
                    const float uu = __builtin_amdgcn_fmed3f(bf16r(uv[j] * HAD_SCALE * svu[j]), -a.limit, a.limit);
                    const float act = bf16r(bf16r(gg / (1.f + expf(-gg))) * uu);
                    v[j] = act * sdd[j];
                }
                fwht128_w64(v, lane);
                store_block(&xs[m][0], v, lane);
                if (hb == 0 && a.xd) {
                    const int p = __builtin_amdgcn_readlane(pair_l, (c0 + m) & 63);
                    *reinterpret_cast<uint32_t*>(a.xd + (size_t)p * a.Kin + n) =
                        f16x2_of_products(v[0], v[1], HAD_SCALE);
                }
            }
        }
    }
    // ---- this wave's two tiles of the first block decoded (they wait for their own words only)
    const CodewordConsts cc = codeword_consts<K>();
    uint32_t cw[TPW][32];
    auto decode_block = [&](int h) {
#pragma unroll
        for (int kk = 0; kk < TPW; ++kk) {
#pragma unroll
            for (int j = 0; j < K; ++j) __asm__ volatile("" : "+v"(wr[h][kk][j]));
            lane_words<K>(wr[h][kk], prev_word(wr[h][kk][K - 1], i), cw[kk], cc);
        }
    };
    decode_block(0);
    __syncthreads();                                     // every member's activations are in LDS
#pragma unroll
    for (int h = 0; h < HB; ++h) {
        if (h > 0) decode_block(h);
#pragma unroll
        for (int m = 0; m < RB; ++m) {
            if (m < nr) {
                float acc[2] = {0.f, 0.f};
#pragma unroll
                for (int kk = 0; kk < TPW; ++kk) {
                    uint32_t xd[16];
                    load_tile_acts(&xs[m][(TPW * wave + kk) * 16], xd);
                    tile_dot(cw[kk], xd, acc);
                }
                red[wave][m][128 * h + 16 * t + i] = acc[0];
                red[wave][m][128 * h + 16 * t + i + 8] = acc[1];
            }
        }
    }
    __syncthreads();
    // ---- the four waves in order, then the down epilogue's transform and scale of this k block's part, a (member,
    // block) a wave
    for (int q = wave; q < nr * HB; q += NW) {
        const int m = q / HB, h = q - m * HB, ob = (hb * HB + h) * 128;
        const uint32_t sv = q < NW ? svd : *reinterpret_cast<const uint32_t*>(a.x1 + (size_t)e * a.N + ob + 2 * lane);
        float v[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int c = 128 * h + 2 * lane + j;
            v[j] = red[0][m][c];
#pragma unroll
            for (int w = 1; w < NW; ++w) v[j] += red[w][m][c];
        }
        fwht128_w64(v, lane);
        const int p = __builtin_amdgcn_readlane(pair_l, (c0 + m) & 63);
        *reinterpret_cast<float2*>(a.z + ((size_t)kb * a.P + p) * a.N + ob + 2 * lane) =
            make_float2(v[0] * HAD_SCALE * f16_to_f32((uint16_t)sv), v[1] * HAD_SCALE * f16_to_f32((uint16_t)(sv >> 16)));
    }
}

template <int K, int RB, int HB, bool TOKEN, int NW, int TZ = 4>
__global__ void __launch_bounds__(NW * 64) down_gemv_kernel(const GemvArgs a) {
    down_gemv_body<K, RB, HB, TOKEN, NW, TZ, false>(a, Fp8Args{});
}
template <int K, int RB, int HB, bool TOKEN, int NW, int TZ = 4>
__global__ void __launch_bounds__(NW * 64) down_gemv_fp8_kernel(const GemvArgs a, const Fp8Args f) {
    down_gemv_body<K, RB, HB, TOKEN, NW, TZ, true>(a, f);
}

// The combine's terms past the EXL3 slots (the reference's combine(y, shared, weights, out), moe.rs:171-181): the
// caller's shared-expert output for each slot s >= exl3_slots, weighted, after the EXL3 slots (slot order).
__device__ __forceinline__ void combine_shared(const float* __restrict__ w, int slots, int exl3_slots,
                                               const float* __restrict__ shared, int shared_stride, int row, int n,
                                               float& o0, float& o1) {
    if (!shared) return;
    for (int s = exl3_slots; s < slots; ++s) {
        const float2 v = *reinterpret_cast<const float2*>(shared + (size_t)row * shared_stride + n);
        o0 += w[s] * v.x;
        o1 += w[s] * v.y;
    }
}

// Finish of the decode path: y[p] = the k-block parts of the down epilogue (Zd, already transformed and scaled) added
// in order; with weights, out[row] = the token's slots in order, weighted. Program (token row, 64-column block), one
// wave a slot (up to 16 at a time), one column a lane (two a lane, over half the workgroups, measured 0.1 us slower
// on config 2's layer: the parts' loads spread over fewer waves; one wave for all of a block's slots, 0.9 us slower).
// Each wave loads its slot's weight (and wave 0 the first shared slot's weight and output) together with the parts,
// so the combine adds no dependent round trip; each wave forms its weighted term and wave 0 adds the terms in slot
// order.
__global__ void __launch_bounds__(1024) sum_finish_kernel(const float* __restrict__ Z, float* __restrict__ y, int P,
                                                           int D, int SK, int slots, int exl3_slots,
                                                           const float* __restrict__ weights,
                                                           const float* __restrict__ shared, int shared_stride,
                                                           float* __restrict__ out) {
    __shared__ float ys[16][64];
    const int row = blockIdx.x, blk = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nwv = blockDim.x >> 6;
    const int n = blk * 64 + lane;
    // the first shared slot's weight and output, loaded up front (wave 0 adds them last)
    const bool sh = weights && shared && exl3_slots < slots && wave == 0;
    float sw = 0.f, sv = 0.f;
    if (sh) {
        sw = weights[row * slots + exl3_slots];
        sv = shared[(size_t)row * shared_stride + n];
    }
    float o = 0.f;
    for (int s0 = 0; s0 < exl3_slots; s0 += nwv) {
        const int s = s0 + wave;
        if (s < exl3_slots) {
            const int p = row * slots + s;
            const float w = weights ? weights[p] : 0.f;
            float zs[16];
            float v = 0.f;
            for (int k0 = 0; k0 < SK; k0 += 16) {           // parts in k order, sixteen in flight
#pragma unroll
                for (int k = 0; k < 16; ++k)
                    if (k0 + k < SK) zs[k] = Z[((size_t)(k0 + k) * P + p) * D + n];
#pragma unroll
                for (int k = 0; k < 16; ++k)
                    if (k0 + k < SK) v += zs[k];
            }
            y[(size_t)p * D + n] = v;
            ys[wave][lane] = w * v;
        }
        if (weights) {
            __syncthreads();
            if (wave == 0)
                for (int q = 0; q < nwv && s0 + q < exl3_slots; ++q) o += ys[q][lane];
            __syncthreads();
        }
    }
    if (weights && wave == 0) {
        if (sh) {
            o += sw * sv;
            for (int s = exl3_slots + 1; s < slots; ++s)
                o += weights[(size_t)row * slots + s] * shared[(size_t)row * shared_stride + n];
        }
        out[(size_t)row * D + n] = o;
    }
}

// Down epilogue (exl3.cu:300-321) and, with weights, the slot-ordered combine of a token. Program (token row,
// 128-column block), one wave a slot (up to 16 at a time): pair p = row * slots + s, its SK down partials summed in
// order, transformed, scaled by svh_d -> y[p]; then out[row] = sum over the slots in order of weights * y.
__global__ void __launch_bounds__(1024) down_finish_kernel(const float* __restrict__ Z, const int* __restrict__ pick,
                                                            const uint16_t* __restrict__ svh_d, float* __restrict__ y,
                                                            int P, int D, int SK, int slots, int exl3_slots,
                                                            const float* __restrict__ weights,
                                                            const float* __restrict__ shared, int shared_stride,
                                                            float* __restrict__ out) {
    __shared__ float2 ys[16][64];
    const int row = blockIdx.x, blk = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nwv = blockDim.x >> 6;
    const int n = blk * 128 + 2 * lane;
    // the first shared slot's weight and output, loaded up front (wave 0 adds them last)
    const bool sh = weights && shared && exl3_slots < slots && wave == 0;
    float sw = 0.f;
    float2 shv = make_float2(0.f, 0.f);
    if (sh) {
        sw = weights[row * slots + exl3_slots];
        shv = *reinterpret_cast<const float2*>(shared + (size_t)row * shared_stride + n);
    }
    float o0 = 0.f, o1 = 0.f;
    for (int s0 = 0; s0 < exl3_slots; s0 += nwv) {
        const int s = s0 + wave;
        if (s < exl3_slots) {
            const int p = row * slots + s;
            const int e = pick[p];
            const float w = weights ? weights[p] : 0.f;
            // the first partials and the expert's scales in flight together (the scale load waits only for e; the
            // loads are unconditional, a split past SK re-reads the last one, so that the wait counts stay exact)
            float2 zs[8];
#pragma unroll
            for (int k = 0; k < 8; ++k)
                zs[k] = *reinterpret_cast<const float2*>(Z + ((size_t)(k < SK ? k : SK - 1) * P + p) * D + n);
            const uint32_t sv = *reinterpret_cast<const uint32_t*>(svh_d + (size_t)e * D + n);
            float v[2] = {0.f, 0.f};
            for (int k0 = 0; k0 < SK; k0 += 8) {            // partials in split order, eight in flight
                if (k0 > 0) {
#pragma unroll
                    for (int k = 0; k < 8; ++k)
                        if (k0 + k < SK)
                            zs[k] = *reinterpret_cast<const float2*>(Z + ((size_t)(k0 + k) * P + p) * D + n);
                }
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    if (k0 + k < SK) {
                        v[0] += zs[k].x;
                        v[1] += zs[k].y;
                    }
            }
            fwht128_w64(v, lane);
            float2 yv;
            yv.x = v[0] * HAD_SCALE * f16_to_f32((uint16_t)sv);
            yv.y = v[1] * HAD_SCALE * f16_to_f32((uint16_t)(sv >> 16));
            *reinterpret_cast<float2*>(y + (size_t)p * D + n) = yv;
            ys[wave][lane] = make_float2(w * yv.x, w * yv.y);
        }
        if (weights) {
            __syncthreads();
            if (wave == 0)
                for (int q = 0; q < nwv && s0 + q < exl3_slots; ++q) {
                    o0 += ys[q][lane].x;
                    o1 += ys[q][lane].y;
                }
            __syncthreads();
        }
    }
    if (weights && wave == 0) {
        if (sh) {
            o0 += sw * shv.x;
            o1 += sw * shv.y;
            combine_shared(weights + (size_t)row * slots, slots, exl3_slots + 1, shared, shared_stride, row, n, o0,
                           o1);
        }
        *reinterpret_cast<float2*>(out + (size_t)row * D + n) = make_float2(o0, o1);
    }
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
    // the gate and up splits' partials eight each at a time in flight (a pair of columns one 8-byte load), added in
    // split order; the expert's scales are loaded once its id has landed
    float gv[2] = {0.f, 0.f}, uv[2] = {0.f, 0.f};
    for (int s0 = 0; s0 < SK; s0 += 8) {
        float2 zg[8], zu[8];
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (s0 + k < SK) {
                zg[k] = *reinterpret_cast<const float2*>(Z + ((size_t)(s0 + k) * P + p) * N + n);
                zu[k] = *reinterpret_cast<const float2*>(Z + ((size_t)(SK + s0 + k) * P + p) * N + n);
            }
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (s0 + k < SK) {
                gv[0] += zg[k].x; gv[1] += zg[k].y;
                uv[0] += zu[k].x; uv[1] += zu[k].y;
            }
    }
    const size_t so = (size_t)e * N + n;
    const uint32_t sg = *reinterpret_cast<const uint32_t*>(svh_g + so), su = *reinterpret_cast<const uint32_t*>(svh_u + so),
                   sd = *reinterpret_cast<const uint32_t*>(suh_d + so);
    fwht128_w64(gv, lane);
    fwht128_w64(uv, lane);
    float v[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const float gg = fminf(bf16r(gv[j] * HAD_SCALE * f16_to_f32((uint16_t)(sg >> (16 * j)))), limit);
        const float uu = __builtin_amdgcn_fmed3f(bf16r(uv[j] * HAD_SCALE * f16_to_f32((uint16_t)(su >> (16 * j)))),
                                                 -limit, limit);
        const float act = bf16r(bf16r(gg / (1.f + expf(-gg))) * uu);
        v[j] = act * f16_to_f32((uint16_t)(sd >> (16 * j)));
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
    // the splits' partials sixteen at a time in flight (each pair of columns one 8-byte load), added in split order
    float v[2] = {0.f, 0.f};
    for (int k0 = 0; k0 < SK; k0 += 16) {
        float2 zs[16];
#pragma unroll
        for (int k = 0; k < 16; ++k)
            if (k0 + k < SK) zs[k] = *reinterpret_cast<const float2*>(Z + ((size_t)(k0 + k) * P + p) * D + n);
#pragma unroll
        for (int k = 0; k < 16; ++k)
            if (k0 + k < SK) {
                v[0] += zs[k].x;
                v[1] += zs[k].y;
            }
    }
    const uint32_t sv = *reinterpret_cast<const uint32_t*>(svh_d + (size_t)e * D + n);
    fwht128_w64(v, lane);
    float2 o;
    o.x = v[0] * HAD_SCALE * f16_to_f32((uint16_t)sv);
    o.y = v[1] * HAD_SCALE * f16_to_f32((uint16_t)(sv >> 16));
    *reinterpret_cast<float2*>(y + (size_t)p * D + n) = o;
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
// k tiles a wave of the gate/up GEMV: 8, one 128-point block (the bs = 1 layer measured 18.94 us against 19.13 with
// 4, twice the waves, each block's rotation built by two of them)
#ifndef GFR_GU_KTW
#define GFR_GU_KTW 8
#endif
int gemv_gateup_splits(int D) { return D / 16 / GFR_GU_KTW / nw_gateup(D); }
int gemv_down_splits(int N) { return N / 128; }   // one part a 128-k block (down_gemv_kernel)

template <int K, int KTW, int NW, int MATS, int XSRC, bool ROUTE1>
static hipError_t gemv_go(int rb, dim3 grid, hipStream_t s, const GemvArgs& a, const Fp8Args* f) {
    if (ROUTE1 && f) expert_gemv_fp8_kernel<K, KTW, NW, MATS, XSRC, 1, ROUTE1><<<grid, NW * 64, 0, s>>>(a, *f);
    else if (ROUTE1 || rb == 1) expert_gemv_kernel<K, KTW, NW, MATS, XSRC, 1, ROUTE1><<<grid, NW * 64, 0, s>>>(a);
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
static hipError_t gemv_bits(int bits, int rb, dim3 grid, hipStream_t s, const GemvArgs& a,
                            const Fp8Args* f = nullptr) {
    switch (bits) {
        case 2: return gemv_go<2, KTW, NW, MATS, XSRC, ROUTE1>(rb, grid, s, a, f);
        case 3: return gemv_go<3, KTW, NW, MATS, XSRC, ROUTE1>(rb, grid, s, a, f);
        case 4: return gemv_go<4, KTW, NW, MATS, XSRC, ROUTE1>(rb, grid, s, a, f);
        case 5: return gemv_go<5, KTW, NW, MATS, XSRC, ROUTE1>(rb, grid, s, a, f);
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
                                int maxm, int slots, int E, int bits, int maxu, const RouteOne* route,
                                const uint32_t* dt_next, const Fp8Shared* fp8) {
    GemvArgs a{};
    Fp8Args f{};
    if (fp8) f = Fp8Args{fp8->gu_w, fp8->gu_s, x, fp8->gu, fp8->act, nullptr, fp8->hidden, fp8->inter};
    a.tnext = dt_next;
    a.next_words = (size_t)(N / 16) * (D / 16) * 8 * bits;
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
        return nw == 4 ? gemv_bits<GFR_GU_KTW, 4, 2, 1, true>(bits, 1, grid, s, a, fp8 ? &f : nullptr)
                       : gemv_bits<GFR_GU_KTW, 2, 2, 1, true>(bits, 1, grid, s, a, fp8 ? &f : nullptr);
    }
    if (fp8) return hipErrorInvalidValue;               // the FP8 shared expert rides on one-token launches only
    return nw == 4 ? gemv_bits<GFR_GU_KTW, 4, 2, 1>(bits, rb, grid, s, a)
                   : gemv_bits<GFR_GU_KTW, 2, 2, 1>(bits, rb, grid, s, a);
}

hipError_t launch_expert_down(hipStream_t s, const float* Zgu, int D, int SKgu, const uint16_t* svh_g,
                              const uint16_t* svh_u, const uint16_t* suh_d, float limit, uint16_t* xd,
                              const uint32_t* dt, const uint16_t* svh_d, const int* uids, const int* ucount,
                              const int* members, float* Zd, int N, int P, int rows, int maxm, int slots, int E,
                              int bits, int maxu, const RouteOne* route, const Fp8Shared* fp8) {
    GemvArgs a{};
    a.zgu = Zgu; a.SKgu = SKgu; a.svh_g = svh_g; a.svh_u = svh_u; a.suh0 = suh_d; a.limit = limit;
    a.xd = xd; a.t0 = dt; a.t1 = dt; a.x1 = svh_d; a.uids = uids; a.ucount = ucount; a.members = members; a.z = Zd;
    a.Kin = N; a.N = D; a.P = P; a.SK = gemv_down_splits(N); a.maxm = maxm; a.slots = slots; a.E = E;
    const int rb = rb_for(rows);
    a.ucap = maxu;
    // two 128-output blocks a workgroup at wide outputs (one gate/up epilogue build and one workgroup's setup for
    // twice the trellis); the sums are the same either way
    const int hbw = (D / 128) % 2 == 0 && D >= DOWN_HB2_MIN ? 2 : 1;
    // a one-token window routed inside the gate/up launch: one program a slot (TOKEN), no grouping tables
    const bool token = route != nullptr && SKgu <= 16;
    // One-token windows with at most 4 gate/up splits and one output block a workgroup (config 2's shape) run
    // one-wave workgroups (all 8 k tiles of the block in the wave, a quarter of the waves to launch): the layer
    // measured 18.43 against 18.53 (2 waves) and 18.69 us (4 waves) on one box. With more splits or two output blocks
    // (config 5: 10 splits, hidden 5120) four waves share the work: 53.4 against 55.0 (2) and 57.4 us (1) a layer.
    const bool one = token && SKgu <= 4 && hbw == 1;
    const int tz = one ? SKgu : (SKgu + 3) / 4;         // a wave's share of the gate/up splits
    if (token) {
        a.pick_out = route->picks;
        a.routed = route->routed;
    } else if (fp8) {
        return hipErrorInvalidValue;                    // the FP8 shared expert rides on one-token launches only
    }
    Fp8Args f{};
    if (fp8) f = Fp8Args{fp8->d_w, fp8->d_s, fp8->act, nullptr, nullptr, fp8->out, fp8->hidden, fp8->inter};
    const dim3 grid(token ? (unsigned)slots : chunks_x(maxu, rows < maxm ? rows : maxm, rb), D / 128 / hbw, N / 128);
#define GFR_DOWN_HB(KB, HB)                                                                                       \
    if (fp8 && one) down_gemv_fp8_kernel<KB, 1, HB, true, 1, 4><<<grid, 64, 0, s>>>(a, f);                         \
    else if (fp8 && tz <= 1) down_gemv_fp8_kernel<KB, 1, HB, true, 4, 1><<<grid, 256, 0, s>>>(a, f);               \
    else if (fp8 && tz <= 2) down_gemv_fp8_kernel<KB, 1, HB, true, 4, 2><<<grid, 256, 0, s>>>(a, f);               \
    else if (fp8) down_gemv_fp8_kernel<KB, 1, HB, true, 4, 4><<<grid, 256, 0, s>>>(a, f);                          \
    else if (one) down_gemv_kernel<KB, 1, HB, true, 1, 4><<<grid, 64, 0, s>>>(a);                                  \
    else if (token && tz <= 1) down_gemv_kernel<KB, 1, HB, true, 4, 1><<<grid, 256, 0, s>>>(a);                   \
    else if (token && tz <= 2) down_gemv_kernel<KB, 1, HB, true, 4, 2><<<grid, 256, 0, s>>>(a);                   \
    else if (token) down_gemv_kernel<KB, 1, HB, true, 4, 4><<<grid, 256, 0, s>>>(a);                              \
    else if (rb == 1) down_gemv_kernel<KB, 1, HB, false, 4><<<grid, 256, 0, s>>>(a);                               \
    else if (rb == 2) down_gemv_kernel<KB, 2, HB, false, 4><<<grid, 256, 0, s>>>(a);                               \
    else if (rb == 4) down_gemv_kernel<KB, 4, HB, false, 4><<<grid, 256, 0, s>>>(a);                               \
    else down_gemv_kernel<KB, 8, HB, false, 4><<<grid, 256, 0, s>>>(a);
#define GFR_DOWN(KB)                                                                                              \
    case KB:                                                                                                    \
        if (hbw == 2) { GFR_DOWN_HB(KB, 2) } else { GFR_DOWN_HB(KB, 1) }                                          \
        break;
    switch (bits) {
        GFR_DOWN(2) GFR_DOWN(3) GFR_DOWN(4) GFR_DOWN(5)
        default: return hipErrorInvalidValue;
    }
#undef GFR_DOWN_HB
#undef GFR_DOWN
    return hipGetLastError();
}

hipError_t launch_sum_finish(hipStream_t s, const float* Zd, float* y, int rows, int P, int D, int SK, int slots,
                             int exl3_slots, const float* weights, const float* shared, int shared_stride,
                             float* out) {
    const int nwv = exl3_slots < 16 ? (exl3_slots > 0 ? exl3_slots : 1) : 16;
    sum_finish_kernel<<<dim3(rows, D / 64), 64 * nwv, 0, s>>>(Zd, y, P, D, SK, slots, exl3_slots, weights, shared,
                                                              shared_stride, out);
    return hipGetLastError();
}

// One linear with its input rotation fused (XSRC 1, fp16 input): Z[split][n] partials of
// W_q[0] over one row, one split a 128-k block (gemv_linear_splits), added in order by the epilogue launch. Four
// waves a split, two k tiles each: (kin / 128) x (n / 128) workgroups, 768 waves at config 1. Measured on MI355X
// with the epilogue loading all splits at once: 5.57 us against 5.90 (384 waves, four tiles), 6.10 (two-wave
// workgroups, four tiles) and 6.85 (two-wave, two tiles).
#ifndef GFR_LIN_KTW
#define GFR_LIN_KTW 2
#endif
#ifndef GFR_LIN_NW
#define GFR_LIN_NW 4
#endif
int gemv_linear_splits(int kin) { return kin / 16 / (GFR_LIN_KTW * GFR_LIN_NW); }
hipError_t launch_linear_fused(hipStream_t s, const uint16_t* x, const uint16_t* suh, const uint32_t* trellis,
                               const int* uids, const int* ucount, const int* members, float* z, int kin, int n,
                               int bits) {
    GemvArgs a{};
    a.x0 = x; a.x_stride = kin; a.x_f16 = 1; a.suh0 = suh; a.suh1 = suh; a.t0 = trellis; a.t1 = trellis;
    a.uids = uids; a.ucount = ucount; a.members = members; a.z = z; a.Kin = kin; a.N = n; a.P = 1;
    a.SK = gemv_linear_splits(kin); a.maxm = 1; a.slots = 1; a.E = 1; a.ucap = 1;
    const dim3 grid(1, n / 128, a.SK);
    switch (bits) {
#define GFR_LIN(KB)                                                                                                 \
        case KB:                                                                                                  \
            expert_gemv_kernel<KB, GFR_LIN_KTW, GFR_LIN_NW, 1, 1, 1, false><<<grid, 64 * GFR_LIN_NW, 0, s>>>(a);   \
            break;
        GFR_LIN(2) GFR_LIN(3) GFR_LIN(4) GFR_LIN(5)
#undef GFR_LIN
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_down_finish(hipStream_t s, const float* Zd, const int* pick, const uint16_t* svh_d, float* y,
                              int rows, int P, int D, int SK, int slots, int exl3_slots, const float* weights,
                              const float* shared, int shared_stride, float* out) {
    const int nwv = exl3_slots < 16 ? (exl3_slots > 0 ? exl3_slots : 1) : 16;
    down_finish_kernel<<<dim3(rows, D / 128), 64 * nwv, 0, s>>>(Zd, pick, svh_d, y, P, D, SK, slots, exl3_slots,
                                                                weights, shared, shared_stride, out);
    return hipGetLastError();
}

hipError_t launch_gateup_epilogue(hipStream_t s, const float* Z, const int* pick, const uint16_t* svh_g,
                                  const uint16_t* svh_u, const uint16_t* suh_d, uint16_t* xd, int P, int N, int SK,
                                  int slots, int exl3_slots, float limit, bool pair_order) {
    gateup_epilogue_kernel<<<dim3(P, N / 128), 64, 0, s>>>(Z, pick, svh_g, svh_u, suh_d, xd, P, N, SK, slots,
                                                           exl3_slots, limit, pair_order ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_down_epilogue(hipStream_t s, const float* Z, const int* pick, const uint16_t* svh_d, float* y,
                                int P, int D, int SK, int slots, int exl3_slots) {
    down_epilogue_kernel<<<dim3(P, D / 128), 64, 0, s>>>(Z, pick, svh_d, y, P, D, SK, slots, exl3_slots);
    return hipGetLastError();
}

}  // namespace gfr
